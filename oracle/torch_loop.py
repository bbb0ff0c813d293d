"""fp32 torch-CPU paged decode in the reference's loop form.  Test infrastructure only.

``paged_decode_attention_loop`` restates cysong2025/flashdec
``flashdec/paged_reference.py:92-125`` in torch on the CPU: for every sequence
gather its first ``ceil(seq_len / block_size)`` physical blocks
(token-major ``[NB, Hkv, bs, D]``, ``index_select`` then
``permute(0, 2, 1, 3)``, paged_reference.py:101-106), keep ``seq_len``
tokens, then for every query head -- the per-(sequence, query-head) loop of
paged_reference.py:115-123 -- ``scores = (K @ q) * scale``, subtract the max,
``exp``, divide by the sum, ``probs @ V`` in fp32, rounded to q's dtype.
``seq_len == 0`` gives a zero row.  Inputs are validated by the caller.

Used only as bench.py's CPU baseline (timed under
``torch.set_num_threads``); pinned against the numpy oracle
(:func:`oracle.attention.paged_decode_attention`) in tests/test_oracle.py.
"""

from __future__ import annotations


def paged_decode_attention_loop(q, k_cache, v_cache, block_tables, seq_lens, sm_scale):
    """q ``[B, Hq, D]``, token-major caches, int tables ``[B, W]``, ``seq_lens`` ``[B]`` (CPU tensors)."""
    import torch

    num_seqs, num_q_heads, head_dim = q.shape
    num_kv_heads, block_size = k_cache.shape[1], k_cache.shape[2]
    group = num_q_heads // num_kv_heads
    out = torch.empty_like(q)
    for seq_idx, seq_len in enumerate(int(n) for n in seq_lens.tolist()):
        if seq_len == 0:
            out[seq_idx].zero_()
            continue
        nblk = (seq_len + block_size - 1) // block_size
        ids = block_tables[seq_idx, :nblk].to(torch.long)
        k_seq = k_cache.index_select(0, ids).permute(0, 2, 1, 3).reshape(-1, num_kv_heads, head_dim)[:seq_len]
        v_seq = v_cache.index_select(0, ids).permute(0, 2, 1, 3).reshape(-1, num_kv_heads, head_dim)[:seq_len]
        for q_head in range(num_q_heads):
            kv_head = q_head // group
            q_vec = q[seq_idx, q_head].to(torch.float32)
            k = k_seq[:, kv_head].to(torch.float32)
            v = v_seq[:, kv_head].to(torch.float32)
            scores = torch.matmul(k, q_vec) * sm_scale
            scores = scores - torch.max(scores)
            probs = torch.exp(scores)
            probs = probs / torch.sum(probs)
            out[seq_idx, q_head] = torch.matmul(probs, v).to(out.dtype)
    return out
