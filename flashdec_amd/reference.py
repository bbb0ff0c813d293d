"""PyTorch dense decode attention (the reference's semantic baseline API).

``dense_decode_attention_ref`` mirrors cysong2025/flashdec
flashdec/reference.py:35-101 (dense ``[B, L, Hkv, D]`` caches, fp32 math,
zero rows for empty sequences).  Explicit-use only, like
:mod:`flashdec_amd.paged_reference`.
"""

from __future__ import annotations


def dense_decode_attention_ref(q, k_cache, v_cache, seq_lens, sm_scale=None):
    """q ``[B, Hq, D]``; k/v ``[B, max_seq_len, Hkv, D]``; seq_lens ``[B]``."""
    import torch

    if q.dim() != 3:
        raise ValueError("q must have shape [num_seqs, num_q_heads, head_dim]")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("k_cache and v_cache must be 4D tensors")
    if seq_lens.dim() != 1:
        raise ValueError("seq_lens must be a 1D tensor")
    if q.device != k_cache.device or q.device != v_cache.device:
        raise ValueError("q, k_cache, and v_cache must be on the same device")
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        raise ValueError("q, k_cache, and v_cache must have the same dtype")
    if not q.is_floating_point():
        raise ValueError("q, k_cache, and v_cache must be floating point tensors")
    num_seqs, num_q_heads, head_dim = q.shape
    k_num_seqs, max_seq_len, num_kv_heads, k_head_dim = k_cache.shape
    v_num_seqs, v_max_seq_len, v_num_kv_heads, v_head_dim = v_cache.shape
    if k_num_seqs != num_seqs or v_num_seqs != num_seqs:
        raise ValueError("q, k_cache, and v_cache must have the same num_seqs")
    if v_max_seq_len != max_seq_len:
        raise ValueError("k_cache and v_cache must have the same max_seq_len")
    if v_num_kv_heads != num_kv_heads:
        raise ValueError("k_cache and v_cache must have the same num_kv_heads")
    if k_head_dim != head_dim or v_head_dim != head_dim:
        raise ValueError("q, k_cache, and v_cache must have the same head_dim")
    if seq_lens.numel() != num_seqs:
        raise ValueError("seq_lens length must match num_seqs")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("num_q_heads must be divisible by num_kv_heads")
    lens = [int(x) for x in seq_lens.detach().cpu().tolist()]
    if any(n < 0 or n > max_seq_len for n in lens):
        raise ValueError("seq_lens values must be in [0, max_seq_len]")
    if sm_scale is None:
        sm_scale = head_dim**-0.5
    group = num_q_heads // num_kv_heads
    out = torch.zeros_like(q)
    for b, n in enumerate(lens):
        if n == 0:
            continue
        k = k_cache[b, :n].float().permute(1, 0, 2)  # [Hkv, n, D]
        v = v_cache[b, :n].float().permute(1, 0, 2)
        qf = q[b].float().view(num_kv_heads, group, head_dim)
        probs = torch.softmax(torch.matmul(qf, k.transpose(1, 2).contiguous()) * sm_scale, dim=-1)
        out[b] = torch.matmul(probs, v).reshape(num_q_heads, head_dim).to(out.dtype)
    return out
