"""PyTorch paged decode attention (the reference's semantic baseline API).

``paged_decode_attention_ref`` is part of cysong2025/flashdec's public API
(flashdec/paged_reference.py:19-125) and backs ``DecodeEngine`` when a caller
explicitly selects ``decode_backend="reference"`` (e.g. CPU-resident caches
in allocator tests).  It is never used as a fallback for the HIP path: the HIP
entry points raise if ``libflashdec_hip.so`` is missing.

Same contract as the reference: fp32 math per sequence, grouped heads map to
KV head ``h // (Hq / Hkv)``, zero rows for ``seq_len == 0``, ``ValueError``
for invalid block ids inside the used range.  The computation is vectorised
per sequence (all query heads of a KV head at once) instead of the
reference's per-head loop; results agree to fp32 rounding.
"""

from __future__ import annotations

_KV_LAYOUT_AXES = {"token_major": (2, 3), "dim_major": (3, 2)}


def _layout_axes(kv_layout):
    try:
        return _KV_LAYOUT_AXES[kv_layout]
    except KeyError as exc:
        raise ValueError("kv_layout must be 'token_major' or 'dim_major'") from exc


def paged_decode_attention_ref(q, k_cache, v_cache, block_tables, seq_lens, sm_scale=None, kv_layout="token_major"):
    """Single-token decode attention over a paged cache (fp32 math).

    q ``[num_seqs, num_q_heads, head_dim]``; token-major caches
    ``[num_blocks, num_kv_heads, block_size, head_dim]`` (dim-major:
    ``[..., head_dim, block_size]``); block_tables ``[num_seqs, max_blocks]``;
    seq_lens ``[num_seqs]``.  Returns q's shape and dtype.
    """
    import torch

    token_axis, dim_axis = _layout_axes(kv_layout)
    if q.dim() != 3:
        raise ValueError("q must have shape [num_seqs, num_q_heads, head_dim]")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("k_cache and v_cache must be 4D tensors")
    if block_tables.dim() != 2:
        raise ValueError("block_tables must have shape [num_seqs, max_blocks_per_seq]")
    if seq_lens.dim() != 1:
        raise ValueError("seq_lens must be a 1D tensor")
    if q.device != k_cache.device or q.device != v_cache.device:
        raise ValueError("q, k_cache, and v_cache must be on the same device")
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        raise ValueError("q, k_cache, and v_cache must have the same dtype")
    if not q.is_floating_point():
        raise ValueError("q, k_cache, and v_cache must be floating point tensors")
    if block_tables.dtype not in (torch.int16, torch.int32, torch.int64):
        raise ValueError("block_tables must contain integer physical block ids")

    num_seqs, num_q_heads, head_dim = q.shape
    num_blocks, num_kv_heads = k_cache.shape[:2]
    block_size = k_cache.shape[token_axis]
    if v_cache.shape[0] != num_blocks:
        raise ValueError("k_cache and v_cache must have the same num_blocks")
    if v_cache.shape[1] != num_kv_heads:
        raise ValueError("k_cache and v_cache must have the same num_kv_heads")
    if v_cache.shape[token_axis] != block_size:
        raise ValueError("k_cache and v_cache must have the same block_size")
    if k_cache.shape[dim_axis] != head_dim or v_cache.shape[dim_axis] != head_dim:
        raise ValueError("q, k_cache, and v_cache must have the same head_dim")
    if block_tables.shape[0] != num_seqs or seq_lens.numel() != num_seqs:
        raise ValueError("block_tables and seq_lens must have one row/value per sequence")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("num_q_heads must be divisible by num_kv_heads")
    lens = [int(x) for x in seq_lens.detach().cpu().tolist()]
    max_seq_len = block_tables.shape[1] * block_size
    if any(n < 0 or n > max_seq_len for n in lens):
        raise ValueError("seq_lens values must be in [0, max_blocks_per_seq * block_size]")
    if sm_scale is None:
        sm_scale = head_dim**-0.5
    group = num_q_heads // num_kv_heads

    # token-major view [num_blocks, num_kv_heads, block_size, head_dim]
    k_tm = k_cache if kv_layout == "token_major" else k_cache.transpose(2, 3)
    v_tm = v_cache if kv_layout == "token_major" else v_cache.transpose(2, 3)
    out = torch.zeros_like(q)
    for b, n in enumerate(lens):
        if n == 0:
            continue
        nblk = (n + block_size - 1) // block_size
        ids = [int(x) for x in block_tables[b, :nblk].detach().cpu().tolist()]
        if any(i < 0 or i >= num_blocks for i in ids):
            raise ValueError("block_tables contains invalid physical block ids for a non-empty sequence")
        index = torch.tensor(ids, device=k_cache.device, dtype=torch.long)
        # [nblk, Hkv, bs, D] -> [Hkv, nblk*bs, D] -> first n tokens
        k = k_tm.index_select(0, index).permute(1, 0, 2, 3).reshape(num_kv_heads, -1, head_dim)[:, :n].float()
        v = v_tm.index_select(0, index).permute(1, 0, 2, 3).reshape(num_kv_heads, -1, head_dim)[:, :n].float()
        qf = q[b].float().view(num_kv_heads, group, head_dim)
        scores = torch.matmul(qf, k.transpose(1, 2).contiguous()) * sm_scale  # [Hkv, G, n]
        probs = torch.softmax(scores, dim=-1)
        out[b] = torch.matmul(probs, v).reshape(num_q_heads, head_dim).to(out.dtype)
    return out
