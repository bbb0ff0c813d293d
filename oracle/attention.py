"""Paged decode attention oracle (numpy).  Test infrastructure only.

``paged_decode_attention`` restates cysong2025/flashdec
``flashdec/paged_reference.py:19-125``: for every sequence, gather its
physical blocks (token-major ``[NB, Hkv, bs, D]`` or dim-major
``[NB, Hkv, D, bs]``), keep the first ``seq_len`` tokens, and for every query
head compute ``softmax((K . q) * scale) . V`` in fp32 with the reference's op
order (scores, subtract max, exp, divide by sum, weighted sum), then round to
the output dtype.  ``seq_len == 0`` gives a zero row; GQA maps query head
``h`` to KV head ``h // (Hq / Hkv)``; invalid block ids inside the used range
raise ``ValueError`` (paged_reference.py:97-99).

``dense_attention_f64`` is the float64 brute force used to pin it.
"""

from __future__ import annotations

import numpy as np

from .rope import round_to

_LAYOUTS = ("token_major", "dim_major")


def paged_decode_attention(
    q,
    k_cache,
    v_cache,
    block_tables,
    seq_lens,
    sm_scale=None,
    kv_layout="token_major",
    out_dtype="float32",
):
    """fp32 oracle; inputs are numpy arrays (fp32 holding the element values).

    ``out_dtype`` in {"float32", "bfloat16", "float16"} selects the final
    rounding (the reference casts to q.dtype, paged_reference.py:123).
    """
    if kv_layout not in _LAYOUTS:
        raise ValueError("kv_layout must be 'token_major' or 'dim_major'")
    q = np.asarray(q, dtype=np.float32)
    k_cache = np.asarray(k_cache, dtype=np.float32)
    v_cache = np.asarray(v_cache, dtype=np.float32)
    block_tables = np.asarray(block_tables)
    seq_lens = np.asarray(seq_lens)
    num_seqs, num_q_heads, head_dim = q.shape
    num_blocks, num_kv_heads = k_cache.shape[:2]
    if kv_layout == "token_major":
        block_size = k_cache.shape[2]
    else:
        block_size = k_cache.shape[3]
    if num_q_heads % num_kv_heads:
        raise ValueError("num_q_heads must be divisible by num_kv_heads")
    group = num_q_heads // num_kv_heads
    if sm_scale is None:
        sm_scale = head_dim ** -0.5
    scale = np.float32(sm_scale)
    out = np.zeros((num_seqs, num_q_heads, head_dim), dtype=np.float32)
    for b in range(num_seqs):
        seq_len = int(seq_lens[b])
        if seq_len == 0:
            continue
        nblk = (seq_len + block_size - 1) // block_size
        ids = [int(x) for x in block_tables[b, :nblk]]
        if any(i < 0 or i >= num_blocks for i in ids):
            raise ValueError("block_tables contains invalid physical block ids for a non-empty sequence")
        kb = k_cache[ids]
        vb = v_cache[ids]
        if kv_layout == "token_major":  # [n, Hkv, bs, D] -> [n*bs, Hkv, D]
            k_seq = kb.transpose(0, 2, 1, 3).reshape(-1, num_kv_heads, head_dim)[:seq_len]
            v_seq = vb.transpose(0, 2, 1, 3).reshape(-1, num_kv_heads, head_dim)[:seq_len]
        else:  # [n, Hkv, D, bs] -> [n*bs, Hkv, D]
            k_seq = kb.transpose(0, 3, 1, 2).reshape(-1, num_kv_heads, head_dim)[:seq_len]
            v_seq = vb.transpose(0, 3, 1, 2).reshape(-1, num_kv_heads, head_dim)[:seq_len]
        for h in range(num_q_heads):
            kvh = h // group
            k = k_seq[:, kvh]
            v = v_seq[:, kvh]
            scores = (k @ q[b, h]) * scale
            scores = scores - scores.max()
            probs = np.exp(scores)
            probs = probs / probs.sum()
            out[b, h] = probs @ v
    return round_to(out, out_dtype)


def dense_attention_f64(q, k, v, seq_lens, sm_scale=None):
    """Float64 brute force over dense ``[B, L, Hkv, D]`` K/V (textbook softmax)."""
    q = np.asarray(q, dtype=np.float64)
    k = np.asarray(k, dtype=np.float64)
    v = np.asarray(v, dtype=np.float64)
    num_seqs, num_q_heads, head_dim = q.shape
    num_kv_heads = k.shape[2]
    group = num_q_heads // num_kv_heads
    if sm_scale is None:
        sm_scale = head_dim ** -0.5
    out = np.zeros((num_seqs, num_q_heads, head_dim), dtype=np.float64)
    for b in range(num_seqs):
        n = int(seq_lens[b])
        if n == 0:
            continue
        for h in range(num_q_heads):
            s = np.array([sum(q[b, h, d] * k[b, t, h // group, d] for d in range(head_dim)) for t in range(n)])
            s = s * sm_scale
            w = np.exp(s - s.max())
            w = w / w.sum()
            out[b, h] = (w[:, None] * v[b, :n, h // group]).sum(axis=0)
    return out


def paged_to_dense(k_cache, v_cache, block_tables, seq_lens, kv_layout="token_major"):
    """Materialise a paged cache as dense ``[B, Lmax, Hkv, D]`` (zero padded).

    Restates the data movement of ``PagedKVCache.to_dense``
    (flashdec/cache.py:986-1021) for a single layer.
    """
    k_cache = np.asarray(k_cache, dtype=np.float32)
    v_cache = np.asarray(v_cache, dtype=np.float32)
    if kv_layout == "dim_major":
        k_cache = k_cache.transpose(0, 1, 3, 2)
        v_cache = v_cache.transpose(0, 1, 3, 2)
    _, hkv, bs, d = k_cache.shape
    lmax = max(1, max(int(x) for x in seq_lens))
    kd = np.zeros((len(seq_lens), lmax, hkv, d), dtype=np.float32)
    vd = np.zeros_like(kd)
    for b, n in enumerate(seq_lens):
        n = int(n)
        for t in range(n):
            blk = int(block_tables[b][t // bs])
            kd[b, t] = k_cache[blk, :, t % bs]
            vd[b, t] = v_cache[blk, :, t % bs]
    return kd, vd


def algorithmic_bytes(seq_lens, num_q_heads, num_kv_heads, head_dim, block_size, elt_bytes=2, max_blocks=None,
                      unique_blocks=None):
    """Bytes a decode call must move, each distinct element counted once.

    sum_b L_b * Hkv * D * 2 * elt (K and V; with ``unique_blocks`` the KV term
    is unique physical blocks * bs instead) + 2 * B * Hq * D * elt (q, out) +
    4 * B * max_blocks (int32 table) + 4 * B (seq_lens).
    """
    seq_lens = [int(x) for x in seq_lens]
    b = len(seq_lens)
    if max_blocks is None:
        max_blocks = max((x + block_size - 1) // block_size for x in seq_lens)
    if unique_blocks is None:
        kv_tokens = sum(seq_lens)
    else:
        kv_tokens = unique_blocks * block_size
    return (
        kv_tokens * num_kv_heads * head_dim * 2 * elt_bytes
        + 2 * b * num_q_heads * head_dim * elt_bytes
        + 4 * b * max_blocks
        + 4 * b
    )
