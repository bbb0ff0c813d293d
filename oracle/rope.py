"""RoPE and paged KV-append oracle (numpy).  Test infrastructure only.

Restates cysong2025/flashdec ``flashdec/rope.py:26-85`` (``apply_rope``) and
the data movement of ``flashdec/csrc/fused_rope_kv_append_kernel.cu:38-82``
(rotated Q into ``q_out``; rotated K and raw V into the token-major slot
``((blk * Hkv + h) * bs + off) * D + d``).

The reference evaluates, in fp32:
    e       = -arange(0, R, 2) / R                (rope.py:66-67)
    inv     = pow(fp32(base), e)
    angle   = fp32(pos) * inv                     (rope.py:68)
    cos/sin = cos(angle), sin(angle)              (rope.py:69-70)
    lo      = x_lo * cos - x_hi * sin             (rope.py:76-81)
    hi      = x_hi * cos + x_lo * sin
rounded to the tensor dtype, with dims past R copied.  Here ``e``, ``angle``
and the rotation products/sums are IEEE fp32 operations exactly as written;
``pow`` and ``cos``/``sin`` are evaluated in float64 and rounded once to fp32,
i.e. the correctly rounded fp32 values (torch's fp32 kernels are within one
ulp of them).  The HIP kernel computes the same numbers, so its output bytes
must equal these bit for bit.
"""

from __future__ import annotations

import math

import numpy as np


def round_to(x, dtype):
    """Round fp32 values to ``dtype`` ("float32" | "bfloat16" | "float16"), RNE.

    bfloat16 results are returned as fp32 arrays holding bf16 values.
    """
    x = np.asarray(x, dtype=np.float32)
    if dtype in ("float32", np.float32):
        return x.copy()
    if dtype in ("float16", np.float16):
        return x.astype(np.float16).astype(np.float32)
    if dtype in ("bfloat16",):
        u = x.view(np.uint32).astype(np.uint64)
        bias = ((u >> 16) & 1) + 0x7FFF
        r = ((u + bias) & 0xFFFF0000).astype(np.uint32)
        nan = np.isnan(x)
        r = np.where(nan, np.uint32(0x7FC00000), r).astype(np.uint32)
        return r.view(np.float32)
    raise ValueError(f"unknown dtype {dtype}")


def bf16_bits(x):
    """uint16 bit patterns of bf16 values stored in fp32 arrays."""
    return (np.asarray(x, dtype=np.float32).view(np.uint32) >> 16).astype(np.uint16)


def rope_cos_sin(positions, rotary_dim, base=10_000.0):
    """fp32 ``(cos, sin)`` of shape ``[B, R/2]`` (rope.py:66-70, see module doc)."""
    if rotary_dim <= 0 or rotary_dim % 2:
        raise ValueError("rotary_dim must be positive and even")
    steps = np.arange(0, rotary_dim, 2, dtype=np.float32)
    e = (-steps) / np.float32(rotary_dim)
    base32 = float(np.float32(base))
    inv = np.array([np.float32(math.pow(base32, float(x))) for x in e], dtype=np.float32)
    pos = np.asarray(positions).astype(np.float32)
    ang = pos[:, None] * inv[None, :]
    cos = np.vectorize(lambda a: np.float32(math.cos(float(a))), otypes=[np.float32])(ang)
    sin = np.vectorize(lambda a: np.float32(math.sin(float(a))), otypes=[np.float32])(ang)
    return cos.astype(np.float32).reshape(ang.shape), sin.astype(np.float32).reshape(ang.shape)


def apply_rope(x, positions, rotary_dim=None, base=10_000.0, out_dtype="float32"):
    """Split-half RoPE of ``x [B, H, D]`` (rope.py:26-85); returns ``out_dtype`` values."""
    x = np.asarray(x, dtype=np.float32)
    head_dim = x.shape[-1]
    if rotary_dim is None:
        rotary_dim = head_dim
    if rotary_dim <= 0 or rotary_dim > head_dim or rotary_dim % 2:
        raise ValueError("rotary_dim must be positive, even, and no larger than head_dim")
    if np.any(np.asarray(positions) < 0):
        raise ValueError("positions must be non-negative")
    half = rotary_dim // 2
    cos, sin = rope_cos_sin(positions, rotary_dim, base)
    cos = cos[:, None, :]
    sin = sin[:, None, :]
    x1 = x[..., :half]
    x2 = x[..., half:rotary_dim]
    lo = (x1 * cos) - (x2 * sin)
    hi = (x2 * cos) + (x1 * sin)
    out = x.copy()
    out[..., :half] = lo
    out[..., half:rotary_dim] = hi
    return round_to(out, out_dtype)


def rope_kv_append(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim=None,
                   base=10_000.0, dtype="bfloat16"):
    """Expected ``(q_out, k_cache', v_cache')`` of one fused RoPE + append call.

    Caches are token-major ``[NB, Hkv, bs, D]`` numpy arrays (copied, not
    mutated).  Rows are written in batch order, so a later row wins a slot
    collision, matching a per-row scatter.
    """
    q_out = apply_rope(q, positions, rotary_dim, base, dtype)
    k_rot = apply_rope(k, positions, rotary_dim, base, dtype)
    kc = np.array(k_cache, dtype=np.float32, copy=True)
    vc = np.array(v_cache, dtype=np.float32, copy=True)
    v = np.asarray(v, dtype=np.float32)
    for b in range(q_out.shape[0]):
        blk = int(block_ids[b])
        off = int(block_offsets[b])
        kc[blk, :, off, :] = k_rot[b]
        vc[blk, :, off, :] = v[b]
    return q_out, kc, vc


def kv_append(k, v, k_cache, v_cache, block_ids, block_offsets):
    """Expected caches after the plain K/V scatter (kv_append_kernel.cu:10-42)."""
    kc = np.array(k_cache, dtype=np.float32, copy=True)
    vc = np.array(v_cache, dtype=np.float32, copy=True)
    for b in range(len(block_ids)):
        kc[int(block_ids[b]), :, int(block_offsets[b]), :] = k[b]
        vc[int(block_ids[b]), :, int(block_offsets[b]), :] = v[b]
    return kc, vc
