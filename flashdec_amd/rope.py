"""Decode-time RoPE and paged KV append (public API of cysong2025/flashdec rope.py).

* :func:`apply_rope` -- split-half (NeoX) RoPE with fp32 math, torch ops in
  the reference's order (flashdec/rope.py:26-85).  It is the ``"torch"``
  append backend's rotation; the HIP fused kernel instead evaluates the two
  transcendental steps in float64 and rounds once (see
  ``fd_fused_rope_kv_append``), so the two backends may differ by one fp32 ulp
  in cos/sin, exactly as the reference's own torch and CUDA backends differ.
* :func:`rope_paged_kv_append` / :func:`rope_paged_kv_append_ref` and
  :class:`RopeAppendResult` (rope.py:16-23, 88-236): positions from the cache,
  rotate, append through the selected backend, return what decode needs.

Backends: ``"torch"`` (reference semantics), ``"cuda"`` / ``"hip"`` (torch
RoPE + the HIP K/V scatter), ``"fused_cuda"`` / ``"fused_hip"`` (one HIP
kernel).  The ``*_cuda`` names are kept so reference callers drop in.
"""

from __future__ import annotations

import math
from dataclasses import dataclass
from typing import Any

_APPEND_BACKENDS = {
    "torch": "torch",
    "cuda": "hip",
    "hip": "hip",
    "fused_cuda": "fused_hip",
    "fused_hip": "fused_hip",
}


def _torch():
    import torch

    return torch


@dataclass(frozen=True)
class RopeAppendResult:
    """Outputs required by the next paged decode attention call."""

    q: Any
    positions: Any
    block_tables: Any
    seq_lens: Any


def apply_rope(x, positions, rotary_dim=None, base=10_000.0):
    """Split-half rotary embedding of ``x [batch, heads, head_dim]`` with fp32 math.

    Dimensions past ``rotary_dim`` are copied unchanged; output keeps x.dtype.
    """
    torch = _torch()
    if not isinstance(x, torch.Tensor) or not isinstance(positions, torch.Tensor):
        raise TypeError("x and positions must be torch tensors")
    if x.dim() != 3:
        raise ValueError("x must have shape [batch, num_heads, head_dim]")
    if positions.dim() != 1 or positions.numel() != x.shape[0]:
        raise ValueError("positions must have shape [batch]")
    if x.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("apply_rope supports float16, bfloat16, and float32")
    if positions.dtype not in (torch.int32, torch.int64):
        raise ValueError("positions must use int32 or int64")
    if positions.device != x.device:
        raise ValueError("x and positions must be on the same device")
    if bool(torch.any(positions < 0).item()):
        raise ValueError("positions must be non-negative")
    head_dim = x.shape[-1]
    if rotary_dim is None:
        rotary_dim = head_dim
    if isinstance(rotary_dim, bool) or not isinstance(rotary_dim, int):
        raise ValueError("rotary_dim must be an even integer")
    if rotary_dim <= 0 or rotary_dim > head_dim or rotary_dim % 2 != 0:
        raise ValueError("rotary_dim must be positive, even, and no larger than head_dim")
    base = float(base)
    if not math.isfinite(base) or base <= 0.0:
        raise ValueError("base must be a positive finite number")

    steps = torch.arange(0, rotary_dim, 2, device=x.device, dtype=torch.float32)
    inv_freq = torch.pow(base, -steps / rotary_dim)
    angles = positions.to(torch.float32)[:, None] * inv_freq[None, :]
    cos = torch.cos(angles)[:, None, :]
    sin = torch.sin(angles)[:, None, :]
    half = rotary_dim // 2
    x_rot = x[..., :rotary_dim].to(torch.float32)
    lo, hi = x_rot[..., :half], x_rot[..., half:]
    rotated = torch.cat((lo * cos - hi * sin, hi * cos + lo * sin), dim=-1).to(x.dtype)
    if rotary_dim == head_dim:
        return rotated
    return torch.cat((rotated, x[..., rotary_dim:]), dim=-1)


def rope_cos_sin_table(num_positions, rotary_dim, base=10_000.0, device="cuda"):
    """fp32 ``[2, num_positions, rotary_dim // 2]``: cos (plane 0) and sin (plane 1) of positions
    ``0 .. num_positions - 1``.

    Evaluated with :func:`apply_rope`'s own torch expression (flashdec/rope.py:
    66-70) on ``device``, so the HIP kernels that read it
    (``fused_rope_kv_append(..., cos_sin_table=...)`` and the engine's fused
    decode launch) rotate exactly as :func:`apply_rope` does there, bit for
    bit.  No counterpart in the reference.
    """
    torch = _torch()
    num_positions = int(num_positions)
    if num_positions <= 0:
        raise ValueError("num_positions must be positive")
    if isinstance(rotary_dim, bool) or not isinstance(rotary_dim, int) or rotary_dim <= 0 or rotary_dim % 2:
        raise ValueError("rotary_dim must be a positive even integer")
    base = float(base)
    if not math.isfinite(base) or base <= 0.0:
        raise ValueError("base must be a positive finite number")
    steps = torch.arange(0, rotary_dim, 2, device=device, dtype=torch.float32)
    inv_freq = torch.pow(base, -steps / rotary_dim)
    positions = torch.arange(num_positions, device=device, dtype=torch.int64)
    angles = positions.to(torch.float32)[:, None] * inv_freq[None, :]
    return torch.stack((torch.cos(angles), torch.sin(angles))).contiguous()


def _prepare_inputs(cache, request_ids, q, k, v):
    """Validate one RoPE + paged append batch (rope.py:88-124, same messages)."""
    from .cache import PagedKVCache

    if not isinstance(cache, PagedKVCache):
        raise TypeError("cache must be a PagedKVCache")
    ids = cache._normalize_request_ids(request_ids)
    if not ids:
        raise ValueError("request_ids must be non-empty")
    if len(set(ids)) != len(ids):
        raise ValueError("request_ids must be unique")
    if q.dim() != 3:
        raise ValueError("q must have shape [num_requests, num_q_heads, head_dim]")
    if k.dim() == 2 and len(ids) == 1:
        k = k.unsqueeze(0)
    if v.dim() == 2 and len(ids) == 1:
        v = v.unsqueeze(0)
    if k.dim() != 3 or v.dim() != 3:
        raise ValueError("k and v must have shape [num_requests, num_kv_heads, head_dim]")
    if q.shape[0] != len(ids) or q.shape[1] <= 0 or q.shape[2] != cache.head_dim:
        raise ValueError("q shape must match request count and cache head_dim")
    expected = (len(ids), cache.num_kv_heads, cache.head_dim)
    if k.shape != expected or v.shape != expected:
        raise ValueError("k and v shapes must match request count and cache dimensions")
    if q.device != cache.device or k.device != cache.device or v.device != cache.device:
        raise ValueError("q, k, and v must be on the cache device")
    if q.dtype != cache.dtype or k.dtype != cache.dtype or v.dtype != cache.dtype:
        raise ValueError("q, k, and v must use the cache dtype")
    return ids, k, v


def _rope_paged_kv_append(cache, layer_idx, request_ids, q, k, v, rotary_dim, base, append_backend):
    if append_backend not in _APPEND_BACKENDS:
        raise ValueError("append_backend must be 'torch', 'cuda', or 'fused_cuda'")
    backend = _APPEND_BACKENDS[append_backend]
    ids, k, v = _prepare_inputs(cache, request_ids, q, k, v)
    positions = cache.next_positions(ids, device=cache.device)
    if backend == "fused_hip":
        q_rot, block_tables = cache.append_fused_cuda(layer_idx, ids, q, k, v, positions, rotary_dim=rotary_dim,
                                                      base=base)
    else:
        q_rot = apply_rope(q, positions, rotary_dim=rotary_dim, base=base)
        k_rot = apply_rope(k, positions, rotary_dim=rotary_dim, base=base)
        if backend == "torch":
            block_tables = cache.append(layer_idx, ids, k_rot, v)
        else:
            block_tables = cache.append_cuda(layer_idx, ids, k_rot, v)
    return RopeAppendResult(q=q_rot, positions=positions, block_tables=block_tables,
                            seq_lens=cache.seq_lens_tensor(ids))


def rope_paged_kv_append_ref(cache, layer_idx, request_ids, q, k, v, rotary_dim=None, base=10_000.0):
    """Rotate Q/K, then append rotated K / raw V through the torch path."""
    return _rope_paged_kv_append(cache, layer_idx, request_ids, q, k, v, rotary_dim, base, "torch")


def rope_paged_kv_append(cache, layer_idx, request_ids, q, k, v, rotary_dim=None, base=10_000.0,
                         append_backend="torch"):
    """Rotate Q/K and append K/V through ``append_backend`` (see module doc)."""
    return _rope_paged_kv_append(cache, layer_idx, request_ids, q, k, v, rotary_dim, base, append_backend)
