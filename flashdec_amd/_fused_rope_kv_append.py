"""Fused RoPE + paged K/V append on MI355X (``fd_fused_rope_kv_append``).

Mirrors cysong2025/flashdec ``flashdec/_fused_rope_kv_append.py``:

* :func:`fused_rope_kv_append` (:210-258) -- checked public primitive; it
  validates structure, then index *values* with device reductions that sync
  (:128-145), then launches.
* :func:`_fused_rope_kv_append_trusted` (:261-309) -- for cache-owned
  transaction metadata: same structural checks, no value reductions, int64
  indices required.
* :func:`load_fused_rope_kv_append_extension` (:34-52) -- here: load
  ``libflashdec_hip.so`` (built ahead of time in-tree, never JIT).

The kernel range-checks block ids/offsets itself, so even the trusted path
cannot write outside the cache.
"""

from __future__ import annotations

import math

import torch

from . import _lib


def load_fused_rope_kv_append_extension():
    """Return the loaded C-ABI library (raises RuntimeError if it is not built)."""
    return _lib.load_library()


def _check_cuda_contiguous_tensor(name, tensor):
    if not tensor.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _validate_structure(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base):
    """Structural contract of _fused_rope_kv_append.py:62-125 (same messages)."""
    for name, tensor in [
        ("q", q),
        ("k", k),
        ("v", v),
        ("k_cache", k_cache),
        ("v_cache", v_cache),
        ("block_ids", block_ids),
        ("block_offsets", block_offsets),
        ("positions", positions),
    ]:
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        _check_cuda_contiguous_tensor(name, tensor)

    if q.dim() != 3 or k.dim() != 3 or v.dim() != 3:
        raise ValueError("q, k, and v must have shape [batch, heads, head_dim]")
    if q.shape[1] <= 0 or k.shape[1] <= 0:
        raise ValueError("q and k must have at least one head")
    if v.shape != k.shape:
        raise ValueError("v must match k shape")
    if k_cache.dim() != 4 or v_cache.shape != k_cache.shape:
        raise ValueError("K/V caches must match shape [blocks, kv_heads, block_size, head_dim]")
    if q.shape[0] != k.shape[0] or q.shape[2] != k.shape[2]:
        raise ValueError("q batch and head_dim must match k/v")
    if k.shape[1] != k_cache.shape[1] or k.shape[2] != k_cache.shape[3]:
        raise ValueError("k/v heads and head_dim must match cache")
    if block_ids.dim() != 1 or block_offsets.dim() != 1 or positions.dim() != 1:
        raise ValueError("block_ids, block_offsets, and positions must be rank-1 tensors")
    if block_ids.numel() != q.shape[0] or block_offsets.numel() != q.shape[0]:
        raise ValueError("block_ids and block_offsets lengths must match batch")
    if positions.numel() != q.shape[0]:
        raise ValueError("positions length must match batch")
    if any(t.dtype not in (torch.int32, torch.int64) for t in (block_ids, block_offsets, positions)):
        raise ValueError("block_ids, block_offsets, and positions must use int32 or int64")
    if any(t.device != q.device for t in (k, v, k_cache, v_cache, block_ids, block_offsets, positions)):
        raise ValueError("all fused RoPE + KV append inputs must share one CUDA device")
    if any(t.dtype != q.dtype for t in (k, v, k_cache, v_cache)):
        raise ValueError("q, k, v, and K/V caches must share one dtype")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("fused RoPE + KV append supports float16, bfloat16, and float32")

    head_dim = q.shape[-1]
    if isinstance(rotary_dim, bool) or not isinstance(rotary_dim, int):
        raise ValueError("rotary_dim must be an even integer")
    if rotary_dim <= 0 or rotary_dim > head_dim or rotary_dim % 2 != 0:
        raise ValueError("rotary_dim must be positive, even, and no larger than head_dim")
    base = float(base)
    if not math.isfinite(base) or base <= 0.0:
        raise ValueError("base must be a positive finite number")
    return base


def _validate_index_values(block_ids, block_offsets, positions, num_blocks, block_size):
    """Synchronous device-value checks of the public primitive (:128-145)."""
    if bool(torch.any(block_ids < 0).item()) or bool(torch.any(block_ids >= num_blocks).item()):
        raise ValueError("block_ids must be within [0, num_blocks)")
    if bool(torch.any(block_offsets < 0).item()) or bool(torch.any(block_offsets >= block_size).item()):
        raise ValueError("block_offsets must be within [0, block_size)")
    if bool(torch.any(positions < 0).item()):
        raise ValueError("positions must be non-negative")


def _check_cos_sin_table(table, rotary_dim, device):
    """A cos/sin table from :func:`flashdec_amd.rope.rope_cos_sin_table` for this rotary width."""
    if not isinstance(table, torch.Tensor):
        raise TypeError("cos_sin_table must be a torch.Tensor")
    if table.device != device:
        raise ValueError("cos_sin_table must be on the inputs' device")
    if table.dtype != torch.float32:
        raise ValueError("cos_sin_table must be float32")
    if table.dim() != 3 or table.shape[0] != 2 or table.shape[1] < 1 or table.shape[2] != rotary_dim // 2:
        raise ValueError("cos_sin_table must have shape [2, num_positions, rotary_dim // 2]")
    if not table.is_contiguous():
        raise ValueError("cos_sin_table must be contiguous")


def _prepare(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base):
    if rotary_dim is None:
        if not isinstance(q, torch.Tensor):
            raise TypeError("q must be a torch.Tensor")
        rotary_dim = q.shape[-1]
    base = _validate_structure(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base)
    return rotary_dim, base


def _launch(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base, q_out=None,
            cos_sin_table=None):
    """One ``fd_fused_rope_kv_append`` launch; the three index tensors share a dtype."""
    if q_out is None:
        q_out = torch.empty_like(q)
    if block_offsets.dtype != block_ids.dtype or positions.dtype != block_ids.dtype:
        # held here until the launch is enqueued
        block_ids = block_ids.to(torch.int64)
        block_offsets = block_offsets.to(torch.int64)
        positions = positions.to(torch.int64)
    args = _launch_args(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base, q_out,
                        cos_sin_table)
    _lib.rope_append(args, _lib.current_stream_handle(q.device), rotate=True)
    return q_out


def _launch_args(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base, q_out,
                 cos_sin_table):
    """The filled ``RopeAppendArgs`` of :func:`_launch` (checked inputs; the three index tensors
    share a dtype)."""
    idx_dtype = block_ids.dtype
    args = _lib.RopeAppendArgs()
    args.dtype = _lib.dtype_code(q.dtype)
    args.batch = q.shape[0]
    args.num_q_heads = q.shape[1]
    args.num_kv_heads = k.shape[1]
    args.head_dim = q.shape[2]
    args.block_size = k_cache.shape[2]
    args.num_blocks = k_cache.shape[0]
    args.rotary_dim = int(rotary_dim)
    args.base = float(base)
    args.q_out = q_out.data_ptr()
    args.q = q.data_ptr()
    args.k = k.data_ptr()
    args.v = v.data_ptr()
    args.k_cache = k_cache.data_ptr()
    args.v_cache = v_cache.data_ptr()
    args.block_ids = block_ids.data_ptr()
    args.block_offsets = block_offsets.data_ptr()
    args.positions = positions.data_ptr()
    args.index_dtype = _lib.index_code(idx_dtype)
    if cos_sin_table is not None:
        args.cos_sin_table = cos_sin_table.data_ptr()
        args.table_rows = cos_sin_table.shape[1]
    return args


def fused_rope_kv_append(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim=None,
                         base=10_000.0, cos_sin_table=None):
    """Rotate Q/K and append rotated K / raw V through one HIP kernel.

    The caller supplies allocated physical ``block_ids`` and ``block_offsets``
    (one per row).  Returns the rotated Q (new tensor, same shape/dtype); the
    caches are written in place.  Allocator state is not touched.

    ``cos_sin_table`` (no counterpart in the reference): a table from
    :func:`flashdec_amd.rope.rope_cos_sin_table` for this ``rotary_dim`` and
    ``base``; the kernel then reads cos/sin instead of evaluating them, and
    q_out and the K bytes equal :func:`flashdec_amd.rope.apply_rope` on the
    same device bit for bit.  Every position must be below its row count.
    """
    rotary_dim, base = _prepare(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base)
    _validate_index_values(block_ids, block_offsets, positions, k_cache.shape[0], k_cache.shape[2])
    if cos_sin_table is not None:
        _check_cos_sin_table(cos_sin_table, rotary_dim, q.device)
        if bool(torch.any(positions >= cos_sin_table.shape[1]).item()):
            raise ValueError("positions must be below the cos_sin_table's rows")
    return _launch(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base,
                   cos_sin_table=cos_sin_table)


def _fused_rope_kv_append_trusted(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions,
                                  rotary_dim=None, base=10_000.0, q_out=None, cos_sin_table=None):
    """Launch with cache-owned transaction metadata: no device reductions, no syncs.

    A ``cos_sin_table`` must cover every position (the caller's contract here).
    """
    rotary_dim, base = _prepare(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base)
    if any(t.dtype != torch.int64 for t in (block_ids, block_offsets, positions)):
        raise ValueError("trusted transaction metadata must use int64")
    if cos_sin_table is not None:
        _check_cos_sin_table(cos_sin_table, rotary_dim, q.device)
    return _launch(q, k, v, k_cache, v_cache, block_ids, block_offsets, positions, rotary_dim, base, q_out=q_out,
                   cos_sin_table=cos_sin_table)
