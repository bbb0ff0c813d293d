"""Paged K/V scatter on MI355X (``fd_kv_append``).

Mirrors cysong2025/flashdec ``flashdec/_cuda_kv_append.py:62-137``: the public
name stays ``cuda_kv_append`` (device type is still "cuda" under ROCm torch)
so callers drop in unchanged.  Same validation and messages, including the
synchronous index-value checks; the kernel also range-checks every row.
"""

from __future__ import annotations

import torch

from . import _lib

_SUPPORTED_DTYPES = (torch.float16, torch.bfloat16, torch.float32)


def load_cuda_kv_append_extension():
    """Return the loaded C-ABI library (raises RuntimeError if it is not built)."""
    return _lib.load_library()


def _check_cuda_tensor(name, tensor):
    if not tensor.is_cuda:
        raise ValueError(f"{name} must be a CUDA tensor")
    if not tensor.is_contiguous():
        raise ValueError(f"{name} must be contiguous")


def _validate_inputs(k_cache, v_cache, block_ids, block_offsets, k, v):
    for name, tensor in [
        ("k_cache", k_cache),
        ("v_cache", v_cache),
        ("block_ids", block_ids),
        ("block_offsets", block_offsets),
        ("k", k),
        ("v", v),
    ]:
        if not isinstance(tensor, torch.Tensor):
            raise TypeError(f"{name} must be a torch.Tensor")
        _check_cuda_tensor(name, tensor)
    if k_cache.device != v_cache.device or k_cache.device != k.device or k_cache.device != v.device:
        raise ValueError("K/V caches and values must share one CUDA device")
    if block_ids.device != k_cache.device or block_offsets.device != k_cache.device:
        raise ValueError("block_ids and block_offsets must be on the cache CUDA device")
    if k_cache.dim() != 4:
        raise ValueError("k_cache must have shape [blocks, heads, block_size, head_dim]")
    if v_cache.shape != k_cache.shape:
        raise ValueError("v_cache must match k_cache shape")
    if k.dim() != 3 or v.dim() != 3:
        raise ValueError("k and v must have shape [batch, heads, head_dim]")
    if v.shape != k.shape:
        raise ValueError("v must match k shape")
    if k.shape[1:] != (k_cache.shape[1], k_cache.shape[3]):
        raise ValueError("k/v heads and head_dim must match cache")
    if block_ids.dim() != 1 or block_offsets.dim() != 1:
        raise ValueError("block_ids and block_offsets must be rank-1 tensors")
    if block_ids.numel() != k.shape[0] or block_offsets.numel() != k.shape[0]:
        raise ValueError("block_ids and block_offsets lengths must match batch")
    if block_ids.dtype not in (torch.int32, torch.int64):
        raise ValueError("block_ids must use int32 or int64")
    if block_offsets.dtype not in (torch.int32, torch.int64):
        raise ValueError("block_offsets must use int32 or int64")
    if k_cache.dtype != v_cache.dtype or k_cache.dtype != k.dtype or k_cache.dtype != v.dtype:
        raise ValueError("K/V caches and values must share one dtype")
    if k_cache.dtype not in _SUPPORTED_DTYPES:
        raise ValueError("CUDA KV append supports float16, bfloat16, and float32")
    if bool(torch.any(block_ids < 0).item()) or bool(torch.any(block_ids >= k_cache.shape[0]).item()):
        raise ValueError("block_ids must be within [0, num_blocks)")
    if bool(torch.any(block_offsets < 0).item()) or bool(torch.any(block_offsets >= k_cache.shape[2]).item()):
        raise ValueError("block_offsets must be within [0, block_size)")


def _launch_kv_append(k_cache, v_cache, block_ids, block_offsets, k, v):
    if block_offsets.dtype != block_ids.dtype:
        block_ids = block_ids.to(torch.int64)
        block_offsets = block_offsets.to(torch.int64)
    args = _lib.RopeAppendArgs()
    args.dtype = _lib.dtype_code(k_cache.dtype)
    args.batch = k.shape[0]
    args.num_q_heads = 0
    args.num_kv_heads = k.shape[1]
    args.head_dim = k.shape[2]
    args.block_size = k_cache.shape[2]
    args.num_blocks = k_cache.shape[0]
    args.k = k.data_ptr()
    args.v = v.data_ptr()
    args.k_cache = k_cache.data_ptr()
    args.v_cache = v_cache.data_ptr()
    args.block_ids = block_ids.data_ptr()
    args.block_offsets = block_offsets.data_ptr()
    args.index_dtype = _lib.index_code(block_ids.dtype)
    _lib.rope_append(args, _lib.current_stream_handle(k.device), rotate=False)


def cuda_kv_append(k_cache, v_cache, block_ids, block_offsets, k, v):
    """Write one K/V token per request into token-major physical cache blocks.

    k_cache/v_cache: contiguous ``[num_blocks, num_kv_heads, block_size, head_dim]``;
    block_ids/block_offsets: integer ``[batch]``; k/v: contiguous
    ``[batch, num_kv_heads, head_dim]``.  Returns None; allocator state is the
    caller's.
    """
    _validate_inputs(k_cache, v_cache, block_ids, block_offsets, k, v)
    _launch_kv_append(k_cache, v_cache, block_ids, block_offsets, k, v)
