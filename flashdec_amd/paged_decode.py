"""Paged single-token decode attention on MI355X through ``libflashdec_hip.so``.

Public surface follows cysong2025/flashdec ``flashdec/kernels/paged_decode.py``:

* :func:`paged_decode_attention` (= ``flashdec.decode``), :922-969
* :func:`paged_decode_attention_into`, :972-1264 (validation :645-725)
* :func:`_vllm_paged_decode_attention_into`, :728-919 (unchecked vLLM launcher)

Argument meaning, defaults and ``ValueError`` messages are the reference's.
``num_warps``/``num_stages`` are Triton launch knobs there; they are still
validated (callers and tests rely on the errors) but have no effect on the HIP
kernels.  With ``num_splits == 1`` and no ``split_kv_workspace`` the library
picks the split count itself (one (request, head) program per KV head cannot
fill 256 CUs); a caller that passes a workspace gets exactly ``num_splits``.
"""

from __future__ import annotations

import math
import threading

import torch

from . import _lib

_KV_LAYOUT_AXES = {
    "token_major": (2, 3),
    "dim_major": (3, 2),
}


def _layout_axes(kv_layout):
    try:
        return _KV_LAYOUT_AXES[kv_layout]
    except KeyError as exc:
        raise ValueError("kv_layout must be 'token_major' or 'dim_major'") from exc


def _validate_inputs(q, k_cache, v_cache, block_tables, seq_lens, block_size, num_warps, num_stages, kv_layout):
    """Argument contract of paged_decode.py:645-725 (same messages)."""
    token_axis, dim_axis = _layout_axes(kv_layout)
    if q.device.type != "cuda" or k_cache.device.type != "cuda" or v_cache.device.type != "cuda":
        raise ValueError("q, k_cache, and v_cache must be CUDA tensors")
    if block_tables.device.type != "cuda" or seq_lens.device.type != "cuda":
        raise ValueError("block_tables and seq_lens must be CUDA tensors")
    if (
        q.device != k_cache.device
        or q.device != v_cache.device
        or q.device != block_tables.device
        or q.device != seq_lens.device
    ):
        raise ValueError("q, k_cache, v_cache, block_tables, and seq_lens must be on the same CUDA device")
    if q.dim() != 3:
        raise ValueError("q must have shape [num_seqs, num_q_heads, head_dim]")
    if k_cache.dim() != 4 or v_cache.dim() != 4:
        raise ValueError("k_cache and v_cache must be 4D tensors")
    if block_tables.dim() != 2:
        raise ValueError("block_tables must have shape [num_seqs, max_blocks_per_seq]")
    if seq_lens.dim() != 1:
        raise ValueError("seq_lens must have shape [num_seqs]")
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        raise ValueError("q, k_cache, and v_cache must have the same dtype")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("paged_decode_attention currently supports float16 and bfloat16 tensors")
    if block_tables.dtype not in (torch.int32, torch.int64):
        raise ValueError("block_tables must be int32 or int64")
    if seq_lens.dtype not in (torch.int32, torch.int64):
        raise ValueError("seq_lens must be int32 or int64")

    num_seqs, num_q_heads, head_dim = q.shape
    num_blocks, num_kv_heads = k_cache.shape[:2]
    v_num_blocks, v_num_kv_heads = v_cache.shape[:2]
    cache_block_size = k_cache.shape[token_axis]
    k_head_dim = k_cache.shape[dim_axis]
    v_block_size = v_cache.shape[token_axis]
    v_head_dim = v_cache.shape[dim_axis]
    if block_tables.shape[0] != num_seqs or seq_lens.numel() != num_seqs:
        raise ValueError("block_tables and seq_lens must have one row/value per sequence")
    if v_num_blocks != num_blocks:
        raise ValueError("k_cache and v_cache must have the same num_blocks")
    if num_blocks <= 0:
        raise ValueError("num_blocks must be positive")
    if num_seqs <= 0:
        raise ValueError("num_seqs must be positive")
    if num_q_heads <= 0 or num_kv_heads <= 0:
        raise ValueError("num_q_heads and num_kv_heads must be positive")
    if block_tables.shape[1] <= 0:
        raise ValueError("max_blocks_per_seq must be positive")
    if v_num_kv_heads != num_kv_heads:
        raise ValueError("k_cache and v_cache must have the same num_kv_heads")
    if v_block_size != cache_block_size:
        raise ValueError("k_cache and v_cache must have the same block_size")
    if cache_block_size != block_size:
        raise ValueError("block_size must match k_cache/v_cache shape")
    if block_size not in (8, 16, 32):
        raise ValueError("paged_decode_attention currently supports block_size 8, 16, or 32")
    if k_head_dim != head_dim or v_head_dim != head_dim:
        raise ValueError("q, k_cache, and v_cache must have the same head_dim")
    if head_dim not in (64, 128):
        raise ValueError("paged_decode_attention currently supports head_dim 64 or 128")
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("num_q_heads must be divisible by num_kv_heads")
    if isinstance(num_warps, bool) or not isinstance(num_warps, int) or num_warps not in (1, 2, 4, 8):
        raise ValueError("num_warps must be one of 1, 2, 4, or 8")
    if num_stages is not None and (
        isinstance(num_stages, bool) or not isinstance(num_stages, int) or num_stages not in (1, 2, 3, 4)
    ):
        raise ValueError("num_stages must be None or one of 1, 2, 3, or 4")


def _cache_strides(cache, token_axis, dim_axis):
    return (cache.stride(0), cache.stride(1), cache.stride(token_axis), cache.stride(dim_axis))


def _fill_common(args, q, k_cache, v_cache, k_strides, v_strides, block_tables, seq_lens, out,
                 num_kv_heads, block_size, sm_scale):
    num_seqs, num_q_heads, head_dim = q.shape
    args.dtype = _lib.dtype_code(q.dtype)
    args.num_seqs = num_seqs
    args.num_q_heads = num_q_heads
    args.num_kv_heads = num_kv_heads
    args.head_dim = head_dim
    args.block_size = block_size
    args.max_blocks_per_seq = block_tables.shape[1]
    args.q = q.data_ptr()
    args.q_stride[:] = q.stride()
    args.k_cache = k_cache.data_ptr()
    args.k_stride[:] = k_strides
    args.v_cache = v_cache.data_ptr()
    args.v_stride[:] = v_strides
    args.block_tables = block_tables.data_ptr()
    args.block_tables_dtype = _lib.index_code(block_tables.dtype)
    args.block_tables_stride[:] = block_tables.stride()
    args.seq_lens = seq_lens.data_ptr()
    args.seq_lens_dtype = _lib.index_code(seq_lens.dtype)
    args.seq_lens_stride = seq_lens.stride(0)
    args.out = out.data_ptr()
    args.out_stride[:] = out.stride()
    args.sm_scale = float(sm_scale)


def _fill_workspace(args, acc, mx, sm, num_splits, counters=None):
    args.num_splits = num_splits
    if num_splits > 1:
        args.split_acc = acc.data_ptr()
        args.split_acc_stride[:] = acc.stride()
        args.split_max = mx.data_ptr()
        args.split_sum = sm.data_ptr()
        args.split_stats_stride[:] = mx.stride()
        if counters is not None:
            args.split_counters = counters.data_ptr()


def _fill_append(args, append_k, append_v, slot_mapping):
    args.append_k = append_k.data_ptr()
    args.append_k_stride[:] = append_k.stride()
    args.append_v = append_v.data_ptr()
    args.append_v_stride[:] = append_v.stride()
    args.slot_mapping = slot_mapping.data_ptr()
    args.slot_mapping_dtype = _lib.index_code(slot_mapping.dtype)
    args.slot_mapping_stride = slot_mapping.stride(0)


class _SplitWorkspace:
    """fp32 split partials (plus zeroed arrival counters), reused across calls.

    One per (device, stream): launches on one stream are ordered.  The
    library-chosen split path merges with the second (reducer) kernel, which
    measured faster on MI355X than the in-launch merge (whose arrival atomics
    serialise at the memory side); the counters are kept for callers that opt
    into the in-launch merge and are left at zero by every launch.  Inside a
    graph capture with no workspace yet for the capturing stream, a private
    one is allocated for that call only.
    """

    __slots__ = ("flat", "counters")

    def __init__(self, device, floats, counters):
        self.flat = torch.empty(floats, device=device, dtype=torch.float32)
        self.counters = torch.zeros(counters, device=device, dtype=torch.int32)

    def views(self, num_seqs, num_q_heads, num_splits, head_dim):
        # acc rows first (16-byte aligned: the kernels store and load them as
        # float4), then max and sum as two [B, Hq, S] planes with equal strides
        rows = num_seqs * num_q_heads * num_splits
        acc = self.flat[: rows * head_dim].view(num_seqs, num_q_heads, num_splits, head_dim)
        stats = self.flat[rows * head_dim : rows * (head_dim + 2)].view(2, num_seqs, num_q_heads, num_splits)
        return acc, stats[0], stats[1], self.counters


_WORKSPACES = {}


def _auto_workspace(q, num_kv_heads, num_splits, stream):
    num_seqs, num_q_heads, head_dim = q.shape
    floats = num_seqs * num_q_heads * num_splits * (head_dim + 2)
    counters = num_seqs * num_kv_heads * _lib.SPLIT_COUNTER_STRIDE
    key = (q.device.index, stream)
    ws = _WORKSPACES.get(key)
    if ws is None or ws.flat.numel() < floats or ws.counters.numel() < counters:
        if torch.cuda.is_current_stream_capturing():
            return _SplitWorkspace(q.device, floats, counters).views(num_seqs, num_q_heads, num_splits, head_dim)
        grow = 1 if ws is None else 2
        ws = _SplitWorkspace(
            q.device,
            max(floats, grow * (ws.flat.numel() if ws else 0)),
            max(counters, grow * (ws.counters.numel() if ws else 0)),
        )
        _WORKSPACES[key] = ws
    return ws.views(num_seqs, num_q_heads, num_splits, head_dim)


def paged_decode_attention(
    q,
    k_cache,
    v_cache,
    block_tables,
    seq_lens,
    sm_scale=None,
    block_size=None,
    num_warps=2,
    kv_layout="token_major",
    num_stages=None,
    ragged=False,
    kv_reuse=False,
):
    """Return paged single-token decode attention (``flashdec.decode``).

    Shapes: q ``[num_seqs, num_q_heads, head_dim]``; token-major caches
    ``[num_blocks, num_kv_heads, block_size, head_dim]`` (dim-major:
    ``[num_blocks, num_kv_heads, head_dim, block_size]``); block_tables
    ``[num_seqs, max_blocks_per_seq]``; seq_lens ``[num_seqs]``.  Returns
    ``[num_seqs, num_q_heads, head_dim]`` in q.dtype.  block_size is inferred
    from the cache when omitted (paged_decode.py:950-955).  ``ragged`` and
    ``kv_reuse``: see :func:`paged_decode_attention_into`.
    """
    token_axis, _ = _layout_axes(kv_layout)
    if block_size is None:
        if k_cache.dim() != 4:
            raise ValueError("k_cache must be a 4D tensor")
        block_size = k_cache.shape[token_axis]
    else:
        block_size = int(block_size)
    out = torch.empty_like(q)
    return paged_decode_attention_into(
        q,
        k_cache,
        v_cache,
        block_tables,
        seq_lens,
        out,
        sm_scale=sm_scale,
        block_size=block_size,
        num_warps=num_warps,
        kv_layout=kv_layout,
        num_stages=num_stages,
        ragged=ragged,
        kv_reuse=kv_reuse,
    )


def paged_decode_attention_into(
    q,
    k_cache,
    v_cache,
    block_tables,
    seq_lens,
    out,
    sm_scale=None,
    block_size=None,
    num_warps=2,
    kv_layout="token_major",
    num_stages=None,
    split_kv_workspace=None,
    num_splits=1,
    append_k=None,
    append_v=None,
    slot_mapping=None,
    ragged=False,
    kv_reuse=False,
):
    """Write paged decode attention into ``out`` (no output allocation).

    K/V, block tables, seq_lens and out may be strided views; their strides go
    to the kernel as-is.  ``append_k``/``append_v``/``slot_mapping`` (together)
    fuse the current token's cache write: the kernel stores it at the slot and
    attends to it from registers.  Mirrors paged_decode.py:972-1264.

    ``ragged=True`` (no counterpart in the reference) tells the library-planned
    path that the batch's lengths vary widely: each row then gets splits in
    proportion to its length, counted on the device from ``seq_lens``
    (``balance_target`` of the C ABI).  It applies without fused append and
    without a caller workspace, and only where the batch leaves room in one
    round of workgroups; elsewhere it changes nothing.

    ``kv_reuse=True`` (no counterpart in the reference) says that rows share
    cache blocks (a common prefix in several rows' tables): K/V are then read
    with plain loads, so re-reads hit the caches.  By default each K/V row is
    assumed to be read once per call and is streamed with non-temporal loads.
    The result is the same either way.
    """
    key = None
    last = getattr(_LAST_LAUNCH, "entry", None)
    if last is not None and isinstance(q, torch.Tensor) and q.is_cuda:
        stream = _lib.current_stream_handle(q.device)
        try:
            key = _launch_key(q, k_cache, v_cache, block_tables, seq_lens, out, split_kv_workspace, append_k,
                              append_v, slot_mapping, (sm_scale, block_size, num_warps, kv_layout, num_stages,
                                                       num_splits, ragged, kv_reuse, stream))
        except (AttributeError, TypeError):
            key = None  # an argument that is not a tensor: the full path raises the reference's message
    if key is not None and last[0] == key:
        # the previous call's shapes, strides, dtypes, devices and settings:
        # its validation and plan stand; only the data pointers change
        args = last[1]
        _set_pointers(args, q, k_cache, v_cache, block_tables, seq_lens, out, split_kv_workspace, append_k,
                      append_v, slot_mapping)
    else:
        args, stream = _decode_args(q, k_cache, v_cache, block_tables, seq_lens, out, sm_scale, block_size,
                                    num_warps, kv_layout, num_stages, split_kv_workspace, num_splits, append_k,
                                    append_v, slot_mapping, ragged, kv_reuse)
        if key is None:
            key = _launch_key(q, k_cache, v_cache, block_tables, seq_lens, out, split_kv_workspace, append_k,
                              append_v, slot_mapping, (sm_scale, block_size, num_warps, kv_layout, num_stages,
                                                       num_splits, ragged, kv_reuse, stream))
        _LAST_LAUNCH.entry = (key, args)
    _lib.paged_decode(args, stream)
    return out


# The last launch of each thread: (metadata key, PagedDecodeArgs).
_LAST_LAUNCH = threading.local()


def _launch_key(q, k_cache, v_cache, block_tables, seq_lens, out, workspace, append_k, append_v, slot_mapping,
                settings):
    """Everything the validation, the plan and the launch arguments depend on except data pointers:
    each tensor's shape, strides, dtype and device, and the call's settings (with the stream, whose
    workspace the library plans into).  One flat tuple for the six tensors every call has (a quarter
    cheaper than a tuple per tensor: 1.3 against 1.8 us on the MI355X host)."""
    def meta(t):
        return None if t is None else (t.shape, t.stride(), t.dtype, t.device)

    app = None
    if append_k is not None or append_v is not None or slot_mapping is not None:
        app = (meta(append_k), meta(append_v), meta(slot_mapping))
    ws = None if workspace is None else tuple(meta(t) for t in workspace)
    return (settings, q.shape, q.stride(), q.dtype, q.device, k_cache.shape, k_cache.stride(), k_cache.dtype,
            k_cache.device, v_cache.shape, v_cache.stride(), v_cache.dtype, v_cache.device, block_tables.shape,
            block_tables.stride(), block_tables.dtype, block_tables.device, seq_lens.shape, seq_lens.stride(),
            seq_lens.dtype, seq_lens.device, out.shape, out.stride(), out.dtype, out.device, app, ws)


def _set_pointers(args, q, k_cache, v_cache, block_tables, seq_lens, out, workspace, append_k, append_v,
                  slot_mapping):
    args.q = q.data_ptr()
    args.k_cache = k_cache.data_ptr()
    args.v_cache = v_cache.data_ptr()
    args.block_tables = block_tables.data_ptr()
    args.seq_lens = seq_lens.data_ptr()
    args.out = out.data_ptr()
    if args.caller_workspace:
        args.split_acc = workspace[0].data_ptr()
        args.split_max = workspace[1].data_ptr()
        args.split_sum = workspace[2].data_ptr()
        args.workspace = tuple(workspace)
    if append_k is not None:
        args.append_k = append_k.data_ptr()
        args.append_v = append_v.data_ptr()
        args.slot_mapping = slot_mapping.data_ptr()


def _decode_args(q, k_cache, v_cache, block_tables, seq_lens, out, sm_scale, block_size, num_warps, kv_layout,
                 num_stages, split_kv_workspace, num_splits, append_k, append_v, slot_mapping, ragged, kv_reuse):
    """Validation, split plan and workspace of :func:`paged_decode_attention_into`: returns the
    filled ``PagedDecodeArgs`` and the stream handle, without launching."""
    token_axis, dim_axis = _layout_axes(kv_layout)
    if block_size is None:
        if k_cache.dim() != 4:
            raise ValueError("k_cache must be a 4D tensor")
        block_size = k_cache.shape[token_axis]
    else:
        block_size = int(block_size)

    _validate_inputs(q, k_cache, v_cache, block_tables, seq_lens, block_size, num_warps, num_stages, kv_layout)
    if out.shape != q.shape:
        raise ValueError("out must have the same shape as q")
    if out.dtype != q.dtype:
        raise ValueError("out must have the same dtype as q")
    if out.device != q.device:
        raise ValueError("out must be on the same device as q")
    if isinstance(num_splits, bool) or not isinstance(num_splits, int) or num_splits <= 0:
        raise ValueError("num_splits must be a positive integer")

    num_seqs, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[1]
    group_size = num_q_heads // num_kv_heads
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)

    use_grouped_gqa = head_dim == 128 and group_size in (4, 8, 16) and block_size in (16, 32)
    append_values = (append_k, append_v, slot_mapping)
    fuse_kv_append = all(value is not None for value in append_values)
    if any(value is not None for value in append_values) and not fuse_kv_append:
        raise ValueError("append_k, append_v, and slot_mapping must be provided together")
    if fuse_kv_append:
        if not use_grouped_gqa:
            raise ValueError("fused KV append requires grouped GQA decode")
        expected_append_shape = (num_seqs, num_kv_heads, head_dim)
        if append_k.shape != expected_append_shape or append_v.shape != expected_append_shape:
            raise ValueError("append_k and append_v must have shape [num_seqs, num_kv_heads, head_dim]")
        if append_k.dtype != q.dtype or append_v.dtype != q.dtype:
            raise ValueError("append_k and append_v must match q.dtype")
        if append_k.device != q.device or append_v.device != q.device:
            raise ValueError("append_k and append_v must be on q.device")
        if slot_mapping.dim() != 1 or slot_mapping.numel() < num_seqs:
            raise ValueError("slot_mapping must have at least one entry per sequence")
        if slot_mapping.dtype not in (torch.int32, torch.int64):
            raise ValueError("slot_mapping must be int32 or int64")
        if slot_mapping.device != q.device:
            raise ValueError("slot_mapping must be on q.device")

    use_split_kv = use_grouped_gqa and num_splits > 1
    if use_split_kv:
        if split_kv_workspace is None or len(split_kv_workspace) != 3:
            raise ValueError("split_kv_workspace must contain acc, max, and sum tensors")
        split_acc, split_max, split_sum = split_kv_workspace
        expected_acc = (num_seqs, num_q_heads, num_splits, head_dim)
        expected_stats = (num_seqs, num_q_heads, num_splits)
        if split_acc.dim() != 4 or split_max.dim() != 3 or split_sum.dim() != 3:
            raise ValueError("split KV workspace ranks must be 4, 3, and 3")
        if any(t.device != q.device or t.dtype != torch.float32 for t in split_kv_workspace):
            raise ValueError("split KV workspace tensors must be float32 on q.device")
        if any(a < e for a, e in zip(split_acc.shape, expected_acc)):
            raise ValueError("split acc workspace is too small")
        if any(a < e for a, e in zip(split_max.shape, expected_stats)):
            raise ValueError("split max workspace is too small")
        if any(a < e for a, e in zip(split_sum.shape, expected_stats)):
            raise ValueError("split sum workspace is too small")
        if split_sum.stride() != split_max.stride():
            raise ValueError("split max and sum workspaces must have identical strides")
    max_seq_len = block_tables.shape[1] * block_size
    stream = _lib.current_stream_handle(q.device)
    counters = None
    balance = 0
    if not use_split_kv:
        if ragged and not fuse_kv_append and use_grouped_gqa:
            balance = _lib.paged_decode_balance_target(num_seqs, num_kv_heads)
        if balance:
            num_splits = max(2, min(balance, -(-max_seq_len // 32)))
        else:
            num_splits = _lib.paged_decode_plan(num_seqs, num_q_heads, num_kv_heads, head_dim, max_seq_len)
            dim_major_mfma = head_dim in (64, 128)
            if kv_layout == "dim_major" and dim_major_mfma:
                if not fuse_kv_append:
                    # the dim-major kernel runs two 4-wave workgroups per CU:
                    # twice the splits, each still >= 4 tiles (one unit per wave)
                    num_splits = max(1, min(2 * num_splits, -(-max_seq_len // 128)))
            elif kv_layout == "dim_major" or head_dim not in (64, 128):
                # the generic kernel runs one wave per workgroup: 8x the splits
                # keeps ~8 waves per CU (dim-major B16 ctx8192: 515 -> 128 us),
                # at most one 64-token tile per split
                num_splits = max(1, min(8 * num_splits, -(-max_seq_len // 64), 4096))
        split_acc = split_max = split_sum = None
        if num_splits > 1:
            split_acc, split_max, split_sum, _ = _auto_workspace(q, num_kv_heads, num_splits, stream)

    args = _lib.PagedDecodeArgs()
    _fill_common(
        args,
        q,
        k_cache,
        v_cache,
        _cache_strides(k_cache, token_axis, dim_axis),
        _cache_strides(v_cache, token_axis, dim_axis),
        block_tables,
        seq_lens,
        out,
        num_kv_heads,
        block_size,
        sm_scale,
    )
    args.num_blocks = k_cache.shape[0]
    args.max_seq_len = max_seq_len
    args.balance_target = balance
    args.kv_reuse = 1 if kv_reuse else 0
    _fill_workspace(args, split_acc, split_max, split_sum, num_splits, counters)
    if fuse_kv_append:
        _fill_append(args, append_k, append_v, slot_mapping)
    # the workspace stays alive as long as the arguments that point into it
    # (a later, larger call may replace the stream's own workspace)
    args.workspace = (split_acc, split_max, split_sum)
    args.caller_workspace = use_split_kv
    return args, stream


def _decode_with_workspace(q, k_cache, v_cache, block_tables, seq_lens, out, sm_scale, block_size, num_splits,
                           workspace, num_blocks, balance_target=0, counters=None, kv_reuse=False, append=None,
                           rope=None):
    """Unchecked launch on a token-major cache with a caller-held split workspace (graph capture).

    ``workspace`` is ``(acc [B, Hq, S, D], max [B, Hq, S], sum [B, Hq, S])`` or
    None for ``num_splits == 1``; any head_dim / group the library supports.
    ``balance_target`` > 0 selects per-row split counts (at most
    ``num_splits``) computed on the device from ``seq_lens``.  ``counters``
    (zeroed int32, ``B * Hkv * SPLIT_COUNTER_STRIDE``) selects the in-launch
    merge: one dispatch, no reducer kernel.  ``kv_reuse``: plain instead of
    non-temporal K/V loads (rows share blocks).  ``append`` = ``(append_k,
    append_v, slot_mapping)`` fuses the current token's cache write; with it,
    ``rope`` = ``(rotary_dim, base)`` or ``(rotary_dim, base, cos_sin_table)``
    (rotary_dim 64 or 128, head_dim 128) takes ``q`` and ``append_k``
    unrotated and rotates both at position ``seq_len - 1`` inside the launch
    -- the same bits as the RoPE + append kernel (with the same table, if
    any) followed by this decode on the rotated q.  No counterpart in the
    reference.
    """
    num_kv_heads = k_cache.shape[1]
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[2])
    args = _lib.PagedDecodeArgs()
    _fill_common(args, q, k_cache, v_cache, _cache_strides(k_cache, 2, 3), _cache_strides(v_cache, 2, 3),
                 block_tables, seq_lens, out, num_kv_heads, block_size, sm_scale)
    args.num_blocks = num_blocks
    args.max_seq_len = block_tables.shape[1] * block_size
    args.balance_target = int(balance_target)
    args.kv_reuse = 1 if kv_reuse else 0
    acc, mx, sm = workspace if workspace is not None else (None, None, None)
    _fill_workspace(args, acc, mx, sm, int(num_splits), counters)
    if append is not None:
        _fill_append(args, *append)
    if rope is not None:
        args.rotary_dim = int(rope[0])
        args.rope_base = float(rope[1])
        if len(rope) > 2 and rope[2] is not None:
            args.rope_cos_sin_table = rope[2].data_ptr()
            args.rope_table_rows = rope[2].shape[1]
    _lib.paged_decode(args, _lib.current_stream_handle(q.device))
    return out


def _vllm_paged_decode_attention_into(
    q,
    append_k,
    append_v,
    kv_cache,
    block_tables,
    seq_lens,
    out,
    slot_mapping,
    split_acc,
    split_max,
    split_sum,
    *,
    num_reqs,
    num_q_heads,
    num_kv_heads,
    head_dim,
    block_size,
    sm_scale,
    num_splits,
    split_counters=None,
    max_seq_len=None,
    kv_reuse=False,
):
    """Checked-by-caller vLLM launcher (paged_decode.py:728-919).

    ``kv_cache`` is vLLM's whole ``[block, plane, token, kv_head, dim]``
    allocation (NHD or HND order through its strides): plane 0 is K, plane 1
    is V.  ``num_reqs`` rows are launched (graph padding included); rows with
    ``slot_mapping == -1`` produce zeros and write nothing; tensor rows past
    ``num_reqs`` are untouched.  No validation, allocation or copy happens.

    Extensions over the reference signature (both optional): ``split_counters``
    (zeroed int32 ``[>= num_reqs * num_kv_heads * 64]``, one 256-byte line per
    (request, KV head), left zero after every launch) merges the splits inside
    the one launch; ``max_seq_len`` (a hint such as vLLM's
    ``attn_metadata.max_seq_len``; any value is correct) lets the first
    tile's block-table and K/V reads of rows that long start before
    ``seq_lens`` arrives.  ``kv_reuse`` (rows share cache blocks, as with
    prefix caching) reads K/V with plain, cached loads instead of streaming
    them.
    """
    sb, sp, st, sh, sd = kv_cache.stride()
    plane_bytes = sp * kv_cache.element_size()
    base = kv_cache.data_ptr()
    args = _lib.PagedDecodeArgs()
    args.dtype = _lib.dtype_code(q.dtype)
    args.num_seqs = num_reqs
    args.num_q_heads = num_q_heads
    args.num_kv_heads = num_kv_heads
    args.head_dim = head_dim
    args.block_size = block_size
    args.num_blocks = kv_cache.shape[0]
    args.max_blocks_per_seq = block_tables.shape[1]
    args.q = q.data_ptr()
    args.q_stride[:] = q.stride()
    args.k_cache = base
    args.k_stride[:] = (sb, sh, st, sd)
    args.v_cache = base + plane_bytes
    args.v_stride[:] = (sb, sh, st, sd)
    args.block_tables = block_tables.data_ptr()
    args.block_tables_dtype = _lib.index_code(block_tables.dtype)
    args.block_tables_stride[:] = block_tables.stride()
    args.seq_lens = seq_lens.data_ptr()
    args.seq_lens_dtype = _lib.index_code(seq_lens.dtype)
    args.seq_lens_stride = seq_lens.stride(0)
    args.out = out.data_ptr()
    args.out_stride[:] = out.stride()
    args.sm_scale = float(sm_scale)
    args.max_seq_len = int(max_seq_len) if max_seq_len else 0
    args.kv_reuse = 1 if kv_reuse else 0
    _fill_workspace(args, split_acc, split_max, split_sum, int(num_splits), split_counters)
    _fill_append(args, append_k, append_v, slot_mapping)
    _lib.paged_decode(args, _lib.current_stream_handle(q.device))
    return out
