"""Paged KV cache runtime: block allocator, multi-layer token transactions,
refcounted shared prefixes -- host-side state with device-resident tables.

Semantics follow cysong2025/flashdec ``flashdec/cache.py`` (``PagedKVCache``,
:74-1409): the physical pool ``[num_layers, max_blocks, num_kv_heads,
block_size, head_dim]`` for K and V (:136-145), a deterministic free list
(``popleft`` to allocate, released blocks pushed back to the front in
reverse, :146, 1245-1255, 1269-1270), one open token transaction at a time
(:438-648), shared-prefix registry with LRU eviction (:192-276, 1365-1397),
the 45-key ``metrics()`` (:705-803) and ``validate_invariants()``
(:805-943).  Method names, arguments and error messages are the reference's
so callers drop in.

MI355X-specific: a transaction's metadata (positions, physical block ids,
offsets, padded block tables, effective lengths) is packed on the host into
one pinned staging buffer and sent with a single H2D copy when the
transaction opens; each layer's fused RoPE + append launch reads that
resident buffer directly.  Views handed to callers are device-side clones, so
a caller mutating them cannot reach the allocator's copy.
"""

from __future__ import annotations

import math
from collections import OrderedDict, deque
from dataclasses import dataclass, field, replace
from typing import Hashable

import numpy as np


@dataclass
class _RequestState:
    status: str = "active"
    seq_len: int = 0
    block_ids: list = field(default_factory=list)
    transaction_id: int | None = None
    prefix_id: Hashable | None = None
    shared_block_count: int = 0


@dataclass
class _PrefixState:
    block_ids: tuple
    active_refcount: int = 0


@dataclass(frozen=True)
class KVTokenTransactionView:
    """Detached public snapshot of one multi-layer token transaction."""

    transaction_id: int
    cache_version: int
    request_ids: tuple
    positions: object
    physical_block_ids: object
    block_offsets: object
    block_tables: object
    effective_seq_lens: object
    next_layer_idx: int
    state: str


def _meta_nbytes(capacity, width):
    return 32 * capacity + 4 * capacity * (1 + width)


class _DeviceMeta:
    """Transaction metadata resident on the cache device (one packed buffer).

    Layout for ``capacity`` rows (bytes): int64 positions[cap] | int64
    block_ids[cap] | int64 offsets[cap] | int64 slots[cap] (block_id *
    block_size + offset, the fused-append slot) | int32
    effective_seq_lens[cap] | int32 block_tables[cap, width].  The views
    cover the first ``batch`` rows, so a buffer laid out for a fixed capacity
    keeps every view's address whatever the batch (the graph-metadata arena).
    """

    __slots__ = ("buf", "capacity", "positions", "block_ids", "offsets", "slots", "eff_lens", "block_tables")

    def __init__(self, buf, batch, width, capacity=None):
        import torch

        capacity = batch if capacity is None else capacity
        self.buf = buf
        self.capacity = capacity
        i64 = buf[: 32 * capacity].view(torch.int64)
        self.positions = i64[:batch]
        self.block_ids = i64[capacity : capacity + batch]
        self.offsets = i64[2 * capacity : 2 * capacity + batch]
        self.slots = i64[3 * capacity : 3 * capacity + batch]
        i32 = buf[32 * capacity : _meta_nbytes(capacity, width)].view(torch.int32)
        self.eff_lens = i32[:batch]
        self.block_tables = i32[capacity : capacity + batch * width].view(batch, width)

    @classmethod
    def build(cls, device, positions, locations, table_rows, width, block_size, arena=None, staging=None):
        """Pack on the host and copy once (pinned staging for GPU caches).

        With ``arena`` (a device buffer laid out for ``arena_capacity`` rows of
        ``width`` table entries) the copy lands in the arena instead of a new
        buffer, staged through ``staging`` (a :class:`_StagingRing`).
        Otherwise pinned staging comes from torch's caching host allocator,
        which does not hand a block out again before its copy has completed.
        """
        import torch

        batch = len(positions)
        capacity = batch if arena is None else arena[1]
        nbytes = _meta_nbytes(capacity, width)
        pinned = device.type == "cuda"
        slot = None
        if staging is not None and pinned:
            slot, host = staging.acquire()
        else:
            host = torch.empty(nbytes, dtype=torch.uint8, pin_memory=pinned)
        arr = host.numpy()
        i64 = arr[: 32 * capacity].view(np.int64)
        i64[:batch] = positions
        i64[capacity : capacity + batch] = [blk for blk, _ in locations]
        i64[2 * capacity : 2 * capacity + batch] = [off for _, off in locations]
        i64[3 * capacity : 3 * capacity + batch] = [blk * block_size + off for blk, off in locations]
        i32 = arr[32 * capacity :].view(np.int32)
        i32[:batch] = [p + 1 for p in positions]
        i32[capacity : capacity + batch * width] = table_rows.reshape(-1)
        if arena is not None:
            arena[0][:nbytes].copy_(host[:nbytes], non_blocking=pinned)
            if slot is not None:
                staging.release(slot)
            return cls(arena[0], batch, width, capacity)
        buf = host.to(device, non_blocking=pinned) if pinned else host
        return cls(buf, batch, width)

    def clone(self):
        return _DeviceMeta(self.buf.clone(), self.positions.numel(), self.block_tables.shape[1], self.capacity)


class _StagingRing:
    """A few pinned host buffers for the per-step metadata copies, reused in turn.

    A buffer is refilled only after the copy that last read it has completed
    (its event), so the host runs at most ``depth`` steps ahead of the device
    and no pinned memory is allocated once the ring exists: letting torch's
    host allocator grow a pool while the host runs far ahead cost ~0.1 ms per
    step on MI355X.
    """

    def __init__(self, nbytes, depth=4):
        import torch

        self.bufs = [torch.empty(nbytes, dtype=torch.uint8, pin_memory=True) for _ in range(depth)]
        self.events = [None] * depth
        self.next = 0

    def acquire(self):
        i = self.next
        self.next = (i + 1) % len(self.bufs)
        if self.events[i] is not None:
            self.events[i].synchronize()
        return i, self.bufs[i]

    def release(self, i):
        import torch

        ev = torch.cuda.Event()
        ev.record()  # after the copy, on the current stream
        self.events[i] = ev


@dataclass
class _KVTokenTransactionState:
    transaction_id: int
    cache_version: int
    request_ids: tuple
    positions: tuple
    locations: tuple
    block_tables: object
    newly_allocated_by_request: dict
    allocation_order: tuple
    meta: object = None
    next_layer_idx: int = 0
    written_layers: set = field(default_factory=set)
    state: str = "open"


@dataclass(frozen=True)
class _TerminalTransactionState:
    """Metadata-only tombstone for a recently closed transaction."""

    transaction_id: int
    cache_version: int
    request_ids: tuple
    state: str


def _torch():
    import torch

    return torch


def _host_to_device(data, dtype, device):
    """A device tensor of host-side values, without a host wait.

    For a GPU the values are staged in pinned memory and copied on the
    current stream (``non_blocking``): a pageable copy would block the host
    until the stream's earlier work -- e.g. a replayed decode step -- has
    finished.  Pinned staging comes from torch's caching host allocator,
    which does not reuse the block before the copy has completed.
    """
    torch = _torch()
    device = torch.device(device)
    if device.type != "cuda":
        return torch.as_tensor(data, dtype=dtype).to(device)
    host = torch.as_tensor(data, dtype=dtype)
    return host.pin_memory().to(device, non_blocking=True)


class PagedKVCache:
    """Fixed-block KV cache runtime for single-token decode.

    Physical layout ``[num_layers, max_blocks, num_kv_heads, block_size,
    head_dim]`` (token-major within a block, the layout the HIP decode kernel
    streams with 16-byte loads).  Each request owns a logical list of physical
    blocks; appending a token writes into the current tail block or allocates
    a new one at a block boundary.  Requests may reference immutable full
    blocks of a registered shared prefix; their tail stays private.
    """

    ACTIVE = "active"
    FINISHED = "finished"
    CANCELLED = "cancelled"
    _TERMINAL_TRANSACTION_HISTORY_LIMIT = 256

    def __init__(self, num_layers, num_kv_heads, head_dim, block_size, max_blocks, dtype=None, device=None,
                 prefix_cache_capacity_blocks=0):
        torch = _torch()
        if dtype is None:
            dtype = torch.float16
        if device is None:
            device = "cuda" if torch.cuda.is_available() else "cpu"
        for name, value in [
            ("num_layers", num_layers),
            ("num_kv_heads", num_kv_heads),
            ("head_dim", head_dim),
            ("block_size", block_size),
            ("max_blocks", max_blocks),
        ]:
            if int(value) <= 0:
                raise ValueError(f"{name} must be positive")
        if not torch.empty((), dtype=dtype).is_floating_point():
            raise ValueError("dtype must be a floating point torch dtype")
        self.num_layers = int(num_layers)
        self.num_kv_heads = int(num_kv_heads)
        self.head_dim = int(head_dim)
        self.block_size = int(block_size)
        self.max_blocks = int(max_blocks)
        self.prefix_cache_capacity_blocks = int(prefix_cache_capacity_blocks)
        if self.prefix_cache_capacity_blocks < 0:
            raise ValueError("prefix_cache_capacity_blocks must be non-negative")
        if self.prefix_cache_capacity_blocks > self.max_blocks:
            raise ValueError("prefix_cache_capacity_blocks must not exceed max_blocks")
        self.dtype = dtype
        shape = (self.num_layers, self.max_blocks, self.num_kv_heads, self.block_size, self.head_dim)
        self.k_cache = torch.zeros(shape, device=device, dtype=dtype)
        self.device = self.k_cache.device
        self.v_cache = torch.zeros_like(self.k_cache)
        self._free_blocks = deque(range(self.max_blocks))
        self._requests: dict = {}
        self._prefixes: OrderedDict = OrderedDict()
        self._ever_allocated_blocks: set = set()
        self._allocation_count = 0
        self._fresh_allocation_count = 0
        self._free_count = 0
        self._reuse_count = 0
        self._capacity_failure_count = 0
        self._state_version = 0
        self._next_transaction_id = 1
        self._open_transaction_id = None
        self._transactions: dict = {}
        self._terminal_transactions: OrderedDict = OrderedDict()
        self._terminal_transaction_history_limit = self._TERMINAL_TRANSACTION_HISTORY_LIMIT
        self._transaction_begin_count = 0
        self._transaction_commit_count = 0
        self._transaction_abort_count = 0
        self._transaction_layer_write_count = 0
        self._transaction_rollback_block_count = 0
        self._transaction_failure_count = 0
        self._prefix_registration_count = 0
        self._prefix_hit_count = 0
        self._prefix_miss_count = 0
        self._prefix_eviction_count = 0
        self._prefix_capacity_failure_count = 0
        self._meta_arena = None  # (device buffer, capacity rows, table width) once enabled
        self._meta_staging = None  # pinned staging ring of the arena copies

    # ------------------------------------------------------------ lifecycle
    def add_request(self, request_id):
        """Register an empty request if it does not already exist."""
        if self._open_transaction_id is not None:
            raise RuntimeError("cannot add a request during an open token transaction")
        self._check_request_id(request_id)
        state = self._requests.get(request_id)
        if state is None:
            self._requests[request_id] = _RequestState()
            self._state_version += 1
        elif state.status != self.ACTIVE:
            raise RuntimeError(f"request_id {request_id!r} is {state.status} and cannot be reactivated")
        return self

    def finish_request(self, request_id):
        """Mark an active request finished and release its private blocks."""
        return self._close_request(request_id, self.FINISHED)

    def cancel_request(self, request_id):
        """Mark an active request cancelled and release its private blocks."""
        return self._close_request(request_id, self.CANCELLED)

    def _prefix_groups(self, request_ids):
        """Rows of ``request_ids`` attached to the same resident prefix, from
        host state: ``[(rows, prefix_blocks)]`` for prefixes with two or more
        of them (the rows' tables all lead with the prefix's blocks)."""
        by_prefix = {}
        for row, rid in enumerate(request_ids):
            state = self._require_request(rid)
            if state.prefix_id is not None and state.shared_block_count > 0:
                by_prefix.setdefault(state.prefix_id, (state.shared_block_count, []))[1].append(row)
        return [(rows, blocks) for blocks, rows in by_prefix.values() if len(rows) >= 2]

    def _host_seq_lens(self, request_ids):
        """Current lengths of known requests, from host state (no device access)."""
        return [self._require_request(rid).seq_len for rid in request_ids]

    def request_state(self, request_id):
        """Detached snapshot of one request's lifecycle state."""
        state = self._require_request(request_id)
        return {
            "request_id": request_id,
            "status": state.status,
            "seq_len": state.seq_len,
            "block_ids": tuple(state.block_ids),
            "prefix_id": state.prefix_id,
            "shared_block_count": state.shared_block_count,
        }

    # -------------------------------------------------------- shared prefix
    def register_prefix(self, prefix_id, k_blocks, v_blocks):
        """Copy immutable full K/V blocks ``[L, n, Hkv, bs, D]`` into the prefix registry.

        Inactive least-recently-used prefixes are evicted when the prefix
        capacity or the shared physical pool needs room.
        """
        if self._open_transaction_id is not None:
            raise RuntimeError("cannot register a prefix during an open token transaction")
        self._check_prefix_id(prefix_id)
        if prefix_id in self._prefixes:
            raise RuntimeError(f"prefix_id {prefix_id!r} is already registered")
        k_blocks, v_blocks = self._prepare_prefix_blocks(k_blocks, v_blocks)
        num_blocks = int(k_blocks.shape[1])
        plan = self._prefix_eviction_plan(num_blocks)
        if plan is None:
            self._capacity_failure_count += 1
            self._prefix_capacity_failure_count += 1
            raise RuntimeError("PagedKVCache has insufficient evictable prefix capacity")
        for evicted in plan:
            self._evict_prefix_entry(evicted)
        block_ids = tuple(self._allocate_block() for _ in range(num_blocks))
        index = _torch().tensor(block_ids, device=self.device, dtype=_torch().long)
        self.k_cache.index_copy_(1, index, k_blocks)
        self.v_cache.index_copy_(1, index, v_blocks)
        self._prefixes[prefix_id] = _PrefixState(block_ids=block_ids)
        self._prefix_registration_count += 1
        self._state_version += 1
        return self.prefix_state(prefix_id)

    def attach_prefix(self, request_id, prefix_id):
        """Attach a resident prefix to an empty active request."""
        if self._open_transaction_id is not None:
            raise RuntimeError("cannot attach a prefix during an open token transaction")
        self._check_prefix_id(prefix_id)
        state = self._require_active_request(request_id)
        if state.transaction_id is not None:
            raise RuntimeError("cannot attach a prefix to a request in a token transaction")
        if state.seq_len or state.block_ids or state.prefix_id is not None:
            raise RuntimeError("shared prefixes can only attach to an empty active request")
        prefix = self._prefixes.get(prefix_id)
        if prefix is None:
            self._prefix_miss_count += 1
            raise KeyError(f"unknown prefix_id: {prefix_id!r}")
        state.block_ids.extend(prefix.block_ids)
        state.seq_len = len(prefix.block_ids) * self.block_size
        state.prefix_id = prefix_id
        state.shared_block_count = len(prefix.block_ids)
        prefix.active_refcount += 1
        self._prefixes.move_to_end(prefix_id)
        self._prefix_hit_count += 1
        self._state_version += 1
        return tuple(prefix.block_ids)

    def evict_prefix(self, prefix_id):
        """Evict one inactive prefix and return its blocks to the free list."""
        if self._open_transaction_id is not None:
            raise RuntimeError("cannot evict a prefix during an open token transaction")
        self._check_prefix_id(prefix_id)
        prefix = self._prefixes.get(prefix_id)
        if prefix is None:
            raise KeyError(f"unknown prefix_id: {prefix_id!r}")
        if prefix.active_refcount:
            raise RuntimeError("cannot evict a prefix with active request references")
        released = self._evict_prefix_entry(prefix_id)
        self._state_version += 1
        return released

    def prefix_state(self, prefix_id):
        """Detached snapshot of one resident shared prefix."""
        self._check_prefix_id(prefix_id)
        prefix = self._prefixes.get(prefix_id)
        if prefix is None:
            raise KeyError(f"unknown prefix_id: {prefix_id!r}")
        return {
            "prefix_id": prefix_id,
            "block_ids": tuple(prefix.block_ids),
            "num_blocks": len(prefix.block_ids),
            "token_count": len(prefix.block_ids) * self.block_size,
            "active_refcount": prefix.active_refcount,
        }

    # ------------------------------------------------ single-layer appends
    def append(self, layer_idx, request_ids, k, v):
        """Append one K/V token per request (single-layer caches); returns block tables."""
        self._require_legacy_append_available()
        layer_idx, ids, k, v = self._prepare_append_inputs(layer_idx, request_ids, k, v)
        self._preflight_append(ids)
        locations = self._allocate_append_locations(ids)
        for row, (blk, off) in enumerate(locations):
            self.k_cache[layer_idx, blk, :, off, :] = k[row]
            self.v_cache[layer_idx, blk, :, off, :] = v[row]
        self._advance_request_lengths(ids)
        self._state_version += 1
        return self.block_tables(ids)

    def append_cuda(self, layer_idx, request_ids, k, v):
        """Append through the HIP K/V scatter (``fd_kv_append``); allocator stays on the host."""
        self._require_legacy_append_available()
        torch = _torch()
        layer_idx, ids, k, v = self._prepare_append_inputs(layer_idx, request_ids, k, v)
        if self.device.type != "cuda":
            raise ValueError("append_cuda requires a CUDA-resident PagedKVCache")
        if self.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("append_cuda supports cache dtype float16, bfloat16, or float32")
        if not k.is_contiguous() or not v.is_contiguous():
            raise ValueError("append_cuda requires contiguous k and v tensors")
        from ._kv_append import _launch_kv_append, load_cuda_kv_append_extension

        load_cuda_kv_append_extension()  # fail before any allocator mutation
        self._preflight_append(ids)
        locations = self._allocate_append_locations(ids)
        blk, off = self._location_tensors(locations)
        _launch_kv_append(self.k_cache[layer_idx], self.v_cache[layer_idx], blk, off, k, v)
        self._advance_request_lengths(ids)
        self._state_version += 1
        return self.block_tables(ids)

    append_hip = append_cuda

    def append_fused_cuda(self, layer_idx, request_ids, q, k, v, positions, rotary_dim=None, base=10_000.0):
        """Fused RoPE + K/V append via ``fd_fused_rope_kv_append``; returns ``(q_rot, tables)``."""
        self._require_legacy_append_available()
        torch = _torch()
        layer_idx, ids, k, v = self._prepare_append_inputs(layer_idx, request_ids, k, v)
        if self.device.type != "cuda":
            raise ValueError("append_fused_cuda requires a CUDA-resident PagedKVCache")
        if self.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError("append_fused_cuda supports cache dtype float16, bfloat16, or float32")
        if q.dim() != 3 or q.shape[0] != len(ids) or q.shape[1] <= 0 or q.shape[2] != self.head_dim:
            raise ValueError("q shape must match request count and cache head_dim")
        if q.device != self.device or q.dtype != self.dtype:
            raise ValueError("q must use the cache device and dtype")
        if positions.dim() != 1 or positions.numel() != len(ids):
            raise ValueError("positions must have shape [num_requests]")
        if positions.device != self.device or positions.dtype not in (torch.int32, torch.int64):
            raise ValueError("positions must use int32/int64 on the cache device")
        if bool(torch.any(positions < 0).item()):
            raise ValueError("positions must be non-negative")
        if rotary_dim is None:
            rotary_dim = self.head_dim
        if isinstance(rotary_dim, bool) or not isinstance(rotary_dim, int):
            raise ValueError("rotary_dim must be an even integer")
        if rotary_dim <= 0 or rotary_dim > self.head_dim or rotary_dim % 2 != 0:
            raise ValueError("rotary_dim must be positive, even, and no larger than head_dim")
        base = float(base)
        if not math.isfinite(base) or base <= 0.0:
            raise ValueError("base must be a positive finite number")
        if not q.is_contiguous() or not k.is_contiguous() or not v.is_contiguous():
            raise ValueError("append_fused_cuda requires contiguous q, k, and v tensors")
        from ._fused_rope_kv_append import _launch, load_fused_rope_kv_append_extension

        load_fused_rope_kv_append_extension()
        self._preflight_append(ids)
        locations = self._allocate_append_locations(ids)
        blk, off = self._location_tensors(locations)
        q_rot = _launch(q, k, v, self.k_cache[layer_idx], self.v_cache[layer_idx], blk, off,
                        positions.to(torch.int64), rotary_dim, base)
        self._advance_request_lengths(ids)
        self._state_version += 1
        return q_rot, self.block_tables(ids)

    append_fused_hip = append_fused_cuda

    # ---------------------------------------------- multi-layer transactions
    def begin_token(self, request_ids):
        """Reserve one token location (all layers) per request; blocks are allocated at boundaries."""
        if self._open_transaction_id is not None:
            raise RuntimeError("PagedKVCache already has an open token transaction")
        ids = tuple(self._normalize_request_ids(request_ids))
        if not ids:
            raise ValueError("request_ids must be non-empty")
        if len(set(ids)) != len(ids):
            raise ValueError("request_ids must be unique within one token transaction")
        states = [self._require_active_request(rid) for rid in ids]
        if any(s.transaction_id is not None for s in states):
            raise RuntimeError("request already belongs to an open token transaction")
        needed = sum(s.seq_len % self.block_size == 0 for s in states)
        if needed > len(self._free_blocks):
            self._capacity_failure_count += 1
            self._transaction_failure_count += 1
            raise RuntimeError("PagedKVCache is out of physical blocks")

        transaction_id = self._next_transaction_id
        positions = tuple(s.seq_len for s in states)
        locations = []
        newly_allocated = {}
        allocation_order = []
        try:
            for rid, s, pos in zip(ids, states, positions):
                off = pos % self.block_size
                if off == 0:
                    blk = self._allocate_block()
                    s.block_ids.append(blk)
                    newly_allocated[rid] = blk
                    allocation_order.append(blk)
                locations.append((s.block_ids[pos // self.block_size], off))
            self._validate_reserved_transaction_locations(ids, states, positions, locations)
            width = max(1, max(len(s.block_ids) for s in states))
            arena = self._meta_arena
            if arena is not None:
                if len(ids) > arena[1] or width > arena[2]:
                    raise RuntimeError("transaction exceeds the graph metadata arena "
                                       f"({len(ids)} rows x {width} blocks > {arena[1]} x {arena[2]})")
                width = arena[2]
            rows = self._table_rows(states, width)
            meta = _DeviceMeta.build(self.device, positions, locations, rows, width, self.block_size, arena,
                                     self._meta_staging)
            for s in states:
                s.transaction_id = transaction_id
        except Exception:
            for rid, blk in newly_allocated.items():
                s = self._requests[rid]
                if s.block_ids and s.block_ids[-1] == blk:
                    s.block_ids.pop()
                s.transaction_id = None
            for blk in reversed(allocation_order):
                self._free_blocks.appendleft(blk)
            self._transaction_failure_count += 1
            raise

        cache_version = self._state_version + 1
        state = _KVTokenTransactionState(
            transaction_id=transaction_id,
            cache_version=cache_version,
            request_ids=ids,
            positions=positions,
            locations=tuple(locations),
            block_tables=meta.block_tables,
            newly_allocated_by_request=newly_allocated,
            allocation_order=tuple(allocation_order),
            meta=meta,
        )
        self._transactions[transaction_id] = state
        self._open_transaction_id = transaction_id
        self._next_transaction_id += 1
        self._transaction_begin_count += 1
        self._state_version = cache_version
        return self._transaction_view(state)

    def write_token_layer(self, transaction, layer_idx, k, v):
        """Write one layer's K/V at the locations reserved by ``begin_token`` (torch path)."""
        state = self._require_open_transaction(transaction)
        try:
            layer_idx, k, v = self._prepare_transaction_layer_write(state, layer_idx, k, v)
            for row, (blk, off) in enumerate(state.locations):
                self.k_cache[layer_idx, blk, :, off, :] = k[row]
                self.v_cache[layer_idx, blk, :, off, :] = v[row]
        except Exception:
            self._transaction_failure_count += 1
            raise
        return self._record_transaction_layer_write(state, layer_idx)

    def write_token_layer_fused_cuda(self, transaction, layer_idx, q, k, v, *, rotary_dim=None, base=10_000.0,
                                     q_out=None, cos_sin_table=None):
        """Fused RoPE + K/V write of one layer at the transaction's reserved slots (HIP).

        The launch reads the allocator's own device copy of the reserved
        locations (resolved from the transaction id, never from the caller's
        view).  Returns ``(q_rotated, view)``.  ``cos_sin_table``: see
        :func:`flashdec_amd.rope.rope_cos_sin_table` (rows must cover the
        transaction's positions).
        """
        state = self._require_open_transaction(transaction)
        try:
            torch = _torch()
            layer_idx, k, v = self._prepare_transaction_layer_write(state, layer_idx, k, v)
            if self.device.type != "cuda":
                raise ValueError("write_token_layer_fused_cuda requires a CUDA-resident PagedKVCache")
            if self.dtype not in (torch.float16, torch.bfloat16, torch.float32):
                raise ValueError("write_token_layer_fused_cuda supports float16, bfloat16, or float32")
            if q.dim() != 3 or q.shape[0] != len(state.request_ids):
                raise ValueError("q shape must match transaction request count and cache head_dim")
            if q.shape[1] <= 0 or q.shape[2] != self.head_dim:
                raise ValueError("q shape must match transaction request count and cache head_dim")
            if q.device != self.device or q.dtype != self.dtype:
                raise ValueError("q must use the cache device and dtype")
            if not q.is_contiguous() or not k.is_contiguous() or not v.is_contiguous():
                raise ValueError("write_token_layer_fused_cuda requires contiguous q, k, and v tensors")
            from ._fused_rope_kv_append import _fused_rope_kv_append_trusted

            meta = state.meta
            q_rot = _fused_rope_kv_append_trusted(q, k, v, self.k_cache[layer_idx], self.v_cache[layer_idx],
                                                  meta.block_ids, meta.offsets, meta.positions,
                                                  rotary_dim=rotary_dim, base=base, q_out=q_out,
                                                  cos_sin_table=cos_sin_table)
        except Exception:
            self._transaction_failure_count += 1
            raise
        return q_rot, self._record_transaction_layer_write(state, layer_idx)

    write_token_layer_fused_hip = write_token_layer_fused_cuda

    def _record_graph_layers(self, transaction):
        """Record every layer as written by a replayed step graph (see DecodeEngine.step_graph)."""
        state = self._require_open_transaction(transaction)
        if state.next_layer_idx != 0:
            raise RuntimeError("a step graph writes every layer; this transaction already wrote some")
        for layer in range(self.num_layers):
            state.written_layers.add(layer)
        state.next_layer_idx = self.num_layers
        self._transaction_layer_write_count += self.num_layers

    def commit_token(self, transaction):
        """Publish the token after every layer has been written."""
        state = self._require_open_transaction(transaction)
        if state.next_layer_idx != self.num_layers:
            raise RuntimeError("cannot commit token before all layers are written")
        view = replace(self._transaction_view(state), state="committed")
        for rid in state.request_ids:
            r = self._requests[rid]
            r.seq_len += 1
            r.transaction_id = None
        state.state = "committed"
        self._open_transaction_id = None
        self._transaction_commit_count += 1
        self._state_version += 1
        self._retire_transaction(state)
        return view

    def abort_token(self, transaction):
        """Abort the open token and return the boundary blocks it reserved."""
        state = self._require_open_transaction(transaction)
        for rid, blk in state.newly_allocated_by_request.items():
            r = self._requests[rid]
            if not r.block_ids or r.block_ids[-1] != blk:
                raise RuntimeError("transaction rollback block ownership is inconsistent")
        view = replace(self._transaction_view(state), state="aborted")
        for rid in state.newly_allocated_by_request:
            self._requests[rid].block_ids.pop()
        for blk in reversed(state.allocation_order):
            self._free_blocks.appendleft(blk)
        for rid in state.request_ids:
            self._requests[rid].transaction_id = None
        state.state = "aborted"
        self._open_transaction_id = None
        self._transaction_abort_count += 1
        self._transaction_rollback_block_count += len(state.allocation_order)
        self._state_version += 1
        self._retire_transaction(state)
        return view

    def transaction_view(self, transaction):
        """Latest detached snapshot of an open transaction."""
        state = self._require_transaction(transaction)
        if isinstance(state, _TerminalTransactionState):
            raise RuntimeError(f"token transaction is already {state.state}")
        return self._transaction_view(state)

    def transaction_device_metadata(self, transaction):
        """The allocator's device-resident metadata of the open transaction.

        Read-only by contract: ``positions``/``block_ids``/``offsets``/``slots``
        (int64), ``eff_lens`` and ``block_tables`` (int32).  For launch paths (e.g.
        graph capture) that must not allocate per layer.
        """
        return self._require_open_transaction(transaction).meta

    def enable_graph_metadata(self, max_batch, max_blocks_per_seq):
        """Give every later transaction's metadata one fixed device address.

        A graph captured against ``graph_metadata()`` replays correctly for
        any later transaction of up to ``max_batch`` requests whose rows need
        at most ``max_blocks_per_seq`` blocks: ``begin_token`` packs positions,
        block ids, offsets, slots, effective lengths and the block table (padded to
        ``max_blocks_per_seq`` with -1) into the arena with one copy, ordered
        on the current stream after any earlier replay that reads it.
        """
        torch = _torch()
        if self._open_transaction_id is not None:
            raise RuntimeError("cannot change the metadata arena during an open token transaction")
        max_batch, width = int(max_batch), int(max_blocks_per_seq)
        if max_batch <= 0 or width <= 0:
            raise ValueError("max_batch and max_blocks_per_seq must be positive")
        buf = torch.zeros(_meta_nbytes(max_batch, width), dtype=torch.uint8, device=self.device)
        self._meta_arena = (buf, max_batch, width)
        self._meta_staging = _StagingRing(buf.numel()) if self.device.type == "cuda" else None
        return self.graph_metadata(max_batch)

    def graph_metadata(self, batch):
        """Views of the arena for a ``batch``-row transaction (fixed addresses)."""
        if self._meta_arena is None:
            raise RuntimeError("graph metadata arena is not enabled")
        buf, capacity, width = self._meta_arena
        if not 0 < int(batch) <= capacity:
            raise ValueError("batch must be in [1, arena capacity]")
        return _DeviceMeta(buf, int(batch), width, capacity)

    def seed_context(self, request_ids, num_tokens, k=None, v=None):
        """Commit ``num_tokens`` tokens per request at once (bulk set-up).

        The allocator ends in the state ``num_tokens`` single-token commits of
        this batch would leave: blocks are taken from the free list in the
        same interleaved order (every request's next block at each block
        boundary, in request order) and ``seq_len`` grows by ``num_tokens``.
        ``k``/``v`` ``[num_layers, B, num_tokens, Hkv, D]`` are scattered into
        the new slots; without them the slots keep the pool's bytes (e.g.
        synthetic benchmark data).  Transaction counters are not advanced.
        """
        torch = _torch()
        if self._open_transaction_id is not None:
            raise RuntimeError("cannot seed context during an open token transaction")
        ids = tuple(self._normalize_request_ids(request_ids))
        if not ids or len(set(ids)) != len(ids):
            raise ValueError("request_ids must be non-empty and unique")
        num_tokens = int(num_tokens)
        if num_tokens <= 0:
            raise ValueError("num_tokens must be positive")
        states = [self._require_active_request(rid) for rid in ids]
        if (k is None) != (v is None):
            raise ValueError("k and v must be provided together")
        if k is not None:
            shape = (self.num_layers, len(ids), num_tokens, self.num_kv_heads, self.head_dim)
            if tuple(k.shape) != shape or tuple(v.shape) != shape:
                raise ValueError("seed K/V must have shape [num_layers, num_requests, num_tokens, Hkv, D]")
            if k.device != self.device or v.device != self.device or k.dtype != self.dtype or v.dtype != self.dtype:
                raise ValueError("seed K/V must use the cache device and dtype")
        bs = self.block_size
        starts = [s.seq_len for s in states]
        needed = [(p + num_tokens + bs - 1) // bs - (p + bs - 1) // bs for p in starts]
        if sum(needed) > len(self._free_blocks):
            self._capacity_failure_count += 1
            raise RuntimeError("PagedKVCache is out of physical blocks")
        # block boundaries in token order, requests in order at each token
        for t in range(num_tokens):
            for s, p in zip(states, starts):
                if (p + t) % bs == 0:
                    s.block_ids.append(self._allocate_block())
        if k is not None:
            for row, (s, p) in enumerate(zip(states, starts)):
                pos = torch.arange(p, p + num_tokens, device=self.device)
                blk = torch.tensor(s.block_ids, device=self.device)[pos // bs]
                off = pos % bs
                # non-adjacent advanced indices put the token axis first: [T, L, Hkv, D]
                self.k_cache[:, blk, :, off, :] = k[:, row].permute(1, 0, 2, 3)
                self.v_cache[:, blk, :, off, :] = v[:, row].permute(1, 0, 2, 3)
        for s in states:
            s.seq_len += num_tokens
        self._state_version += 1
        return self.seq_lens_tensor(ids)

    # -------------------------------------------------------------- queries
    def next_positions(self, request_ids, device=None):
        """Each request's pre-append token position, without mutation."""
        torch = _torch()
        ids = self._normalize_request_ids(request_ids)
        if not ids:
            raise ValueError("request_ids must be non-empty")
        if len(set(ids)) != len(ids):
            raise ValueError("request_ids must be unique")
        positions = []
        for rid in ids:
            s = self._requests.get(rid)
            if s is None:
                positions.append(0)
            elif s.status != self.ACTIVE:
                raise RuntimeError(f"request_id {rid!r} is {s.status} and cannot accept append")
            elif s.transaction_id is not None:
                raise RuntimeError(f"request_id {rid!r} belongs to an open token transaction")
            else:
                positions.append(s.seq_len)
        return _host_to_device(positions, torch.int64, self.device if device is None else device)

    def block_tables(self, request_ids=None, max_blocks_per_seq=None, pad_value=-1):
        """Padded physical block ids ``[num_requests, max_blocks_per_seq]`` (int32)."""
        torch = _torch()
        ids = self._normalize_active_request_ids(request_ids)
        if max_blocks_per_seq is None:
            max_blocks_per_seq = max(1, max((len(self._requests[r].block_ids) for r in ids), default=0))
        max_blocks_per_seq = int(max_blocks_per_seq)
        if max_blocks_per_seq <= 0:
            raise ValueError("max_blocks_per_seq must be positive")
        states = [self._requests[r] for r in ids]
        if any(len(s.block_ids) > max_blocks_per_seq for s in states):
            raise ValueError("max_blocks_per_seq is smaller than a request's block count")
        rows = self._table_rows(states, max_blocks_per_seq, int(pad_value))
        return _host_to_device(rows, torch.int32, self.device)

    def seq_lens_tensor(self, request_ids=None, device=None):
        """Sequence lengths (int32) for the requested rows."""
        torch = _torch()
        ids = self._normalize_active_request_ids(request_ids)
        lens = [self._requests[r].seq_len for r in ids]
        return _host_to_device(lens, torch.int32, self.device if device is None else device)

    def request_block_ids(self, request_id):
        """Logical-to-physical block list of one request."""
        return tuple(self._require_request(request_id).block_ids)

    def to_dense(self, layer_idx=0, request_ids=None, max_seq_len=None):
        """Materialise ``(k_dense, v_dense, seq_lens)`` with K/V ``[B, L, Hkv, D]``."""
        torch = _torch()
        layer_idx = self._validate_layer_idx(layer_idx)
        ids = self._normalize_active_request_ids(request_ids)
        longest = max((self._requests[r].seq_len for r in ids), default=0)
        if max_seq_len is None:
            max_seq_len = max(1, longest)
        max_seq_len = int(max_seq_len)
        if max_seq_len < longest:
            raise ValueError("max_seq_len is smaller than an existing request length")
        shape = (len(ids), max_seq_len, self.num_kv_heads, self.head_dim)
        k_dense = torch.zeros(shape, device=self.device, dtype=self.dtype)
        v_dense = torch.zeros_like(k_dense)
        for row, rid in enumerate(ids):
            s = self._requests[rid]
            if s.seq_len == 0:
                continue
            index = torch.tensor(s.block_ids, device=self.device, dtype=torch.long)
            kt = self.k_cache[layer_idx].index_select(0, index).permute(0, 2, 1, 3)
            vt = self.v_cache[layer_idx].index_select(0, index).permute(0, 2, 1, 3)
            k_dense[row, : s.seq_len] = kt.reshape(-1, self.num_kv_heads, self.head_dim)[: s.seq_len]
            v_dense[row, : s.seq_len] = vt.reshape(-1, self.num_kv_heads, self.head_dim)[: s.seq_len]
        return k_dense, v_dense, self.seq_lens_tensor(ids)

    @property
    def num_free_blocks(self):
        return len(self._free_blocks)

    @property
    def num_used_blocks(self):
        return self.max_blocks - len(self._free_blocks)

    @property
    def state_version(self):
        return self._state_version

    @property
    def has_open_transaction(self):
        return self._open_transaction_id is not None

    def metrics(self):
        """Block-pool, fragmentation, lifecycle, transaction and prefix counters (45 keys)."""
        states = list(self._requests.values())
        active = [s for s in states if s.status == self.ACTIVE]
        used = self.num_used_blocks
        resident_prefix_blocks = self._resident_prefix_blocks()
        refs = sum(p.active_refcount for p in self._prefixes.values())
        shared_prefix_blocks = sum(len(p.block_ids) for p in self._prefixes.values() if p.active_refcount >= 2)
        saved_prefix_blocks = sum(max(0, p.active_refcount - 1) * len(p.block_ids) for p in self._prefixes.values())
        bytes_per_block = (self.num_layers * 2 * self.num_kv_heads * self.block_size * self.head_dim
                           * self.k_cache.element_size())
        open_tx = self._transactions.get(self._open_transaction_id) if self._open_transaction_id is not None else None
        reserved_tx_blocks = len(open_tx.allocation_order) if open_tx is not None else 0
        reserved_tokens = used * self.block_size
        active_tokens = sum(s.seq_len for s in active)
        physical_tokens = resident_prefix_blocks * self.block_size + sum(
            max(0, s.seq_len - s.shared_block_count * self.block_size) for s in active
        )
        frag = reserved_tokens - physical_tokens
        lookups = self._prefix_hit_count + self._prefix_miss_count
        return {
            "max_blocks": self.max_blocks,
            "used_blocks": used,
            "free_blocks": self.num_free_blocks,
            "block_utilization": used / self.max_blocks,
            "active_tokens": active_tokens,
            "physical_data_tokens": physical_tokens,
            "reserved_tokens": reserved_tokens,
            "internal_fragmentation_tokens": frag,
            "internal_fragmentation_ratio": frag / reserved_tokens if reserved_tokens else 0.0,
            "allocation_count": self._allocation_count,
            "fresh_allocation_count": self._fresh_allocation_count,
            "free_count": self._free_count,
            "reuse_count": self._reuse_count,
            "capacity_failure_count": self._capacity_failure_count,
            "active_requests": sum(s.status == self.ACTIVE for s in states),
            "finished_requests": sum(s.status == self.FINISHED for s in states),
            "cancelled_requests": sum(s.status == self.CANCELLED for s in states),
            "transaction_begin_count": self._transaction_begin_count,
            "transaction_commit_count": self._transaction_commit_count,
            "transaction_abort_count": self._transaction_abort_count,
            "open_transaction_count": int(open_tx is not None),
            "retained_transaction_state_count": len(self._transactions),
            "terminal_transaction_history_count": len(self._terminal_transactions),
            "terminal_transaction_history_limit": self._terminal_transaction_history_limit,
            "pending_request_count": len(open_tx.request_ids) if open_tx is not None else 0,
            "reserved_transaction_blocks": reserved_tx_blocks,
            "transaction_layer_write_count": self._transaction_layer_write_count,
            "transaction_rollback_block_count": self._transaction_rollback_block_count,
            "transaction_failure_count": self._transaction_failure_count,
            "bytes_per_block": bytes_per_block,
            "allocated_kv_bytes": used * bytes_per_block,
            "reserved_transaction_bytes": reserved_tx_blocks * bytes_per_block,
            "prefix_cache_capacity_blocks": self.prefix_cache_capacity_blocks,
            "resident_prefix_count": len(self._prefixes),
            "resident_prefix_blocks": resident_prefix_blocks,
            "active_prefix_references": refs,
            "shared_prefix_blocks": shared_prefix_blocks,
            "saved_prefix_blocks": saved_prefix_blocks,
            "saved_prefix_bytes": saved_prefix_blocks * bytes_per_block,
            "prefix_registration_count": self._prefix_registration_count,
            "prefix_hit_count": self._prefix_hit_count,
            "prefix_miss_count": self._prefix_miss_count,
            "prefix_hit_ratio": self._prefix_hit_count / lookups if lookups else 0.0,
            "prefix_eviction_count": self._prefix_eviction_count,
            "prefix_capacity_failure_count": self._prefix_capacity_failure_count,
        }

    def validate_invariants(self):
        """Raise RuntimeError if ownership, free list and transactions disagree."""
        free = list(self._free_blocks)
        if len(free) != len(set(free)):
            raise RuntimeError("PagedKVCache free list contains duplicate blocks")
        prefix_blocks = []
        expected_refs = {pid: 0 for pid in self._prefixes}
        for prefix in self._prefixes.values():
            if not prefix.block_ids:
                raise RuntimeError("resident prefix must own at least one block")
            if prefix.active_refcount < 0:
                raise RuntimeError("prefix active_refcount must be non-negative")
            prefix_blocks.extend(prefix.block_ids)
        if len(prefix_blocks) != len(set(prefix_blocks)):
            raise RuntimeError("a physical block belongs to multiple prefixes")
        if len(prefix_blocks) > self.prefix_cache_capacity_blocks:
            raise RuntimeError("resident prefixes exceed configured prefix capacity")
        private = []
        for s in self._requests.values():
            if s.status == self.ACTIVE:
                pending = int(s.transaction_id is not None)
                if len(s.block_ids) != (s.seq_len + pending + self.block_size - 1) // self.block_size:
                    raise RuntimeError("active request block count does not match seq_len")
                if s.prefix_id is None:
                    if s.shared_block_count:
                        raise RuntimeError("request without prefix has shared blocks")
                else:
                    prefix = self._prefixes.get(s.prefix_id)
                    if prefix is None:
                        raise RuntimeError("request references a non-resident prefix")
                    if s.shared_block_count != len(prefix.block_ids):
                        raise RuntimeError("request shared block count does not match prefix")
                    if tuple(s.block_ids[: s.shared_block_count]) != prefix.block_ids:
                        raise RuntimeError("request shared block ids do not match prefix")
                    if s.seq_len < s.shared_block_count * self.block_size:
                        raise RuntimeError("request seq_len is shorter than its shared prefix")
                    expected_refs[s.prefix_id] += 1
                private.extend(s.block_ids[s.shared_block_count :])
            else:
                if s.block_ids:
                    raise RuntimeError("terminal request still owns physical blocks")
                if s.transaction_id is not None:
                    raise RuntimeError("terminal request belongs to a token transaction")
                if s.prefix_id is not None or s.shared_block_count:
                    raise RuntimeError("terminal request still references a shared prefix")
        for pid, prefix in self._prefixes.items():
            if prefix.active_refcount != expected_refs[pid]:
                raise RuntimeError("prefix active_refcount does not match attached requests")
        if len(private) != len(set(private)):
            raise RuntimeError("a private physical block is owned by multiple requests")
        if set(private) & set(prefix_blocks):
            raise RuntimeError("a physical block is both private and prefix-owned")
        owned = prefix_blocks + private
        if set(owned) & set(free):
            raise RuntimeError("a physical block is both owned and free")
        if set(owned) | set(free) != set(range(self.max_blocks)):
            raise RuntimeError("physical block accounting does not cover the cache")
        if len(self._transactions) > 1:
            raise RuntimeError("PagedKVCache retains more than one transaction state")
        if any(t.state != "open" for t in self._transactions.values()):
            raise RuntimeError("terminal transaction retained device-backed state")
        if self._terminal_transaction_history_limit < 0:
            raise RuntimeError("terminal transaction history limit is negative")
        if len(self._terminal_transactions) > self._terminal_transaction_history_limit:
            raise RuntimeError("terminal transaction history exceeds its limit")
        if set(self._transactions) & set(self._terminal_transactions):
            raise RuntimeError("transaction appears in both open and terminal state")
        if any(t.state not in {"committed", "aborted"} for t in self._terminal_transactions.values()):
            raise RuntimeError("terminal transaction history contains an open state")
        terminal_ids = tuple(self._terminal_transactions)
        if any(tid != t.transaction_id for tid, t in self._terminal_transactions.items()):
            raise RuntimeError("terminal transaction history key does not match its state")
        if any(tid <= 0 or tid >= self._next_transaction_id for tid in terminal_ids):
            raise RuntimeError("terminal transaction history contains an invalid id")
        if any(t.cache_version <= 0 or t.cache_version > self._state_version
               for t in self._terminal_transactions.values()):
            raise RuntimeError("terminal transaction history contains an invalid version")
        if terminal_ids != tuple(sorted(terminal_ids)):
            raise RuntimeError("terminal transaction history is not ordered by id")
        open_states = list(self._transactions.values())
        if self._open_transaction_id is None:
            if open_states:
                raise RuntimeError("open transaction is missing from cache state")
            if any(s.transaction_id is not None for s in self._requests.values()):
                raise RuntimeError("request has an in-flight marker without an open transaction")
        else:
            if len(open_states) != 1:
                raise RuntimeError("PagedKVCache must have exactly one open transaction")
            tx = open_states[0]
            if tx.transaction_id != self._open_transaction_id:
                raise RuntimeError("open transaction id does not match cache state")
            if tx.written_layers != set(range(tx.next_layer_idx)):
                raise RuntimeError("transaction written layers are not sequential")
            if not 0 <= tx.next_layer_idx <= self.num_layers:
                raise RuntimeError("transaction next layer is out of range")
            for rid, pos, loc in zip(tx.request_ids, tx.positions, tx.locations):
                r = self._require_active_request(rid)
                if r.transaction_id != tx.transaction_id:
                    raise RuntimeError("request transaction marker does not match")
                if pos != r.seq_len:
                    raise RuntimeError("transaction position is not the committed seq_len")
                if loc != (r.block_ids[pos // self.block_size], pos % self.block_size):
                    raise RuntimeError("transaction physical location does not match ownership")
        return True

    # ------------------------------------------------------------ internals
    def _table_rows(self, states, width, pad=-1):
        rows = np.full((len(states), width), pad, dtype=np.int32)
        for i, s in enumerate(states):
            if s.block_ids:
                rows[i, : len(s.block_ids)] = s.block_ids
        return rows

    def _location_tensors(self, locations):
        torch = _torch()
        arr = np.asarray(locations, dtype=np.int64).reshape(-1, 2)
        both = _host_to_device(np.ascontiguousarray(arr.T), torch.int64, self.device)
        return both[0], both[1]

    def _transaction_view(self, transaction):
        meta = transaction.meta.clone()
        return KVTokenTransactionView(
            transaction_id=transaction.transaction_id,
            cache_version=transaction.cache_version,
            request_ids=transaction.request_ids,
            positions=meta.positions,
            physical_block_ids=meta.block_ids,
            block_offsets=meta.offsets,
            block_tables=meta.block_tables,
            effective_seq_lens=meta.eff_lens,
            next_layer_idx=transaction.next_layer_idx,
            state=transaction.state,
        )

    def _require_transaction(self, transaction):
        if not isinstance(transaction, KVTokenTransactionView):
            raise TypeError("transaction must be a KVTokenTransactionView")
        state = self._transactions.get(transaction.transaction_id)
        if state is None:
            state = self._terminal_transactions.get(transaction.transaction_id)
        if state is None:
            raise RuntimeError("unknown token transaction")
        if transaction.cache_version != state.cache_version or transaction.request_ids != state.request_ids:
            raise RuntimeError("stale or invalid token transaction handle")
        return state

    def _retire_transaction(self, transaction):
        retained = self._transactions.pop(transaction.transaction_id, None)
        if retained is not transaction:
            raise RuntimeError("token transaction retention state is inconsistent")
        self._terminal_transactions[transaction.transaction_id] = _TerminalTransactionState(
            transaction_id=transaction.transaction_id,
            cache_version=transaction.cache_version,
            request_ids=transaction.request_ids,
            state=transaction.state,
        )
        while len(self._terminal_transactions) > self._terminal_transaction_history_limit:
            self._terminal_transactions.popitem(last=False)

    def _require_open_transaction(self, transaction):
        state = self._require_transaction(transaction)
        if state.state != "open":
            raise RuntimeError(f"token transaction is already {state.state}")
        if self._open_transaction_id != state.transaction_id:
            raise RuntimeError("token transaction is not the current open transaction")
        return state

    def _require_legacy_append_available(self):
        if self.num_layers != 1:
            raise RuntimeError("multi-layer cache writes require the token transaction API")
        if self._open_transaction_id is not None:
            raise RuntimeError("legacy append is not allowed during an open token transaction")

    def _prepare_append_inputs(self, layer_idx, request_ids, k, v):
        layer_idx = self._validate_layer_idx(layer_idx)
        ids = self._normalize_request_ids(request_ids)
        if not ids:
            raise ValueError("request_ids must be non-empty")
        if len(set(ids)) != len(ids):
            raise ValueError("request_ids must be unique within one append call")
        if k.dim() == 2 and len(ids) == 1:
            k = k.unsqueeze(0)
        if v.dim() == 2 and len(ids) == 1:
            v = v.unsqueeze(0)
        if k.dim() != 3 or v.dim() != 3:
            raise ValueError("k and v must have shape [num_requests, num_kv_heads, head_dim]")
        if k.shape != v.shape:
            raise ValueError("k and v must have the same shape")
        if k.shape != (len(ids), self.num_kv_heads, self.head_dim):
            raise ValueError("k and v shapes must match request count, num_kv_heads, and head_dim")
        if k.device != self.device or v.device != self.device:
            raise ValueError("k and v must be on the cache device")
        if k.dtype != self.dtype or v.dtype != self.dtype:
            raise ValueError("k and v must use the cache dtype")
        if not k.is_floating_point() or not v.is_floating_point():
            raise ValueError("k and v must be floating point tensors")
        return layer_idx, ids, k, v

    def _prepare_transaction_layer_write(self, state, layer_idx, k, v):
        layer_idx = self._validate_layer_idx(layer_idx)
        if layer_idx != state.next_layer_idx:
            raise RuntimeError(f"transaction requires layer {state.next_layer_idx}, got layer {layer_idx}")
        _, ids, k, v = self._prepare_append_inputs(layer_idx, state.request_ids, k, v)
        if tuple(ids) != state.request_ids:
            raise RuntimeError("transaction request order changed unexpectedly")
        return layer_idx, k, v

    def _record_transaction_layer_write(self, state, layer_idx):
        state.written_layers.add(layer_idx)
        state.next_layer_idx += 1
        self._transaction_layer_write_count += 1
        return self._transaction_view(state)

    def _validate_reserved_transaction_locations(self, request_ids, states, positions, locations):
        """Prove raw-kernel indices from host allocator state before publication."""
        if not len(request_ids) == len(states) == len(positions) == len(locations):
            raise RuntimeError("transaction location metadata has inconsistent rows")
        for rid, s, pos, (blk, off) in zip(request_ids, states, positions, locations):
            if pos < 0:
                raise RuntimeError("transaction position must be non-negative")
            if not 0 <= blk < self.max_blocks:
                raise RuntimeError("transaction physical block id is out of range")
            if not 0 <= off < self.block_size:
                raise RuntimeError("transaction block offset is out of range")
            if off != pos % self.block_size:
                raise RuntimeError("transaction block offset does not match position")
            logical = pos // self.block_size
            if logical >= len(s.block_ids):
                raise RuntimeError("transaction logical block is not allocated")
            if s.block_ids[logical] != blk:
                raise RuntimeError(f"transaction physical block does not match request {rid!r}")

    def _preflight_append(self, ids):
        needed = 0
        for rid in ids:
            s = self._requests.get(rid)
            if s is not None and s.status != self.ACTIVE:
                raise RuntimeError(f"request_id {rid!r} is {s.status} and cannot accept append")
            if (s.seq_len if s is not None else 0) % self.block_size == 0:
                needed += 1
        if needed > len(self._free_blocks):
            self._capacity_failure_count += 1
            raise RuntimeError("PagedKVCache is out of physical blocks")

    def _allocate_append_locations(self, ids):
        locations = []
        for rid in ids:
            s = self._requests.get(rid)
            if s is None:
                s = _RequestState()
                self._requests[rid] = s
            off = s.seq_len % self.block_size
            if off == 0:
                s.block_ids.append(self._allocate_block())
            locations.append((s.block_ids[s.seq_len // self.block_size], off))
        return locations

    def _advance_request_lengths(self, ids):
        for rid in ids:
            self._requests[rid].seq_len += 1

    def _allocate_block(self):
        if not self._free_blocks:
            raise RuntimeError("PagedKVCache is out of physical blocks")
        blk = self._free_blocks.popleft()
        self._allocation_count += 1
        if blk in self._ever_allocated_blocks:
            self._reuse_count += 1
        else:
            self._ever_allocated_blocks.add(blk)
            self._fresh_allocation_count += 1
        return blk

    def _close_request(self, request_id, terminal_status):
        if self._open_transaction_id is not None:
            raise RuntimeError("cannot close a request during an open token transaction")
        s = self._require_active_request(request_id)
        prefix = None
        if s.prefix_id is not None:
            prefix = self._prefixes.get(s.prefix_id)
            if prefix is None or prefix.active_refcount <= 0:
                raise RuntimeError("shared prefix reference accounting is inconsistent")
        released = tuple(s.block_ids[s.shared_block_count :])
        # K/V bytes are not cleared: ownership plus the next owner's seq_len mask them
        for blk in reversed(released):
            self._free_blocks.appendleft(blk)
        self._free_count += len(released)
        s.block_ids.clear()
        if prefix is not None:
            prefix.active_refcount -= 1
            self._prefixes.move_to_end(s.prefix_id)
        s.prefix_id = None
        s.shared_block_count = 0
        s.status = terminal_status
        self._state_version += 1
        return released

    def _validate_layer_idx(self, layer_idx):
        layer_idx = int(layer_idx)
        if layer_idx < 0 or layer_idx >= self.num_layers:
            raise ValueError("layer_idx must be in [0, num_layers)")
        return layer_idx

    def _normalize_request_ids(self, request_ids):
        torch = _torch()
        if isinstance(request_ids, torch.Tensor):
            if request_ids.dim() == 0:
                ids = [int(request_ids.detach().cpu().item())]
            else:
                ids = [int(x) for x in request_ids.detach().cpu().reshape(-1).tolist()]
        elif isinstance(request_ids, (str, bytes)):
            ids = [request_ids]
        else:
            try:
                ids = list(request_ids)
            except TypeError:
                ids = [request_ids]
        for rid in ids:
            self._check_request_id(rid)
        return ids

    def _normalize_active_request_ids(self, request_ids):
        if request_ids is None:
            ids = [rid for rid, s in self._requests.items() if s.status == self.ACTIVE]
        else:
            ids = self._normalize_request_ids(request_ids)
        for rid in ids:
            self._require_active_request(rid)
        return ids

    @staticmethod
    def _check_request_id(request_id):
        try:
            hash(request_id)
        except TypeError as exc:
            raise ValueError("request ids must be hashable") from exc

    @staticmethod
    def _check_prefix_id(prefix_id):
        if prefix_id is None:
            raise ValueError("prefix_id must not be None")
        try:
            hash(prefix_id)
        except TypeError as exc:
            raise ValueError("prefix ids must be hashable") from exc

    def _prepare_prefix_blocks(self, k_blocks, v_blocks):
        torch = _torch()
        if not isinstance(k_blocks, torch.Tensor) or not isinstance(v_blocks, torch.Tensor):
            raise TypeError("k_blocks and v_blocks must be torch tensors")
        if k_blocks.dim() != 5 or v_blocks.dim() != 5:
            raise ValueError("prefix K/V must have shape [num_layers, num_prefix_blocks, num_kv_heads, block_size, head_dim]")
        if k_blocks.shape != v_blocks.shape:
            raise ValueError("prefix k_blocks and v_blocks must have the same shape")
        tail = (self.num_kv_heads, self.block_size, self.head_dim)
        if k_blocks.shape[0] != self.num_layers or tuple(k_blocks.shape[2:]) != tail:
            raise ValueError("prefix K/V shape does not match the PagedKVCache layout")
        if k_blocks.shape[1] <= 0:
            raise ValueError("prefix must contain at least one full block")
        if k_blocks.device != self.device or v_blocks.device != self.device:
            raise ValueError("prefix K/V must be on the cache device")
        if k_blocks.dtype != self.dtype or v_blocks.dtype != self.dtype:
            raise ValueError("prefix K/V must use the cache dtype")
        return k_blocks, v_blocks

    def _resident_prefix_blocks(self):
        return sum(len(p.block_ids) for p in self._prefixes.values())

    def _prefix_eviction_plan(self, required_blocks):
        if required_blocks > self.prefix_cache_capacity_blocks:
            return None
        need = max(0, self._resident_prefix_blocks() + required_blocks - self.prefix_cache_capacity_blocks,
                   required_blocks - len(self._free_blocks))
        if not need:
            return ()
        released = 0
        plan = []
        for pid, prefix in self._prefixes.items():
            if prefix.active_refcount:
                continue
            plan.append(pid)
            released += len(prefix.block_ids)
            if released >= need:
                return tuple(plan)
        return None

    def _evict_prefix_entry(self, prefix_id):
        prefix = self._prefixes[prefix_id]
        if prefix.active_refcount:
            raise RuntimeError("cannot evict a prefix with active request references")
        del self._prefixes[prefix_id]
        for blk in reversed(prefix.block_ids):
            self._free_blocks.appendleft(blk)
        self._free_count += len(prefix.block_ids)
        self._prefix_eviction_count += 1
        return tuple(prefix.block_ids)

    def _require_request(self, request_id):
        s = self._requests.get(request_id)
        if s is None:
            raise KeyError(f"unknown request_id: {request_id!r}")
        return s

    def _require_active_request(self, request_id):
        s = self._require_request(request_id)
        if s.status != self.ACTIVE:
            raise RuntimeError(f"request_id {request_id!r} is {s.status}, not active")
        return s
