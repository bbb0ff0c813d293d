"""Paged KV cache runtime: block pool, multi-layer token transactions and
refcounted shared prefixes -- host-side state with device-resident tables.

Public surface and observable behaviour follow cysong2025/flashdec
``flashdec/cache.py`` (``PagedKVCache``, :74-1409): the physical pool
``[num_layers, max_blocks, num_kv_heads, block_size, head_dim]`` for K and V
(:136-145), the order in which block ids are handed out and returned
(:146, 1245-1255, 1269-1270), one open token transaction at a time
(:438-648), the shared-prefix registry with LRU eviction (:192-276,
1365-1397), the 45-key ``metrics()`` (:705-803), ``validate_invariants()``
(:805-943), method names, arguments, error types and messages, and where the
state version advances.  Reference-recorded operation traces
(``tests/golden/cache_traces.json``) pin all of it.

Internal organisation (this module's own):

* :class:`_Pool` -- the free list and its allocation statistics; the only
  code that moves block ids in or out of it.
* :class:`_Seq` -- one request: status, committed length, page list (logical
  block -> physical block), the leading pages it borrows from a prefix, and
  the open transaction it belongs to.
* :class:`_PrefixBook` -- resident shared prefixes in LRU order.
* :class:`_Journal` -- the open transaction (:class:`_Txn`, at most one) and
  a bounded, tensor-free history of closed ones (:class:`_Closed`).
* :class:`_Tally` -- event counters reported by ``metrics()``.
* Argument contracts are rule tables (``_rules``) checked in order, and the
  ownership invariants are one rule list over a snapshot of the ledger.

MI355X-specific: a transaction's metadata (positions, physical block ids,
offsets, slots, padded block tables, effective lengths) is packed on the host
into one pinned staging buffer and sent with a single H2D copy when the
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


@dataclass(frozen=True)
class KVTokenTransactionView:
    """Detached public snapshot of one multi-layer token transaction.

    Its tensors are a device copy of the transaction's metadata, apart from
    the allocator's own; the views of one transaction share that copy (the
    metadata does not change while the transaction is open).
    """

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


def _rope_key(rotary_dim, base, cos_sin_table):
    """What a layer's prepared RoPE launch arguments depend on: the rotary width, the base and
    the cos/sin table (its address and rows)."""
    table = (0, 0) if cos_sin_table is None else (cos_sin_table.data_ptr(), tuple(cos_sin_table.shape))
    return rotary_dim, base, table


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


# ------------------------------------------------------------------ ledger --
OUT_OF_BLOCKS = "PagedKVCache is out of physical blocks"


class _Pool:
    """Free physical blocks (a deque: taken from the front; returned blocks go
    back to the front, last one first, so they are the next handed out) and
    allocation statistics."""

    __slots__ = ("free", "seen", "taken", "fresh", "reused", "released")

    def __init__(self, size):
        self.free = deque(range(size))
        self.seen = bytearray(size)  # 1 once a block has ever been handed out
        self.taken = 0
        self.fresh = 0
        self.reused = 0
        self.released = 0  # blocks given back by closed requests and evicted prefixes

    def __len__(self):
        return len(self.free)

    def take(self):
        if not self.free:
            raise RuntimeError(OUT_OF_BLOCKS)
        blk = self.free.popleft()
        self.taken += 1
        if self.seen[blk]:
            self.reused += 1
        else:
            self.seen[blk] = 1
            self.fresh += 1
        return blk

    def give_back(self, blocks, *, released):
        """Return ``blocks`` to the front so that ``blocks[0]`` is the next one
        taken; ``released`` counts them as freed (closing and eviction do,
        transaction rollback does not)."""
        for blk in reversed(blocks):
            self.free.appendleft(blk)
        if released:
            self.released += len(blocks)


@dataclass(eq=False)
class _Seq:
    """One request's ledger entry."""

    __slots__ = ("status", "length", "pages", "txn", "prefix", "shared")
    status: str
    length: int  # committed tokens
    pages: list  # physical block of each logical block
    txn: int | None  # id of the open transaction holding a reserved token
    prefix: Hashable | None
    shared: int  # leading pages that belong to the prefix

    @classmethod
    def empty(cls):
        return cls("active", 0, [], None, None, 0)

    def private_pages(self):
        return self.pages[self.shared:]


@dataclass(eq=False)
class _PrefixEntry:
    __slots__ = ("pages", "refs")
    pages: tuple
    refs: int


class _PrefixBook:
    """Resident prefixes, least recently used first."""

    __slots__ = ("entries",)

    def __init__(self):
        self.entries: OrderedDict = OrderedDict()

    def __contains__(self, pid):
        return pid in self.entries

    def get(self, pid):
        return self.entries.get(pid)

    def touch(self, pid):
        self.entries.move_to_end(pid)

    def resident_blocks(self):
        return sum(len(e.pages) for e in self.entries.values())

    def room_plan(self, blocks, capacity, free):
        """Idle prefixes to evict (LRU first) so that ``blocks`` more fit both
        the prefix capacity and the free pool: ``()`` if none need to go,
        None if even evicting every idle prefix would not do."""
        if blocks > capacity:
            return None
        short = max(0, self.resident_blocks() + blocks - capacity, blocks - free)
        plan, gained = [], 0
        for pid, entry in self.entries.items():
            if gained >= short:
                break
            if not entry.refs:
                plan.append(pid)
                gained += len(entry.pages)
        return tuple(plan) if gained >= short else None

    def drop(self, pid):
        entry = self.entries[pid]
        if entry.refs:
            raise RuntimeError("cannot evict a prefix with active request references")
        del self.entries[pid]
        return entry.pages


@dataclass(eq=False)
class _Txn:
    """The open token transaction."""

    __slots__ = ("tid", "version", "rids", "positions", "slots", "grown", "meta", "layers", "phase", "view_meta",
                 "launch")
    tid: int
    version: int  # the state version its opening published
    rids: tuple
    positions: tuple  # pre-append length of each row
    slots: tuple  # (block, offset) of each row's reserved token
    grown: tuple  # (request id, block) of each page this transaction appended, in allocation order
    meta: object  # _DeviceMeta
    layers: int  # layers written so far (always 0 .. layers-1, in order)
    phase: str
    view_meta: object  # the callers' copy of meta, made by the first view (meta never changes); None before
    launch: object  # prepared fused RoPE + append arguments: ((RoPE key, q/k/v shapes), RopeAppendArgs) or None


@dataclass(frozen=True)
class _Closed:
    """Tensor-free record of a committed or aborted transaction."""

    __slots__ = ("tid", "version", "rids", "phase")
    tid: int
    version: int
    rids: tuple
    phase: str


class _Journal:
    """At most one open transaction plus the last ``limit`` closed ones."""

    __slots__ = ("open", "history", "limit", "next_id")

    def __init__(self, limit):
        self.open: _Txn | None = None
        self.history: OrderedDict = OrderedDict()
        self.limit = limit
        self.next_id = 1

    def find(self, handle):
        if not isinstance(handle, KVTokenTransactionView):
            raise TypeError("transaction must be a KVTokenTransactionView")
        tid = handle.transaction_id
        rec = self.open if self.open is not None and self.open.tid == tid else self.history.get(tid)
        if rec is None:
            raise RuntimeError("unknown token transaction")
        if handle.cache_version != rec.version or handle.request_ids != rec.rids:
            raise RuntimeError("stale or invalid token transaction handle")
        return rec

    def find_open(self, handle):
        rec = self.find(handle)
        if rec.phase != "open":
            raise RuntimeError(f"token transaction is already {rec.phase}")
        if self.open is not rec:
            raise RuntimeError("token transaction is not the current open transaction")
        return rec

    def close(self, txn, phase):
        if self.open is not txn:
            raise RuntimeError("token transaction retention state is inconsistent")
        txn.phase = phase
        self.open = None
        self.history[txn.tid] = _Closed(txn.tid, txn.version, txn.rids, phase)
        while len(self.history) > self.limit:
            self.history.popitem(last=False)


class _Tally:
    """Event counters (the pool keeps its own allocation statistics)."""

    __slots__ = ("capacity_failures", "begins", "commits", "aborts", "layer_writes", "rollback_blocks", "failures",
                 "prefix_registrations", "prefix_hits", "prefix_misses", "prefix_evictions",
                 "prefix_capacity_failures")

    def __init__(self):
        for name in self.__slots__:
            setattr(self, name, 0)


def _rules(*checks):
    """An argument contract: ``(predicate, exception type, message)`` rows, checked in order."""

    def check(*args):
        for ok, exc, msg in checks:
            if not ok(*args):
                raise exc(msg)

    return check


def _require_hashable(x, what="request ids"):
    try:
        hash(x)
    except TypeError as exc:
        raise ValueError(f"{what} must be hashable") from exc


# per-token K/V rows [num_requests, num_kv_heads, head_dim] for one layer
# (args: cache, row count, k, v)
_check_kv_rows = _rules(
    (lambda c, n, k, v: k.dim() == 3 and v.dim() == 3, ValueError,
     "k and v must have shape [num_requests, num_kv_heads, head_dim]"),
    (lambda c, n, k, v: k.shape == v.shape, ValueError, "k and v must have the same shape"),
    (lambda c, n, k, v: k.shape == (n, c.num_kv_heads, c.head_dim), ValueError,
     "k and v shapes must match request count, num_kv_heads, and head_dim"),
    (lambda c, n, k, v: k.device == c.device and v.device == c.device, ValueError,
     "k and v must be on the cache device"),
    (lambda c, n, k, v: k.dtype == c.dtype and v.dtype == c.dtype, ValueError, "k and v must use the cache dtype"),
    (lambda c, n, k, v: k.is_floating_point() and v.is_floating_point(), ValueError,
     "k and v must be floating point tensors"),
)

# shared-prefix blocks [num_layers, n, num_kv_heads, block_size, head_dim] (args: cache, k, v)
_check_prefix_blocks = _rules(
    (lambda c, k, v: isinstance(k, _torch().Tensor) and isinstance(v, _torch().Tensor), TypeError,
     "k_blocks and v_blocks must be torch tensors"),
    (lambda c, k, v: k.dim() == 5 and v.dim() == 5, ValueError,
     "prefix K/V must have shape [num_layers, num_prefix_blocks, num_kv_heads, block_size, head_dim]"),
    (lambda c, k, v: k.shape == v.shape, ValueError, "prefix k_blocks and v_blocks must have the same shape"),
    (lambda c, k, v: k.shape[0] == c.num_layers and tuple(k.shape[2:]) == (c.num_kv_heads, c.block_size, c.head_dim),
     ValueError, "prefix K/V shape does not match the PagedKVCache layout"),
    (lambda c, k, v: k.shape[1] > 0, ValueError, "prefix must contain at least one full block"),
    (lambda c, k, v: k.device == c.device and v.device == c.device, ValueError,
     "prefix K/V must be on the cache device"),
    (lambda c, k, v: k.dtype == c.dtype and v.dtype == c.dtype, ValueError, "prefix K/V must use the cache dtype"),
)

# q of a fused RoPE + append [num_requests, num_q_heads, head_dim] (args: cache, row count, q)
_check_fused_q = _rules(
    (lambda c, n, q: q.dim() == 3 and q.shape[0] == n and q.shape[1] > 0 and q.shape[2] == c.head_dim, ValueError,
     "q shape must match request count and cache head_dim"),
    (lambda c, n, q: q.device == c.device and q.dtype == c.dtype, ValueError, "q must use the cache device and dtype"),
)

_check_transaction_q = _rules(
    (lambda c, n, q: q.dim() == 3 and q.shape[0] == n and q.shape[1] > 0 and q.shape[2] == c.head_dim, ValueError,
     "q shape must match transaction request count and cache head_dim"),
    (lambda c, n, q: q.device == c.device and q.dtype == c.dtype, ValueError, "q must use the cache device and dtype"),
)


def _rotary_dim_and_base(head_dim, rotary_dim, base):
    if rotary_dim is None:
        rotary_dim = head_dim
    if isinstance(rotary_dim, bool) or not isinstance(rotary_dim, int):
        raise ValueError("rotary_dim must be an even integer")
    if not 0 < rotary_dim <= head_dim or rotary_dim % 2:
        raise ValueError("rotary_dim must be positive, even, and no larger than head_dim")
    base = float(base)
    if not math.isfinite(base) or base <= 0.0:
        raise ValueError("base must be a positive finite number")
    return rotary_dim, base


def _rows_unique(ids, message):
    if not ids:
        raise ValueError("request_ids must be non-empty")
    if len(set(ids)) != len(ids):
        raise ValueError(message)


# ------------------------------------------------------------------ facade --
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
        dtype = torch.float16 if dtype is None else dtype
        device = ("cuda" if torch.cuda.is_available() else "cpu") if device is None else device
        dims = {"num_layers": num_layers, "num_kv_heads": num_kv_heads, "head_dim": head_dim,
                "block_size": block_size, "max_blocks": max_blocks}
        for name, value in dims.items():
            if int(value) <= 0:
                raise ValueError(f"{name} must be positive")
        if not torch.empty((), dtype=dtype).is_floating_point():
            raise ValueError("dtype must be a floating point torch dtype")
        for name, value in dims.items():
            setattr(self, name, int(value))
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
        self._pool = _Pool(self.max_blocks)
        self._seqs: dict = {}  # request id -> _Seq, in first-seen order
        self._prefix_book = _PrefixBook()
        self._journal = _Journal(self._TERMINAL_TRANSACTION_HISTORY_LIMIT)
        self._tally = _Tally()
        self._version = 0
        self._meta_arena = None  # (device buffer, capacity rows, table width) once enabled
        self._meta_staging = None  # pinned staging ring of the arena copies
        # The HIP RoPE + append launches read cos/sin from the cache's own
        # tables (rope_table), evaluated with apply_rope's torch expression,
        # so the appended K and the rotated q equal the torch backend's bit
        # for bit.  False: the kernels evaluate cos/sin themselves (float64,
        # rounded once), which may differ from torch by one fp32 ulp.
        self.rope_tables = True
        self._rope_tables: dict = {}  # (rotary_dim, base) -> fp32 [2, rows, rotary_dim // 2]

    # ---------------------------------------------------------- state guards
    def _no_transaction(self, message):
        if self._journal.open is not None:
            raise RuntimeError(message)

    def _publish(self):
        """Advance the state version (every successful mutation does, once)."""
        self._version += 1

    def _seq(self, request_id):
        seq = self._seqs.get(request_id)
        if seq is None:
            raise KeyError(f"unknown request_id: {request_id!r}")
        return seq

    def _active_seq(self, request_id):
        seq = self._seq(request_id)
        if seq.status != self.ACTIVE:
            raise RuntimeError(f"request_id {request_id!r} is {seq.status}, not active")
        return seq

    def _prefix_entry(self, prefix_id):
        if prefix_id is None:
            raise ValueError("prefix_id must not be None")
        _require_hashable(prefix_id, "prefix ids")
        return self._prefix_book.get(prefix_id)

    def _pages_for(self, length):
        return -(-length // self.block_size)

    # ------------------------------------------------------------ lifecycle
    def add_request(self, request_id):
        """Register an empty request if it does not already exist."""
        self._no_transaction("cannot add a request during an open token transaction")
        _require_hashable(request_id)
        seq = self._seqs.get(request_id)
        if seq is None:
            self._seqs[request_id] = _Seq.empty()
            self._publish()
        elif seq.status != self.ACTIVE:
            raise RuntimeError(f"request_id {request_id!r} is {seq.status} and cannot be reactivated")
        return self

    def finish_request(self, request_id):
        """Mark an active request finished and release its private blocks."""
        return self._retire_request(request_id, self.FINISHED)

    def cancel_request(self, request_id):
        """Mark an active request cancelled and release its private blocks."""
        return self._retire_request(request_id, self.CANCELLED)

    def _retire_request(self, request_id, status):
        self._no_transaction("cannot close a request during an open token transaction")
        seq = self._active_seq(request_id)
        entry = self._prefix_book.get(seq.prefix) if seq.prefix is not None else None
        if seq.prefix is not None and (entry is None or entry.refs <= 0):
            raise RuntimeError("shared prefix reference accounting is inconsistent")
        # the K/V bytes stay: ownership and the next owner's length mask them
        released = tuple(seq.private_pages())
        self._pool.give_back(released, released=True)
        if entry is not None:
            entry.refs -= 1
            self._prefix_book.touch(seq.prefix)
        seq.pages, seq.prefix, seq.shared, seq.status = [], None, 0, status
        self._publish()
        return released

    def request_state(self, request_id):
        """Detached snapshot of one request's lifecycle state."""
        seq = self._seq(request_id)
        return {"request_id": request_id, "status": seq.status, "seq_len": seq.length,
                "block_ids": tuple(seq.pages), "prefix_id": seq.prefix, "shared_block_count": seq.shared}

    def _prefix_groups(self, request_ids):
        """Rows of ``request_ids`` attached to the same resident prefix, from
        host state: ``[(rows, prefix_blocks)]`` for prefixes with two or more
        of them (the rows' tables all lead with the prefix's blocks)."""
        by_prefix = {}
        for row, rid in enumerate(request_ids):
            seq = self._seq(rid)
            if seq.prefix is not None and seq.shared > 0:
                by_prefix.setdefault(seq.prefix, (seq.shared, []))[1].append(row)
        return [(rows, blocks) for blocks, rows in by_prefix.values() if len(rows) >= 2]

    def _host_seq_lens(self, request_ids):
        """Current lengths of known requests, from host state (no device access)."""
        return [self._seq(rid).length for rid in request_ids]

    # -------------------------------------------------------- shared prefix
    def register_prefix(self, prefix_id, k_blocks, v_blocks):
        """Copy immutable full K/V blocks ``[L, n, Hkv, bs, D]`` into the prefix registry.

        Inactive least-recently-used prefixes are evicted when the prefix
        capacity or the shared physical pool needs room.
        """
        self._no_transaction("cannot register a prefix during an open token transaction")
        self._prefix_entry(prefix_id)
        if prefix_id in self._prefix_book:
            raise RuntimeError(f"prefix_id {prefix_id!r} is already registered")
        _check_prefix_blocks(self, k_blocks, v_blocks)
        count = int(k_blocks.shape[1])
        plan = self._prefix_book.room_plan(count, self.prefix_cache_capacity_blocks, len(self._pool))
        if plan is None:
            self._tally.capacity_failures += 1
            self._tally.prefix_capacity_failures += 1
            raise RuntimeError("PagedKVCache has insufficient evictable prefix capacity")
        for victim in plan:
            self._evict(victim)
        pages = tuple(self._pool.take() for _ in range(count))
        index = _torch().tensor(pages, device=self.device, dtype=_torch().long)
        self.k_cache.index_copy_(1, index, k_blocks)
        self.v_cache.index_copy_(1, index, v_blocks)
        self._prefix_book.entries[prefix_id] = _PrefixEntry(pages, 0)
        self._tally.prefix_registrations += 1
        self._publish()
        return self.prefix_state(prefix_id)

    def attach_prefix(self, request_id, prefix_id):
        """Attach a resident prefix to an empty active request."""
        self._no_transaction("cannot attach a prefix during an open token transaction")
        self._prefix_entry(prefix_id)
        seq = self._active_seq(request_id)
        if seq.txn is not None:
            raise RuntimeError("cannot attach a prefix to a request in a token transaction")
        if seq.length or seq.pages or seq.prefix is not None:
            raise RuntimeError("shared prefixes can only attach to an empty active request")
        entry = self._prefix_book.get(prefix_id)
        if entry is None:
            self._tally.prefix_misses += 1
            raise KeyError(f"unknown prefix_id: {prefix_id!r}")
        seq.pages.extend(entry.pages)
        seq.length = len(entry.pages) * self.block_size
        seq.prefix, seq.shared = prefix_id, len(entry.pages)
        entry.refs += 1
        self._prefix_book.touch(prefix_id)
        self._tally.prefix_hits += 1
        self._publish()
        return tuple(entry.pages)

    def evict_prefix(self, prefix_id):
        """Evict one inactive prefix and return its blocks to the free list."""
        self._no_transaction("cannot evict a prefix during an open token transaction")
        entry = self._prefix_entry(prefix_id)
        if entry is None:
            raise KeyError(f"unknown prefix_id: {prefix_id!r}")
        if entry.refs:
            raise RuntimeError("cannot evict a prefix with active request references")
        released = self._evict(prefix_id)
        self._publish()
        return released

    def _evict(self, prefix_id):
        pages = self._prefix_book.drop(prefix_id)
        self._pool.give_back(pages, released=True)
        self._tally.prefix_evictions += 1
        return tuple(pages)

    def prefix_state(self, prefix_id):
        """Detached snapshot of one resident shared prefix."""
        entry = self._prefix_entry(prefix_id)
        if entry is None:
            raise KeyError(f"unknown prefix_id: {prefix_id!r}")
        return {"prefix_id": prefix_id, "block_ids": tuple(entry.pages), "num_blocks": len(entry.pages),
                "token_count": len(entry.pages) * self.block_size, "active_refcount": entry.refs}

    # ------------------------------------------------ single-layer appends
    def _single_layer_rows(self, layer_idx, request_ids, k, v):
        """Common contract of the single-layer appends: returns (layer, ids, k, v)."""
        if self.num_layers != 1:
            raise RuntimeError("multi-layer cache writes require the token transaction API")
        self._no_transaction("legacy append is not allowed during an open token transaction")
        return self._kv_rows(layer_idx, request_ids, k, v, "request_ids must be unique within one append call")

    def _kv_rows(self, layer_idx, request_ids, k, v, duplicate_message):
        layer_idx = self._validate_layer_idx(layer_idx)
        ids = self._normalize_request_ids(request_ids)
        _rows_unique(ids, duplicate_message)
        if len(ids) == 1:
            k = k.unsqueeze(0) if k.dim() == 2 else k
            v = v.unsqueeze(0) if v.dim() == 2 else v
        _check_kv_rows(self, len(ids), k, v)
        return layer_idx, ids, k, v

    def _reserve_single_layer(self, ids):
        """Allocate each request's next slot (implicitly adding unknown ids);
        all-or-nothing: capacity is checked before anything changes."""
        grow = 0
        for rid in ids:
            seq = self._seqs.get(rid)
            if seq is not None and seq.status != self.ACTIVE:
                raise RuntimeError(f"request_id {rid!r} is {seq.status} and cannot accept append")
            grow += (seq.length if seq is not None else 0) % self.block_size == 0
        if grow > len(self._pool):
            self._tally.capacity_failures += 1
            raise RuntimeError(OUT_OF_BLOCKS)
        slots = []
        for rid in ids:
            seq = self._seqs.setdefault(rid, _Seq.empty())
            if seq.length % self.block_size == 0:
                seq.pages.append(self._pool.take())
            slots.append((seq.pages[seq.length // self.block_size], seq.length % self.block_size))
        return slots

    def _commit_single_layer(self, ids):
        for rid in ids:
            self._seqs[rid].length += 1
        self._publish()

    def append(self, layer_idx, request_ids, k, v):
        """Append one K/V token per request (single-layer caches); returns block tables."""
        layer_idx, ids, k, v = self._single_layer_rows(layer_idx, request_ids, k, v)
        for row, (blk, off) in enumerate(self._reserve_single_layer(ids)):
            self.k_cache[layer_idx, blk, :, off, :] = k[row]
            self.v_cache[layer_idx, blk, :, off, :] = v[row]
        self._commit_single_layer(ids)
        return self.block_tables(ids)

    def _require_gpu_cache(self, what):
        torch = _torch()
        if self.device.type != "cuda":
            raise ValueError(f"{what} requires a CUDA-resident PagedKVCache")
        if self.dtype not in (torch.float16, torch.bfloat16, torch.float32):
            raise ValueError(f"{what} supports cache dtype float16, bfloat16, or float32")

    def append_cuda(self, layer_idx, request_ids, k, v):
        """Append through the HIP K/V scatter (``fd_kv_append``); allocator stays on the host."""
        layer_idx, ids, k, v = self._single_layer_rows(layer_idx, request_ids, k, v)
        self._require_gpu_cache("append_cuda")
        if not k.is_contiguous() or not v.is_contiguous():
            raise ValueError("append_cuda requires contiguous k and v tensors")
        from ._kv_append import _launch_kv_append, load_cuda_kv_append_extension

        load_cuda_kv_append_extension()  # fail before any allocator mutation
        blk, off = self._slot_tensors(self._reserve_single_layer(ids))
        _launch_kv_append(self.k_cache[layer_idx], self.v_cache[layer_idx], blk, off, k, v)
        self._commit_single_layer(ids)
        return self.block_tables(ids)

    append_hip = append_cuda

    def rope_table(self, rotary_dim=None, base=10_000.0, rows=1):
        """The cache's cos/sin table for ``(rotary_dim, base)`` with at least ``rows`` rows.

        fp32 ``[2, R, rotary_dim // 2]`` on the cache device, built by
        :func:`flashdec_amd.rope.rope_cos_sin_table` (``apply_rope``'s own
        torch expression, flashdec/rope.py:66-70).  Row counts grow in powers
        of two (at least 4096) and never shrink; a grown table is a new
        tensor, so launches prepared or captured with the old one keep it
        alive through their own reference.  No counterpart in the reference.
        """
        from .rope import rope_cos_sin_table

        rotary_dim, base = _rotary_dim_and_base(self.head_dim, rotary_dim, base)
        rows = int(rows)
        table = self._rope_tables.get((rotary_dim, base))
        if table is None or table.shape[1] < rows:
            n = max(rows, 4096 if table is None else 2 * table.shape[1])
            table = rope_cos_sin_table(1 << (n - 1).bit_length(), rotary_dim, base, device=self.device)
            self._rope_tables[(rotary_dim, base)] = table
        return table

    def _launch_table(self, cos_sin_table, rotary_dim, base, max_position):
        """The cos/sin table a fused RoPE launch reads: the caller's (checked to cover
        ``max_position``), the cache's own by default, or None (cos/sin evaluated in the
        kernels) with ``rope_tables`` off."""
        if cos_sin_table is None:
            if not self.rope_tables or self.device.type != "cuda":
                return None
            return self.rope_table(rotary_dim, base, max_position + 1)
        if max_position >= cos_sin_table.shape[1]:
            raise ValueError("positions must be below the cos_sin_table's rows")
        return cos_sin_table

    def _txn_max_position(self, transaction):
        """Largest position the open transaction writes (host-side, no device sync)."""
        return max(self._journal.find_open(transaction).positions)

    def append_fused_cuda(self, layer_idx, request_ids, q, k, v, positions, rotary_dim=None, base=10_000.0,
                          cos_sin_table=None):
        """Fused RoPE + K/V append via ``fd_fused_rope_kv_append``; returns ``(q_rot, tables)``.

        ``cos_sin_table``: see :func:`flashdec_amd.rope.rope_cos_sin_table`;
        by default the cache's own table (:meth:`rope_table`), so q and K are
        rotated exactly as ``apply_rope`` rotates them on this device.
        """
        torch = _torch()
        layer_idx, ids, k, v = self._single_layer_rows(layer_idx, request_ids, k, v)
        self._require_gpu_cache("append_fused_cuda")
        _check_fused_q(self, len(ids), q)
        if positions.dim() != 1 or positions.numel() != len(ids):
            raise ValueError("positions must have shape [num_requests]")
        if positions.device != self.device or positions.dtype not in (torch.int32, torch.int64):
            raise ValueError("positions must use int32/int64 on the cache device")
        if bool(torch.any(positions < 0).item()):
            raise ValueError("positions must be non-negative")
        rotary_dim, base = _rotary_dim_and_base(self.head_dim, rotary_dim, base)
        if not q.is_contiguous() or not k.is_contiguous() or not v.is_contiguous():
            raise ValueError("append_fused_cuda requires contiguous q, k, and v tensors")
        from ._fused_rope_kv_append import _check_cos_sin_table, _launch, load_fused_rope_kv_append_extension

        if cos_sin_table is not None:
            _check_cos_sin_table(cos_sin_table, rotary_dim, self.device)
            if bool(torch.any(positions >= cos_sin_table.shape[1]).item()):
                raise ValueError("positions must be below the cos_sin_table's rows")
        elif self.rope_tables:
            cos_sin_table = self.rope_table(rotary_dim, base, int(positions.max().item()) + 1)
        load_fused_rope_kv_append_extension()
        blk, off = self._slot_tensors(self._reserve_single_layer(ids))
        q_rot = _launch(q, k, v, self.k_cache[layer_idx], self.v_cache[layer_idx], blk, off,
                        positions.to(torch.int64), rotary_dim, base, cos_sin_table=cos_sin_table)
        self._commit_single_layer(ids)
        return q_rot, self.block_tables(ids)

    append_fused_hip = append_fused_cuda

    # ---------------------------------------------- multi-layer transactions
    def begin_token(self, request_ids):
        """Reserve one token location (all layers) per request; blocks are allocated at boundaries."""
        self._no_transaction("PagedKVCache already has an open token transaction")
        ids = tuple(self._normalize_request_ids(request_ids))
        _rows_unique(ids, "request_ids must be unique within one token transaction")
        seqs = [self._active_seq(rid) for rid in ids]
        if any(seq.txn is not None for seq in seqs):
            raise RuntimeError("request already belongs to an open token transaction")
        if sum(seq.length % self.block_size == 0 for seq in seqs) > len(self._pool):
            self._tally.capacity_failures += 1
            self._tally.failures += 1
            raise RuntimeError(OUT_OF_BLOCKS)
        tid = self._journal.next_id
        positions = tuple(seq.length for seq in seqs)
        grown = []
        try:
            for rid, seq in zip(ids, seqs):
                if seq.length % self.block_size == 0:
                    blk = self._pool.take()
                    seq.pages.append(blk)
                    grown.append((rid, blk))
            slots = tuple((seq.pages[p // self.block_size], p % self.block_size) for seq, p in zip(seqs, positions))
            self._validate_reserved_transaction_locations(ids, seqs, positions, slots)
            meta = self._pack_metadata(seqs, positions, slots)
            for seq in seqs:
                seq.txn = tid
        except Exception:
            self._undo_growth(grown)
            for seq in seqs:
                seq.txn = None
            self._tally.failures += 1
            raise
        self._publish()
        txn = _Txn(tid, self._version, ids, positions, slots, tuple(grown), meta, 0, "open", None, None)
        self._journal.open = txn
        self._journal.next_id += 1
        self._tally.begins += 1
        return self._snapshot(txn)

    def _pack_metadata(self, seqs, positions, slots):
        """The transaction's device metadata: in the graph arena when enabled."""
        width = max(1, max(len(seq.pages) for seq in seqs))
        arena = self._meta_arena
        if arena is not None:
            if len(seqs) > arena[1] or width > arena[2]:
                raise RuntimeError("transaction exceeds the graph metadata arena "
                                   f"({len(seqs)} rows x {width} blocks > {arena[1]} x {arena[2]})")
            width = arena[2]
        return _DeviceMeta.build(self.device, positions, slots, self._table_rows(seqs, width), width,
                                 self.block_size, arena, self._meta_staging)

    def _undo_growth(self, grown):
        """Take back the pages a reservation appended (newest first) and return
        them to the front of the pool in allocation order."""
        for rid, blk in reversed(grown):
            pages = self._seqs[rid].pages
            if pages and pages[-1] == blk:
                pages.pop()
        self._pool.give_back([blk for _, blk in grown], released=False)

    def _validate_reserved_transaction_locations(self, request_ids, seqs, positions, slots):
        """Check every reserved (block, offset) against the ledger before any kernel sees it."""
        if not len(request_ids) == len(seqs) == len(positions) == len(slots):
            raise RuntimeError("transaction location metadata has inconsistent rows")
        for rid, seq, pos, (blk, off) in zip(request_ids, seqs, positions, slots):
            problem = (
                "transaction position must be non-negative" if pos < 0 else
                "transaction physical block id is out of range" if not 0 <= blk < self.max_blocks else
                "transaction block offset is out of range" if not 0 <= off < self.block_size else
                "transaction block offset does not match position" if off != pos % self.block_size else
                "transaction logical block is not allocated" if pos // self.block_size >= len(seq.pages) else
                f"transaction physical block does not match request {rid!r}"
                if seq.pages[pos // self.block_size] != blk else None)
            if problem is not None:
                raise RuntimeError(problem)

    def _layer_rows(self, txn, layer_idx, k, v):
        """One transaction layer write's contract: returns (layer, k, v).  The
        transaction's request ids were checked when it opened."""
        layer_idx = self._validate_layer_idx(layer_idx)
        if layer_idx != txn.layers:
            raise RuntimeError(f"transaction requires layer {txn.layers}, got layer {layer_idx}")
        if len(txn.rids) == 1:
            k = k.unsqueeze(0) if k.dim() == 2 else k
            v = v.unsqueeze(0) if v.dim() == 2 else v
        _check_kv_rows(self, len(txn.rids), k, v)
        return layer_idx, k, v

    def _layer_written(self, txn):
        txn.layers += 1
        self._tally.layer_writes += 1
        return self._snapshot(txn)

    def write_token_layer(self, transaction, layer_idx, k, v):
        """Write one layer's K/V at the locations reserved by ``begin_token`` (torch path)."""
        txn = self._journal.find_open(transaction)
        try:
            layer_idx, k, v = self._layer_rows(txn, layer_idx, k, v)
            for row, (blk, off) in enumerate(txn.slots):
                self.k_cache[layer_idx, blk, :, off, :] = k[row]
                self.v_cache[layer_idx, blk, :, off, :] = v[row]
        except Exception:
            self._tally.failures += 1
            raise
        return self._layer_written(txn)

    def write_token_layer_fused_cuda(self, transaction, layer_idx, q, k, v, *, rotary_dim=None, base=10_000.0,
                                     q_out=None, cos_sin_table=None):
        """Fused RoPE + K/V write of one layer at the transaction's reserved slots (HIP).

        The launch reads the allocator's own device copy of the reserved
        locations (resolved from the transaction id, never from the caller's
        view).  Returns ``(q_rotated, view)``.  ``cos_sin_table``: see
        :func:`flashdec_amd.rope.rope_cos_sin_table` (rows must cover the
        transaction's positions); by default the cache's own
        (:meth:`rope_table`).
        """
        txn = self._journal.find_open(transaction)
        try:
            torch = _torch()
            layer_idx, k, v = self._layer_rows(txn, layer_idx, k, v)
            if self.device.type != "cuda":
                raise ValueError("write_token_layer_fused_cuda requires a CUDA-resident PagedKVCache")
            if self.dtype not in (torch.float16, torch.bfloat16, torch.float32):
                raise ValueError("write_token_layer_fused_cuda supports float16, bfloat16, or float32")
            _check_transaction_q(self, len(txn.rids), q)
            if not q.is_contiguous() or not k.is_contiguous() or not v.is_contiguous():
                raise ValueError("write_token_layer_fused_cuda requires contiguous q, k, and v tensors")
            from ._fused_rope_kv_append import _fused_rope_kv_append_trusted

            rdim, rbase = _rotary_dim_and_base(self.head_dim, rotary_dim, base)
            cos_sin_table = self._launch_table(cos_sin_table, rdim, rbase, max(txn.positions))
            meta = txn.meta
            q_rot = _fused_rope_kv_append_trusted(q, k, v, self.k_cache[layer_idx], self.v_cache[layer_idx],
                                                  meta.block_ids, meta.offsets, meta.positions,
                                                  rotary_dim=rotary_dim, base=base, q_out=q_out,
                                                  cos_sin_table=cos_sin_table)
        except Exception:
            self._tally.failures += 1
            raise
        return q_rot, self._layer_written(txn)

    write_token_layer_fused_hip = write_token_layer_fused_cuda

    def _write_layer_fused_prepared(self, transaction, layer_idx, q, k, v, rotary_dim, base, cos_sin_table):
        """``write_token_layer_fused_cuda`` for ``DecodeEngine.step_layer``, whose step-input rules
        have checked q, k and v (types, [batch, heads, head_dim] shapes, device, dtype).

        The transaction's first layer (or a change of RoPE setting) goes the
        checked way and leaves the filled launch arguments in the
        transaction; its later layers check the layer order and contiguity
        and change only the q, out, k, v and per-layer cache pointers.
        """
        torch = _torch()
        from . import _lib

        txn = self._journal.find_open(transaction)
        try:
            rdim, rbase = _rotary_dim_and_base(self.head_dim, rotary_dim, base)
            cos_sin_table = self._launch_table(cos_sin_table, rdim, rbase, max(txn.positions))
        except Exception:
            self._tally.failures += 1
            raise
        # the prepared arguments fix the batch and head counts of q, k and v as
        # well: a layer of other shapes goes the checked way
        key = (_rope_key(rotary_dim, base, cos_sin_table), tuple(q.shape), tuple(k.shape), tuple(v.shape))
        if (txn.launch is None or txn.launch[0] != key or not q.is_contiguous() or not k.is_contiguous()
                or not v.is_contiguous()):
            extra = {} if cos_sin_table is None else {"cos_sin_table": cos_sin_table}
            q_rot, view = self.write_token_layer_fused_cuda(transaction, layer_idx, q, k, v, rotary_dim=rotary_dim,
                                                            base=base, **extra)
            if q_rot.is_contiguous() and q.is_contiguous() and k.is_contiguous() and v.is_contiguous():
                from ._fused_rope_kv_append import _launch_args

                layer = txn.layers - 1
                rdim = q.shape[-1] if rotary_dim is None else rotary_dim
                txn.launch = (key, _launch_args(q, k, v, self.k_cache[layer], self.v_cache[layer], txn.meta.block_ids,
                                                txn.meta.offsets, txn.meta.positions, rdim, float(base), q_rot,
                                                cos_sin_table))
            return q_rot, view
        try:
            layer_idx = self._validate_layer_idx(layer_idx)
            if layer_idx != txn.layers:
                raise RuntimeError(f"transaction requires layer {txn.layers}, got layer {layer_idx}")
            q_out = torch.empty_like(q)
            args = txn.launch[1]
            args.q_out = q_out.data_ptr()
            args.q = q.data_ptr()
            args.k = k.data_ptr()
            args.v = v.data_ptr()
            args.k_cache = self.k_cache.data_ptr() + layer_idx * self.k_cache.stride(0) * self.k_cache.element_size()
            args.v_cache = self.v_cache.data_ptr() + layer_idx * self.v_cache.stride(0) * self.v_cache.element_size()
            _lib.rope_append(args, _lib.current_stream_handle(q.device), rotate=True)
        except Exception:
            self._tally.failures += 1
            raise
        return q_out, self._layer_written(txn)

    def _layer_in_fused_decode(self, transaction, layer_idx, rotary_dim, base, cos_sin_table):
        """Bookkeeping of one layer whose RoPE + K/V write runs inside the decode launch
        (``DecodeEngine.step_layer``).  Only after an earlier layer of the transaction went
        the checked way (``_write_layer_fused_prepared``) with the same RoPE setting: then
        the layer order is all there is left to check.  Returns the view, or None (nothing
        recorded) without such a layer."""
        txn = self._journal.find_open(transaction)
        if txn.launch is None or txn.launch[0][0] != _rope_key(rotary_dim, base, cos_sin_table):
            return None
        try:
            layer_idx = self._validate_layer_idx(layer_idx)
            if layer_idx != txn.layers:
                raise RuntimeError(f"transaction requires layer {txn.layers}, got layer {layer_idx}")
        except Exception:
            self._tally.failures += 1
            raise
        return self._layer_written(txn)

    def _record_graph_layers(self, transaction):
        """Record every layer as written by a replayed step graph (see DecodeEngine.step_graph)."""
        txn = self._journal.find_open(transaction)
        if txn.layers != 0:
            raise RuntimeError("a step graph writes every layer; this transaction already wrote some")
        txn.layers = self.num_layers
        self._tally.layer_writes += self.num_layers

    def commit_token(self, transaction):
        """Publish the token after every layer has been written."""
        txn = self._journal.find_open(transaction)
        if txn.layers != self.num_layers:
            raise RuntimeError("cannot commit token before all layers are written")
        view = replace(self._snapshot(txn), state="committed")  # before any change: a failure leaves it open
        for rid in txn.rids:
            seq = self._seqs[rid]
            seq.length += 1
            seq.txn = None
        self._tally.commits += 1
        self._publish()
        self._journal.close(txn, "committed")
        return view

    def abort_token(self, transaction):
        """Abort the open token and return the boundary blocks it reserved."""
        txn = self._journal.find_open(transaction)
        for rid, blk in txn.grown:
            pages = self._seqs[rid].pages
            if not pages or pages[-1] != blk:
                raise RuntimeError("transaction rollback block ownership is inconsistent")
        view = replace(self._snapshot(txn), state="aborted")  # before any change: a failure leaves it open
        self._undo_growth(txn.grown)
        for rid in txn.rids:
            self._seqs[rid].txn = None
        self._tally.aborts += 1
        self._tally.rollback_blocks += len(txn.grown)
        self._publish()
        self._journal.close(txn, "aborted")
        return view

    def transaction_view(self, transaction):
        """Latest detached snapshot of an open transaction."""
        rec = self._journal.find(transaction)
        if isinstance(rec, _Closed):
            raise RuntimeError(f"token transaction is already {rec.phase}")
        return self._snapshot(rec)

    def transaction_device_metadata(self, transaction):
        """The allocator's device-resident metadata of the open transaction.

        Read-only by contract: ``positions``/``block_ids``/``offsets``/``slots``
        (int64), ``eff_lens`` and ``block_tables`` (int32).  For launch paths (e.g.
        graph capture) that must not allocate per layer.
        """
        return self._journal.find_open(transaction).meta

    def _snapshot(self, txn):
        # one device copy per transaction serves every view of it: the
        # metadata is fixed when the transaction opens, and the copy keeps
        # callers away from the allocator's own
        if txn.view_meta is None:
            txn.view_meta = txn.meta.clone()
        meta = txn.view_meta
        return KVTokenTransactionView(
            transaction_id=txn.tid, cache_version=txn.version, request_ids=txn.rids, positions=meta.positions,
            physical_block_ids=meta.block_ids, block_offsets=meta.offsets, block_tables=meta.block_tables,
            effective_seq_lens=meta.eff_lens, next_layer_idx=txn.layers, state=txn.phase)

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
        self._no_transaction("cannot change the metadata arena during an open token transaction")
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
        self._no_transaction("cannot seed context during an open token transaction")
        ids = tuple(self._normalize_request_ids(request_ids))
        if not ids or len(set(ids)) != len(ids):
            raise ValueError("request_ids must be non-empty and unique")
        num_tokens = int(num_tokens)
        if num_tokens <= 0:
            raise ValueError("num_tokens must be positive")
        seqs = [self._active_seq(rid) for rid in ids]
        if (k is None) != (v is None):
            raise ValueError("k and v must be provided together")
        if k is not None:
            shape = (self.num_layers, len(ids), num_tokens, self.num_kv_heads, self.head_dim)
            if tuple(k.shape) != shape or tuple(v.shape) != shape:
                raise ValueError("seed K/V must have shape [num_layers, num_requests, num_tokens, Hkv, D]")
            if k.device != self.device or v.device != self.device or k.dtype != self.dtype or v.dtype != self.dtype:
                raise ValueError("seed K/V must use the cache device and dtype")
        starts = [seq.length for seq in seqs]
        grow = [self._pages_for(p + num_tokens) - self._pages_for(p) for p in starts]
        if sum(grow) > len(self._pool):
            self._tally.capacity_failures += 1
            raise RuntimeError(OUT_OF_BLOCKS)
        # new pages in the order token-by-token appends would take them: at
        # each token index, every request that crosses a block boundary
        for t in range(num_tokens):
            for seq, p in zip(seqs, starts):
                if (p + t) % self.block_size == 0:
                    seq.pages.append(self._pool.take())
        if k is not None:
            for row, (seq, p) in enumerate(zip(seqs, starts)):
                pos = torch.arange(p, p + num_tokens, device=self.device)
                blk = torch.tensor(seq.pages, device=self.device)[pos // self.block_size]
                off = pos % self.block_size
                # non-adjacent advanced indices put the token axis first: [T, L, Hkv, D]
                self.k_cache[:, blk, :, off, :] = k[:, row].permute(1, 0, 2, 3)
                self.v_cache[:, blk, :, off, :] = v[:, row].permute(1, 0, 2, 3)
        for seq in seqs:
            seq.length += num_tokens
        self._publish()
        return self.seq_lens_tensor(ids)

    # -------------------------------------------------------------- queries
    def next_positions(self, request_ids, device=None):
        """Each request's pre-append token position, without mutation."""
        ids = self._normalize_request_ids(request_ids)
        _rows_unique(ids, "request_ids must be unique")
        positions = []
        for rid in ids:
            seq = self._seqs.get(rid)
            if seq is not None and seq.status != self.ACTIVE:
                raise RuntimeError(f"request_id {rid!r} is {seq.status} and cannot accept append")
            if seq is not None and seq.txn is not None:
                raise RuntimeError(f"request_id {rid!r} belongs to an open token transaction")
            positions.append(0 if seq is None else seq.length)
        return _host_to_device(positions, _torch().int64, self.device if device is None else device)

    def block_tables(self, request_ids=None, max_blocks_per_seq=None, pad_value=-1):
        """Padded physical block ids ``[num_requests, max_blocks_per_seq]`` (int32)."""
        seqs = [self._seqs[rid] for rid in self._normalize_active_request_ids(request_ids)]
        width = max(1, max((len(seq.pages) for seq in seqs), default=0)) if max_blocks_per_seq is None \
            else int(max_blocks_per_seq)
        if width <= 0:
            raise ValueError("max_blocks_per_seq must be positive")
        if any(len(seq.pages) > width for seq in seqs):
            raise ValueError("max_blocks_per_seq is smaller than a request's block count")
        return _host_to_device(self._table_rows(seqs, width, int(pad_value)), _torch().int32, self.device)

    def seq_lens_tensor(self, request_ids=None, device=None):
        """Sequence lengths (int32) for the requested rows."""
        lens = [self._seqs[rid].length for rid in self._normalize_active_request_ids(request_ids)]
        return _host_to_device(lens, _torch().int32, self.device if device is None else device)

    def request_block_ids(self, request_id):
        """Logical-to-physical block list of one request."""
        return tuple(self._seq(request_id).pages)

    def to_dense(self, layer_idx=0, request_ids=None, max_seq_len=None):
        """Materialise ``(k_dense, v_dense, seq_lens)`` with K/V ``[B, L, Hkv, D]``."""
        torch = _torch()
        layer_idx = self._validate_layer_idx(layer_idx)
        ids = self._normalize_active_request_ids(request_ids)
        longest = max((self._seqs[rid].length for rid in ids), default=0)
        max_seq_len = max(1, longest) if max_seq_len is None else int(max_seq_len)
        if max_seq_len < longest:
            raise ValueError("max_seq_len is smaller than an existing request length")
        k_dense = torch.zeros((len(ids), max_seq_len, self.num_kv_heads, self.head_dim), device=self.device,
                              dtype=self.dtype)
        v_dense = torch.zeros_like(k_dense)
        for row, rid in enumerate(ids):
            seq = self._seqs[rid]
            if not seq.length:
                continue
            index = torch.tensor(seq.pages, device=self.device, dtype=torch.long)
            for dense, pool in ((k_dense, self.k_cache), (v_dense, self.v_cache)):
                tokens = pool[layer_idx].index_select(0, index).permute(0, 2, 1, 3)
                dense[row, : seq.length] = tokens.reshape(-1, self.num_kv_heads, self.head_dim)[: seq.length]
        return k_dense, v_dense, self.seq_lens_tensor(ids)

    @property
    def num_free_blocks(self):
        return len(self._pool)

    @property
    def num_used_blocks(self):
        return self.max_blocks - len(self._pool)

    @property
    def state_version(self):
        return self._version

    @property
    def has_open_transaction(self):
        return self._journal.open is not None

    def metrics(self):
        """Block-pool, fragmentation, lifecycle, transaction and prefix counters (45 keys)."""
        pool, tally, book, txn = self._pool, self._tally, self._prefix_book, self._journal.open
        seqs = list(self._seqs.values())
        live = [seq for seq in seqs if seq.status == self.ACTIVE]
        by_status = {s: sum(seq.status == s for seq in seqs) for s in (self.ACTIVE, self.FINISHED, self.CANCELLED)}
        used = self.num_used_blocks
        entries = list(book.entries.values())
        resident = book.resident_blocks()
        block_bytes = (self.num_layers * 2 * self.num_kv_heads * self.block_size * self.head_dim
                       * self.k_cache.element_size())
        reserving = len(txn.grown) if txn is not None else 0
        reserved_tokens = used * self.block_size
        data_tokens = resident * self.block_size + sum(
            max(0, seq.length - seq.shared * self.block_size) for seq in live)
        frag = reserved_tokens - data_tokens
        saved = sum(max(0, e.refs - 1) * len(e.pages) for e in entries)
        lookups = tally.prefix_hits + tally.prefix_misses
        return {
            "max_blocks": self.max_blocks,
            "used_blocks": used,
            "free_blocks": len(pool),
            "block_utilization": used / self.max_blocks,
            "active_tokens": sum(seq.length for seq in live),
            "physical_data_tokens": data_tokens,
            "reserved_tokens": reserved_tokens,
            "internal_fragmentation_tokens": frag,
            "internal_fragmentation_ratio": frag / reserved_tokens if reserved_tokens else 0.0,
            "allocation_count": pool.taken,
            "fresh_allocation_count": pool.fresh,
            "free_count": pool.released,
            "reuse_count": pool.reused,
            "capacity_failure_count": tally.capacity_failures,
            "active_requests": by_status[self.ACTIVE],
            "finished_requests": by_status[self.FINISHED],
            "cancelled_requests": by_status[self.CANCELLED],
            "transaction_begin_count": tally.begins,
            "transaction_commit_count": tally.commits,
            "transaction_abort_count": tally.aborts,
            "open_transaction_count": int(txn is not None),
            "retained_transaction_state_count": int(txn is not None),
            "terminal_transaction_history_count": len(self._journal.history),
            "terminal_transaction_history_limit": self._journal.limit,
            "pending_request_count": len(txn.rids) if txn is not None else 0,
            "reserved_transaction_blocks": reserving,
            "transaction_layer_write_count": tally.layer_writes,
            "transaction_rollback_block_count": tally.rollback_blocks,
            "transaction_failure_count": tally.failures,
            "bytes_per_block": block_bytes,
            "allocated_kv_bytes": used * block_bytes,
            "reserved_transaction_bytes": reserving * block_bytes,
            "prefix_cache_capacity_blocks": self.prefix_cache_capacity_blocks,
            "resident_prefix_count": len(entries),
            "resident_prefix_blocks": resident,
            "active_prefix_references": sum(e.refs for e in entries),
            "shared_prefix_blocks": sum(len(e.pages) for e in entries if e.refs >= 2),
            "saved_prefix_blocks": saved,
            "saved_prefix_bytes": saved * block_bytes,
            "prefix_registration_count": tally.prefix_registrations,
            "prefix_hit_count": tally.prefix_hits,
            "prefix_miss_count": tally.prefix_misses,
            "prefix_hit_ratio": tally.prefix_hits / lookups if lookups else 0.0,
            "prefix_eviction_count": tally.prefix_evictions,
            "prefix_capacity_failure_count": tally.prefix_capacity_failures,
        }

    def validate_invariants(self):
        """Raise RuntimeError if ownership, free list and transactions disagree."""
        for ok, message in self._invariant_rules():
            if not ok():
                raise RuntimeError(message)
        return True

    def _invariant_rules(self):
        """(check, message) in the order they are reported; each check is lazy
        and may rely on the ones before it having passed."""
        free = list(self._pool.free)
        book = self._prefix_book.entries
        seqs = list(self._seqs.values())
        live = [seq for seq in seqs if seq.status == self.ACTIVE]
        closed = [seq for seq in seqs if seq.status != self.ACTIVE]
        attached = [seq for seq in live if seq.prefix is not None]
        prefix_pages = [blk for e in book.values() for blk in e.pages]
        private = [blk for seq in live for blk in seq.private_pages()]
        txn, history = self._journal.open, self._journal.history
        hist_ids = tuple(history)

        def each(items, pred):
            return lambda: all(pred(x) for x in items)

        def refs_match():
            want = {pid: 0 for pid in book}
            for seq in attached:
                want[seq.prefix] += 1
            return all(e.refs == want[pid] for pid, e in book.items())

        def txn_rows():
            for rid in txn.rids:
                self._active_seq(rid)  # raises as a lookup of that request would
            return True

        rules = [
            (lambda: len(free) == len(set(free)), "PagedKVCache free list contains duplicate blocks"),
            (each(book.values(), lambda e: len(e.pages) > 0), "resident prefix must own at least one block"),
            (each(book.values(), lambda e: e.refs >= 0), "prefix active_refcount must be non-negative"),
            (lambda: len(prefix_pages) == len(set(prefix_pages)), "a physical block belongs to multiple prefixes"),
            (lambda: len(prefix_pages) <= self.prefix_cache_capacity_blocks,
             "resident prefixes exceed configured prefix capacity"),
            (each(live, lambda s: len(s.pages) == self._pages_for(s.length + (s.txn is not None))),
             "active request block count does not match seq_len"),
            (each(live, lambda s: s.prefix is not None or not s.shared), "request without prefix has shared blocks"),
            (each(attached, lambda s: s.prefix in book), "request references a non-resident prefix"),
            (each(attached, lambda s: s.shared == len(book[s.prefix].pages)),
             "request shared block count does not match prefix"),
            (each(attached, lambda s: tuple(s.pages[: s.shared]) == book[s.prefix].pages),
             "request shared block ids do not match prefix"),
            (each(attached, lambda s: s.length >= s.shared * self.block_size),
             "request seq_len is shorter than its shared prefix"),
            (each(closed, lambda s: not s.pages), "terminal request still owns physical blocks"),
            (each(closed, lambda s: s.txn is None), "terminal request belongs to a token transaction"),
            (each(closed, lambda s: s.prefix is None and not s.shared),
             "terminal request still references a shared prefix"),
            (refs_match, "prefix active_refcount does not match attached requests"),
            (lambda: len(private) == len(set(private)), "a private physical block is owned by multiple requests"),
            (lambda: not set(private) & set(prefix_pages), "a physical block is both private and prefix-owned"),
            (lambda: not set(private + prefix_pages) & set(free), "a physical block is both owned and free"),
            (lambda: set(private + prefix_pages) | set(free) == set(range(self.max_blocks)),
             "physical block accounting does not cover the cache"),
            (lambda: txn is None or txn.phase == "open", "terminal transaction retained device-backed state"),
            (lambda: self._journal.limit >= 0, "terminal transaction history limit is negative"),
            (lambda: len(history) <= self._journal.limit, "terminal transaction history exceeds its limit"),
            (lambda: txn is None or txn.tid not in history, "transaction appears in both open and terminal state"),
            (each(history.values(), lambda c: c.phase in ("committed", "aborted")),
             "terminal transaction history contains an open state"),
            (each(history.items(), lambda kv: kv[0] == kv[1].tid), "terminal transaction history key does not match its state"),
            (each(hist_ids, lambda tid: 0 < tid < self._journal.next_id),
             "terminal transaction history contains an invalid id"),
            (each(history.values(), lambda c: 0 < c.version <= self._version),
             "terminal transaction history contains an invalid version"),
            (lambda: hist_ids == tuple(sorted(hist_ids)), "terminal transaction history is not ordered by id"),
            (lambda: txn is not None or all(s.txn is None for s in seqs),
             "request has an in-flight marker without an open transaction"),
        ]
        if txn is not None:
            rules += [
                (lambda: 0 <= txn.layers <= self.num_layers, "transaction next layer is out of range"),
                (txn_rows, "request_id is not active"),
                (lambda: all(self._seqs[rid].txn == txn.tid for rid in txn.rids),
                 "request transaction marker does not match"),
                (lambda: all(self._seqs[rid].length == pos for rid, pos in zip(txn.rids, txn.positions)),
                 "transaction position is not the committed seq_len"),
                (lambda: all(slot == (self._seqs[rid].pages[pos // self.block_size], pos % self.block_size)
                             for rid, pos, slot in zip(txn.rids, txn.positions, txn.slots)),
                 "transaction physical location does not match ownership"),
            ]
        return rules

    # ------------------------------------------------------------ internals
    @staticmethod
    def _table_rows(seqs, width, pad=-1):
        rows = np.full((len(seqs), width), pad, dtype=np.int32)
        for i, seq in enumerate(seqs):
            rows[i, : len(seq.pages)] = seq.pages
        return rows

    def _slot_tensors(self, slots):
        both = np.ascontiguousarray(np.asarray(slots, dtype=np.int64).reshape(-1, 2).T)
        both = _host_to_device(both, _torch().int64, self.device)
        return both[0], both[1]

    def _validate_layer_idx(self, layer_idx):
        layer_idx = int(layer_idx)
        if not 0 <= layer_idx < self.num_layers:
            raise ValueError("layer_idx must be in [0, num_layers)")
        return layer_idx

    def _normalize_request_ids(self, request_ids):
        torch = _torch()
        if isinstance(request_ids, torch.Tensor):
            ids = [int(x) for x in request_ids.detach().cpu().reshape(-1).tolist()]
        elif isinstance(request_ids, (str, bytes)):
            ids = [request_ids]
        else:
            try:
                ids = list(request_ids)
            except TypeError:
                ids = [request_ids]
        for rid in ids:
            _require_hashable(rid)
        return ids

    def _normalize_active_request_ids(self, request_ids):
        if request_ids is None:
            return [rid for rid, seq in self._seqs.items() if seq.status == self.ACTIVE]
        ids = self._normalize_request_ids(request_ids)
        for rid in ids:
            self._active_seq(rid)
        return ids
