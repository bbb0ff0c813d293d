"""Decode engine: request lifecycle, RoPE/KV append and paged decode per layer.

Mirrors cysong2025/flashdec ``flashdec/engine.py``: result/handle types
(:21-68), lifecycle (``add_request``/``admit``/``finish_request``/
``cancel_request``), the multi-layer token transaction
(``begin_step``/``step_layer``/``commit_step``/``abort_step``, :594-752) with
automatic abort on any layer error (:709-711, 1117-1126), the single-layer
``step`` with its backpressure result (:754-871), ``metrics`` and
``validate_invariants``.  The scheduler-managed mode (:200-573) is policy,
not this data path, and is not provided.

Backends.  ``append_backend``: ``"fused_hip"`` (alias ``"fused_cuda"``: one
HIP kernel rotates Q/K and writes K/V), ``"hip"`` (alias ``"cuda"``: torch
RoPE + HIP scatter; single-layer ``step`` only, as in the reference),
``"torch"``.  ``decode_backend``: ``"hip"`` (alias ``"triton"``: the HIP
paged-decode kernels), ``"reference"`` (torch).  Left as ``None`` they
resolve to the HIP backends for a GPU-resident cache and to the torch
backends for a CPU-resident cache (the only ones that can run there); the
HIP backends never fall back -- they raise if the library is missing.

Per layer on the HIP path the engine launches the fused RoPE + append kernel
and the decode kernel(s) on torch's current stream, reading the
transaction's device-resident metadata (one H2D copy per ``begin_step``), and
performs no host synchronisation.
"""

from __future__ import annotations

import contextlib
from dataclasses import dataclass
from typing import Any, Hashable

import numpy as np

PROFILE_RANGE_PREFLIGHT = "flashdec::engine_preflight"
PROFILE_RANGE_APPEND = "flashdec::rope_kv_append"
PROFILE_RANGE_DECODE = "flashdec::paged_decode"

_APPEND_ALIASES = {"torch": "torch", "cuda": "hip", "hip": "hip", "fused_cuda": "fused_hip", "fused_hip": "fused_hip"}
_DECODE_ALIASES = {"reference": "reference", "triton": "hip", "hip": "hip"}


def _torch():
    import torch

    return torch


@dataclass(frozen=True)
class AdmissionResult:
    """State transition result for a request submitted to the engine."""

    request_id: Hashable
    status: str


@dataclass(frozen=True)
class DecodeStepResult:
    """One decode-step result, or an explicit backpressure response."""

    status: str
    request_ids: tuple
    output: Any | None
    positions: Any | None
    block_tables: Any | None
    seq_lens: Any | None
    needed_new_blocks: int
    free_blocks: int
    reason: str | None = None


@dataclass(frozen=True)
class DecodeStepTransaction:
    """Stable engine handle for one open multi-layer token transaction."""

    transaction_id: int
    engine_version: int
    request_ids: tuple
    positions: Any
    physical_block_ids: Any
    block_offsets: Any
    block_tables: Any
    effective_seq_lens: Any


@dataclass(frozen=True)
class DecodeLayerResult:
    """Output of one layer inside an open decode token transaction."""

    transaction_id: int
    layer_idx: int
    request_ids: tuple
    output: Any
    positions: Any
    block_tables: Any
    effective_seq_lens: Any


@dataclass(frozen=True)
class DecodeStepGraph:
    """A captured hipGraph of one whole token step for a fixed batch size.

    Replaying it runs, for every layer in order, the fused RoPE + K/V append
    (``q[l]``, ``k[l]``, ``v[l]`` -> the reserved slots, ``q_rot[l]``) and the
    paged decode (``q_rot[l]`` -> ``out[l]``), reading the open
    transaction's metadata from the cache's graph-metadata arena.  With
    ``fused_rope`` the two are one launch per layer: the decode kernel rotates
    q and the new K itself, stores K/V to the slots and leaves ``q_rot``
    untouched (same outputs and cache bytes).  The caller writes
    ``q``/``k``/``v`` ``[num_layers, B, H, D]`` before each replay; ``out``
    holds every layer's attention output afterwards.
    """

    graph: Any
    batch_size: int
    q: Any
    k: Any
    v: Any
    q_rot: Any
    out: Any
    num_splits: int
    rotary_dim: int
    base: float
    metadata: Any
    workspace: Any = None  # split partials (and merge counters) the graph uses, kept alive with it
    balance_target: int = 0  # > 0: per-row split counts from the lengths at replay
    kv_reuse: bool = False  # rows shared prefix blocks at capture: plain (cached) K/V loads
    fused_rope: bool = False  # RoPE + append inside the decode launch (q_rot unused)
    cascade: Any = None  # _GraphCascade: shared-prefix decode with per-replay group tables
    cos_sin_table: Any = None  # RoPE cos/sin table every launch reads (None: evaluated in the kernels)


@dataclass
class _GraphCascade:
    """Group tables a cascade step graph reads at every replay.

    The launch grid is fixed at capture for ``num_groups`` groups of at most
    ``max_members`` rows; ``step_graph`` writes each step's groups (unused
    slots -1 / 0) into ``buf`` before the replay, through a pinned staging ring.
    """

    groups: Any  # CascadeGroups whose tensors are views of buf
    buf: Any
    num_groups: int
    max_members: int
    staging: Any
    chunk_rows: int = 16  # group rows per prefix-role workgroup, fixed at capture


@dataclass
class _OpenStep:
    handle: DecodeStepTransaction
    cache_transaction: Any
    needed_new_blocks: int
    next_layer_idx: int = 0
    last_output: Any | None = None
    state: str = "open"
    ragged: bool = False  # the batch's lengths vary widely: per-row split counts
    cascade: Any = None  # CascadeGroups: rows sharing a resident prefix decode it once per group
    kv_reuse: bool = False  # rows share prefix blocks (per-row path): plain, cached K/V loads
    decode_launch: Any = None  # eager HIP decode: ((stream, q shape, q strides), PagedDecodeArgs) of this step
    fused_launch: Any = None  # eager decode with RoPE + append inside the launch: (RoPE key, PagedDecodeArgs)


class _Roster:
    """The engine's request statuses, in submission order."""

    __slots__ = ("status",)

    def __init__(self):
        self.status: dict = {}

    def __bool__(self):
        return bool(self.status)

    def submit(self, request_id, status):
        _require_hashable(request_id)
        if request_id in self.status:
            raise RuntimeError(f"request_id {request_id!r} already exists in the DecodeEngine")
        self.status[request_id] = status

    def of(self, request_id):
        _require_hashable(request_id)
        if request_id not in self.status:
            raise KeyError(f"unknown request_id: {request_id!r}")
        return self.status[request_id]

    def expect(self, request_id, wanted):
        have = self.of(request_id)
        if have != wanted:
            raise RuntimeError(f"request_id {request_id!r} is {have}, expected {wanted}")

    def having(self, wanted):
        return tuple(rid for rid, st in self.status.items() if st == wanted)


class _EngineCounts:
    """Engine event counters reported by ``DecodeEngine.metrics``."""

    __slots__ = ("steps", "tokens", "backpressure", "layer_steps", "aborts")

    def __init__(self):
        self.steps = self.tokens = self.backpressure = self.layer_steps = self.aborts = 0


def _require_hashable(request_id):
    try:
        hash(request_id)
    except TypeError as exc:
        raise ValueError("request ids must be hashable") from exc


def _as_id_tuple(request_ids):
    """One id (a string, bytes or any non-iterable) or an iterable of ids, as a tuple."""
    if isinstance(request_ids, (str, bytes)):
        return (request_ids,)
    try:
        return tuple(request_ids)
    except TypeError:
        return (request_ids,)


def _step_input_rules(engine, ids, q, k, v):
    """(broken?, exception, message) of one step's q/k/v, in the order they are reported."""
    torch = _torch()
    cache = engine.cache
    rows = (len(ids), cache.num_kv_heads, cache.head_dim)
    return (
        (lambda: not all(isinstance(t, torch.Tensor) for t in (q, k, v)), TypeError,
         "q, k, and v must be torch tensors"),
        (lambda: q.dim() != 3, ValueError, "q must have shape [num_requests, num_q_heads, head_dim]"),
        (lambda: q.shape[0] != len(ids) or q.shape[1] <= 0 or q.shape[2] != cache.head_dim, ValueError,
         "q shape must match active request count and cache head_dim"),
        (lambda: k.shape != rows or v.shape != rows, ValueError,
         "k and v shapes must match active request count and cache dimensions"),
        (lambda: any(t.device != cache.device for t in (q, k, v)), ValueError, "q, k, and v must be on the cache device"),
        (lambda: any(t.dtype != cache.dtype for t in (q, k, v)), ValueError, "q, k, and v must use the cache dtype"),
    )


_NO_RANGE = contextlib.nullcontext()  # reusable: a phase without a profiler range


def _own_method(obj, name):
    """``obj.name`` is its class's own method, not one replaced on the instance."""
    return getattr(getattr(obj, name, None), "__func__", None) is getattr(type(obj), name, None)


def _is_ragged(lengths):
    """A batch whose longest row is over twice its mean length."""
    if not lengths:
        return False
    return max(lengths) * len(lengths) > 2 * max(1, sum(lengths))


class DecodeEngine:
    """Coordinate request lifecycle, RoPE/KV append and paged decode."""

    WAITING = "waiting"
    ACTIVE = "active"
    FINISHED = "finished"
    CANCELLED = "cancelled"
    REJECTED = "rejected"

    STEP_OK = "ok"
    STEP_BACKPRESSURE = "backpressure"

    def __init__(self, cache, append_backend=None, decode_backend=None, sm_scale=None, num_warps=2, num_stages=None,
                 profile_ranges=False):
        from .cache import PagedKVCache

        if not isinstance(cache, PagedKVCache):
            raise TypeError("cache must be a PagedKVCache")
        on_gpu = cache.device.type == "cuda"
        if append_backend is None:
            append_backend = "fused_hip" if on_gpu else "torch"
        if decode_backend is None:
            decode_backend = "hip" if on_gpu else "reference"
        if append_backend not in _APPEND_ALIASES:
            raise ValueError("append_backend must be 'torch', 'cuda', or 'fused_cuda'")
        if decode_backend not in _DECODE_ALIASES:
            raise ValueError("decode_backend must be 'reference' or 'triton'")
        if not isinstance(profile_ranges, bool):
            raise ValueError("profile_ranges must be a bool")
        self.cache = cache
        self.append_backend = append_backend
        self.decode_backend = decode_backend
        self._append = _APPEND_ALIASES[append_backend]
        self._decode_kind = _DECODE_ALIASES[decode_backend]
        self.sm_scale = sm_scale
        self.num_warps = num_warps
        self.num_stages = num_stages
        self.profile_ranges = profile_ranges
        # eager steps: layers after the first run RoPE + K/V write inside the
        # decode launch where it applies (no counterpart in the reference; the
        # bits are those of the two launches, and False keeps two)
        self.eager_fuse_rope = True
        self._range = _torch().profiler.record_function if profile_ranges else None
        self._roster = _Roster()
        self._counts = _EngineCounts()
        self._version = 0
        self._cache_seen = cache.state_version  # the cache version this engine last left it at
        self._open: _OpenStep | None = None
        # Eager steps decode rows attached to one resident prefix with the
        # shared-prefix (cascade) launch once a group's sharers x prefix tokens
        # reach this many (None: never).  On MI355X the cascade takes 13.2 us
        # against 14.4 per row at 16 x 4096 and 18.6 against 32.8 at 32 x 8192.
        self.cascade_min_shared_tokens = 64 * 1024
        self._cascade_cache = None
        self._cascade_decode_count = 0

    # ------------------------------------------------------------ lifecycle
    def _advanced(self, cache_changed=True):
        """One engine state change; ``cache_changed``: it went through the cache,
        whose new version is then the one this engine expects to find."""
        if cache_changed:
            self._cache_seen = self.cache.state_version
        self._version += 1

    def register_prefix(self, prefix_id, k_blocks, v_blocks):
        """Register shared full blocks before any request enters the engine."""
        self._require_no_open_step("register a shared prefix")
        for broken, message in (
                (lambda: bool(self._roster), "shared prefixes must be registered before request submission"),
                (lambda: self.cache.state_version != self._cache_seen, "PagedKVCache mutated outside DecodeEngine"),
                (lambda: any(self.cache.metrics()[f"{st}_requests"] for st in ("active", "finished", "cancelled")),
                 "shared prefix registration requires an empty PagedKVCache")):
            if broken():
                raise RuntimeError(message)
        result = self.cache.register_prefix(prefix_id, k_blocks, v_blocks)
        self._cache_seen = self.cache.state_version  # no engine state changed
        return result

    def evict_prefix(self, prefix_id):
        """Evict one inactive prefix after every request is resolved."""
        self._require_no_open_step("evict a shared prefix")
        if self._roster.having(self.WAITING) or self._roster.having(self.ACTIVE):
            raise RuntimeError("shared prefixes can only be evicted after all requests are resolved")
        released = self.cache.evict_prefix(prefix_id)
        self._advanced()
        return released

    def add_request(self, request_id):
        """Submit a request in ``waiting`` state (no KV memory yet)."""
        self._require_no_open_step("submit a request")
        self._roster.submit(request_id, self.WAITING)
        self._advanced(cache_changed=False)
        return AdmissionResult(request_id=request_id, status=self.WAITING)

    def admit(self, request_ids=None, prefix_id=None):
        """Move waiting requests to ``active``; optionally attach a resident shared prefix."""
        self._require_no_open_step("admit requests")
        ids = self._roster.having(self.WAITING) if request_ids is None else self._normalize_ids(request_ids)
        if not ids:
            raise ValueError("at least one waiting request is required for admission")
        for rid in ids:
            self._roster.expect(rid, self.WAITING)
        for rid in ids:  # each row enters the cache (and its prefix) before the next
            self.cache.add_request(rid)
            if prefix_id is not None:
                self.cache.attach_prefix(rid, prefix_id)
            self._roster.status[rid] = self.ACTIVE
        self._advanced()
        return tuple(AdmissionResult(request_id=rid, status=self.ACTIVE) for rid in ids)

    @property
    def state_version(self):
        return self._version

    def active_request_ids(self):
        """Active request ids in admission order."""
        return self._roster.having(self.ACTIVE)

    def request_state(self, request_id):
        status = self._roster.of(request_id)
        state = {"request_id": request_id, "status": status}
        if status in (self.ACTIVE, self.FINISHED, self.CANCELLED):  # the rows the cache knows
            state["cache"] = self.cache.request_state(request_id)
        return state

    # terminal outcome -> (action named in the open-step error, cache method)
    _RESOLUTIONS = {FINISHED: ("finish a request", "finish_request"),
                    CANCELLED: ("cancel a request", "cancel_request")}

    def _resolve(self, request_id, outcome):
        action, method = self._RESOLUTIONS[outcome]
        self._require_no_open_step(action)
        self._roster.expect(request_id, self.ACTIVE)
        released = getattr(self.cache, method)(request_id)
        self._roster.status[request_id] = outcome
        self._advanced()
        return released

    def finish_request(self, request_id):
        """Finish an active request and release its blocks."""
        return self._resolve(request_id, self.FINISHED)

    def cancel_request(self, request_id):
        """Cancel an active request and release its blocks."""
        return self._resolve(request_id, self.CANCELLED)

    # ---------------------------------------------------- token transaction
    def begin_step(self, request_ids=None):
        """Open one token transaction for a stable batch of active requests."""
        self._require_no_open_step("begin another decode step")
        if self._append not in ("torch", "fused_hip"):
            raise RuntimeError("multi-layer transactions require append_backend='torch' or 'fused_cuda'")
        ids = self._normalize_active_ids(request_ids)
        needed = self._needed_new_blocks(ids)
        if needed > self.cache.num_free_blocks:
            self._counts.backpressure += 1
            raise RuntimeError("insufficient physical blocks to begin decode step")
        tx = self.cache.begin_token(ids)
        self._advanced()
        handle = DecodeStepTransaction(
            transaction_id=tx.transaction_id, engine_version=self._version, request_ids=ids, positions=tx.positions,
            physical_block_ids=tx.physical_block_ids, block_offsets=tx.block_offsets, block_tables=tx.block_tables,
            effective_seq_lens=tx.effective_seq_lens)
        # decode planning for this batch, from host state
        lengths = self.cache._host_seq_lens(ids)
        groups = self.cache._prefix_groups(ids)
        cascade = self._step_cascade(ids, lengths, groups)
        self._open = _OpenStep(handle=handle, cache_transaction=tx, needed_new_blocks=needed,
                               ragged=_is_ragged(lengths), cascade=cascade,
                               kv_reuse=bool(groups) and cascade is None)
        return handle

    def _cascade_pays(self, groups):
        """Whether a batch with these prefix groups should decode them with the cascade."""
        if self._decode_kind != "hip" or self.cache.device.type != "cuda" or self.cascade_min_shared_tokens is None:
            return False
        bs = self.cache.block_size
        return bool(groups) and max(len(rows) * blocks * bs for rows, blocks in groups) >= self.cascade_min_shared_tokens

    def _write_graph_cascade(self, ids, gc):
        """Pack this step's prefix groups into the cascade graph's tables (one async copy)."""
        groups = self.cache._prefix_groups(ids)
        if len(groups) > gc.num_groups or any(len(rows) > gc.max_members for rows, _ in groups):
            raise RuntimeError(f"the step's prefix groups exceed the cascade step graph's capacity ({gc.num_groups} "
                               f"groups of {gc.max_members} rows)")
        bs = self.cache.block_size
        ng, mm = gc.num_groups, gc.max_members
        slot, host = gc.staging.acquire()
        arr = host.numpy().view(np.int32)
        members = arr[: ng * mm].reshape(ng, mm)
        members.fill(-1)
        arr[ng * mm:] = 0
        for g, (rows, blocks) in enumerate(groups):
            members[g, : len(rows)] = rows
            arr[ng * mm + g] = blocks * bs
            arr[ng * mm + ng + np.asarray(rows)] = blocks * bs
        gc.buf.copy_(host.view(_torch().int32)[: gc.buf.numel()], non_blocking=True)
        gc.staging.release(slot)

    def _step_cascade(self, ids, lengths, groups):
        """Prefix groups of this step's batch when the shared-prefix decode pays
        (the eager HIP path), else None.  Device tensors are kept per batch
        composition; only the planning figures follow the lengths."""
        if not self._cascade_pays(groups):
            return None
        bs = self.cache.block_size
        import dataclasses

        from .cascade import CascadeGroups

        key = (tuple(ids), tuple((tuple(rows), blocks) for rows, blocks in groups))
        if self._cascade_cache is None or self._cascade_cache[0] != key:
            torch = _torch()
            width = max(len(rows) for rows, _ in groups)
            members = torch.full((len(groups), width), -1, dtype=torch.int32)
            prefix = torch.zeros(len(groups), dtype=torch.int32)
            row_prefix = torch.zeros(len(ids), dtype=torch.int32)
            for g, (rows, blocks) in enumerate(groups):
                members[g, : len(rows)] = torch.tensor(rows, dtype=torch.int32)
                prefix[g] = blocks * bs
                row_prefix[rows] = blocks * bs
            dev = self.cache.device
            self._cascade_cache = (key, CascadeGroups(members=members.to(dev), prefix_len=prefix.to(dev),
                                                      row_prefix_len=row_prefix.to(dev),
                                                      max_prefix_len=int(prefix.max()), max_tail_len=0,
                                                      total_tail_len=0), row_prefix.tolist())
        _, cached, row_prefix = self._cascade_cache
        tails = [max(0, n + 1 - p) for n, p in zip(lengths, row_prefix)]  # the new token included
        return dataclasses.replace(cached, max_tail_len=max(tails), total_tail_len=sum(tails))

    def step_layer(self, transaction, layer_idx, q, k, v, *, rotary_dim=None, base=10_000.0, cos_sin_table=None):
        """RoPE + KV write + paged decode for one layer; any error aborts the whole token.

        ``cos_sin_table`` (HIP append backend; no counterpart in the reference):
        a :func:`flashdec_amd.rope.rope_cos_sin_table` covering the step's
        positions (checked on the host; a short table raises ``ValueError``
        and aborts the step).  By default the cache's own table
        (``PagedKVCache.rope_table``): either way q and the appended K are
        rotated exactly as :func:`flashdec_amd.rope.apply_rope` rotates them
        on this device.
        """
        state = self._require_open_step(transaction)
        try:
            layer_idx = int(layer_idx)
            if layer_idx != state.next_layer_idx:
                raise RuntimeError(f"decode transaction requires layer {state.next_layer_idx}, got layer {layer_idx}")
            ids = state.handle.request_ids
            self._validate_step_inputs(ids, q, k, v)
            k, v = (t.unsqueeze(0) if t.dim() == 2 else t for t in (k, v))
            cos_sin_table = self._step_rope_table(state, rotary_dim, base, cos_sin_table)
            with self._phase(PROFILE_RANGE_APPEND):
                fused = self._fused_layer(state, layer_idx, q, k, v, rotary_dim, base, cos_sin_table)
                if fused is None:
                    q_rot, view, meta = self._write_layer(state, layer_idx, q, k, v, rotary_dim, base,
                                                          cos_sin_table)
                else:
                    view, meta = fused
            with self._phase(PROFILE_RANGE_DECODE):
                if fused is None:
                    output = self._decode_layer(q_rot, view, meta, layer_idx)
                else:
                    output = self._decode_fused_layer(state, q, k, v, meta, layer_idx, rotary_dim, base,
                                                      cos_sin_table)
        except Exception:
            self._close_step(state, "aborted")
            raise
        state.next_layer_idx += 1
        state.last_output = output
        self._counts.layer_steps += 1
        return DecodeLayerResult(transaction_id=state.handle.transaction_id, layer_idx=layer_idx,
                                 request_ids=state.handle.request_ids, output=output, positions=view.positions,
                                 block_tables=view.block_tables, effective_seq_lens=view.effective_seq_lens)

    def _step_rope_table(self, state, rotary_dim, base, cos_sin_table):
        """The cos/sin table this layer's HIP RoPE launches read: the caller's, checked to
        cover the step's positions, else the cache's own (None where the kernels evaluate
        cos/sin themselves: ``rope_tables`` off, other append backends, caches without
        tables)."""
        cache = self.cache
        launch_table = getattr(cache, "_launch_table", None)
        if (self._append != "fused_hip" or launch_table is None or not _own_method(cache, "_launch_table")
                or not _own_method(cache, "write_token_layer_fused_cuda")):
            return cos_sin_table  # a replaced fused write keeps the reference's signature
        from .cache import _rotary_dim_and_base

        rdim, rbase = _rotary_dim_and_base(cache.head_dim, rotary_dim, base)
        return launch_table(cos_sin_table, rdim, rbase, cache._txn_max_position(state.cache_transaction))

    def _phase(self, name):
        """A profiler range around one phase when ``profile_ranges`` is on."""
        return self._range(name) if self._range is not None else _NO_RANGE

    def commit_step(self, transaction):
        """Commit the open token after every layer has run."""
        state = self._require_open_step(transaction)
        if state.next_layer_idx != self.cache.num_layers:
            raise RuntimeError("cannot commit decode step before all layers are complete")
        committed = self._close_step(state, "committed")
        # the committed lengths are the token's effective lengths, already on the
        # device: no host-to-device copy per step
        return DecodeStepResult(status=self.STEP_OK, request_ids=state.handle.request_ids, output=state.last_output,
                                positions=committed.positions, block_tables=committed.block_tables,
                                seq_lens=committed.effective_seq_lens, needed_new_blocks=state.needed_new_blocks,
                                free_blocks=self.cache.num_free_blocks)

    def abort_step(self, transaction):
        """Explicitly abort the open token transaction."""
        return self._close_step(self._require_open_step(transaction), "aborted")

    def _close_step(self, state, outcome):
        """Commit or abort the open step in the cache; returns the cache's final view."""
        if self._open is not state or state.state != "open":
            raise RuntimeError("decode step transaction is not open")
        tx = state.cache_transaction
        view = self.cache.commit_token(tx) if outcome == "committed" else self.cache.abort_token(tx)
        state.state = outcome
        self._open = None
        if outcome == "committed":
            self._counts.steps += 1
            self._counts.tokens += len(state.handle.request_ids)
        else:
            self._counts.aborts += 1
        self._advanced()
        return view

    def capture_step_graph(self, batch_size, num_q_heads, *, rotary_dim=None, base=10_000.0, num_splits=None,
                           merge=False, kv_reuse=None, fuse_rope=None, cascade=None, cos_sin_table=None):
        """Capture every layer's launches of one token step into a hipGraph.

        Needs the HIP backends, a GPU cache and its graph-metadata arena
        (``PagedKVCache.enable_graph_metadata``) with room for ``batch_size``
        rows.  Nothing runs at capture time and no allocator state changes;
        input and output buffers are allocated here and returned in the
        :class:`DecodeStepGraph`.  The decode split count is fixed for the
        arena's table width (``num_splits`` overrides it); each row's split
        range follows its own length at replay, so growing sequences stay
        correct.  ``merge=True`` merges the split partials inside the attention
        launch (the last workgroup of each request and KV head), so each layer
        runs two kernels instead of three.  ``kv_reuse`` (default: whether
        active requests share a resident prefix now) reads K/V with plain,
        cached loads instead of streaming them.  ``fuse_rope`` (default: where
        supported -- head_dim 128, rotary_dim 64 or 128, a 16-bit cache, no
        merge and no per-row splits) runs RoPE + append inside each layer's
        decode launch, one kernel fewer per layer.  ``cascade`` (default: when
        active requests share a resident prefix as the eager steps' cascade
        threshold asks) decodes each layer with the shared-prefix launch; the
        group count and size of the active batch at capture bound every later
        step's prefix groups, which each replay reads from the graph's tables.
        ``cos_sin_table``: a :func:`flashdec_amd.rope.rope_cos_sin_table` with a
        row for every position the arena's table width allows; every launch
        then rotates with it (bit-identical to ``apply_rope`` on this device).
        By default the cache's own table (``PagedKVCache.rope_table``, unless
        its ``rope_tables`` is off).
        """
        torch = _torch()
        from . import _lib
        from ._fused_rope_kv_append import _fused_rope_kv_append_trusted
        from .paged_decode import _decode_with_workspace, _validate_inputs

        self._require_no_open_step("capture a step graph")
        cache = self.cache
        if self._append != "fused_hip" or self._decode_kind != "hip":
            raise RuntimeError("step graphs require append_backend='fused_cuda' and decode_backend='triton'")
        if cache.device.type != "cuda":
            raise ValueError("step graphs require a CUDA-resident PagedKVCache")
        batch_size, num_q_heads = int(batch_size), int(num_q_heads)
        if num_q_heads <= 0 or num_q_heads % cache.num_kv_heads:
            raise ValueError("num_q_heads must be a positive multiple of num_kv_heads")
        meta = cache.graph_metadata(batch_size)
        if rotary_dim is None:
            rotary_dim = cache.head_dim
        if cos_sin_table is None and getattr(cache, "rope_tables", False):
            # the cache's own table, with a row for every position the arena's
            # table width allows (the graph keeps a reference to it)
            cos_sin_table = cache.rope_table(int(rotary_dim), base, meta.block_tables.shape[1] * cache.block_size)
        if cos_sin_table is not None:
            from ._fused_rope_kv_append import _check_cos_sin_table

            _check_cos_sin_table(cos_sin_table, int(rotary_dim), cache.device)
            if cos_sin_table.shape[1] < meta.block_tables.shape[1] * cache.block_size:
                raise ValueError("cos_sin_table needs a row for every position of the metadata arena's table width")
        shape_q = (cache.num_layers, batch_size, num_q_heads, cache.head_dim)
        shape_kv = (cache.num_layers, batch_size, cache.num_kv_heads, cache.head_dim)
        dev, dt = cache.device, cache.dtype
        q = torch.zeros(shape_q, device=dev, dtype=dt)
        k = torch.zeros(shape_kv, device=dev, dtype=dt)
        v = torch.zeros(shape_kv, device=dev, dtype=dt)
        q_rot = torch.zeros_like(q)
        out = torch.zeros_like(q)
        width = meta.block_tables.shape[1]
        groups_now = cache._prefix_groups(self.active_request_ids())
        if kv_reuse is None:
            kv_reuse = bool(groups_now)
        kv_reuse = bool(kv_reuse)
        cas_ok = (self._cascade_pays(groups_now) and cache.head_dim == 128 and not merge
                  and num_q_heads // cache.num_kv_heads <= 16 and dt in (torch.bfloat16, torch.float16))
        if cascade is None:
            cascade = cas_ok and not fuse_rope
        elif cascade and (not cas_ok or fuse_rope):
            raise ValueError("cascade needs active requests sharing a resident prefix (at least "
                             "cascade_min_shared_tokens sharer-tokens), head_dim 128, <= 16 query heads per KV "
                             "head, a bf16/fp16 cache, no merge and no fuse_rope")
        cascade = bool(cascade)
        balance = 0
        gc = None
        prefix_splits = 0
        chunk_rows = 16
        if cascade:
            from ._lib import paged_decode_plan
            from .cache import _StagingRing
            from .cascade import (CascadeGroups, _num_cus, plan_cascade_splits, plan_chunk_rows, plan_prefix_splits,
                                  prefix_chunks)

            ng = len(groups_now)
            mm = max(len(rows) for rows, _ in groups_now)
            buf = torch.zeros(ng * mm + ng + batch_size, dtype=torch.int32, device=dev)
            prefix_tokens = [blocks * cache.block_size for _, blocks in groups_now]
            active = cache._host_seq_lens(self.active_request_ids())
            row_prefix = [0] * len(active)
            for (rows, _), plen in zip(groups_now, prefix_tokens):
                for r in rows:
                    row_prefix[r] = plen
            tails = [max(1, n + 1 - pr) for n, pr in zip(active, row_prefix)] or [1]
            groups = CascadeGroups(members=buf[: ng * mm].view(ng, mm), prefix_len=buf[ng * mm: ng * mm + ng],
                                   row_prefix_len=buf[ng * mm + ng:], max_prefix_len=max(prefix_tokens),
                                   max_tail_len=max(tails), total_tail_len=sum(tails))
            gc = _GraphCascade(groups=groups, buf=buf, num_groups=ng, max_members=mm,
                               staging=_StagingRing(buf.numel() * 4))
            chunk_rows = gc.chunk_rows = plan_chunk_rows(groups, num_q_heads, cache.num_kv_heads)
            chunks = prefix_chunks(groups, num_q_heads, cache.num_kv_heads, chunk_rows)
            if num_splits is None:
                prefix_splits, num_splits = plan_cascade_splits(batch_size, num_q_heads, cache.num_kv_heads,
                                                                cache.head_dim, groups, chunks, _num_cus(dev))
            else:
                prefix_splits = plan_prefix_splits(ng, cache.num_kv_heads, chunks, groups.max_prefix_len,
                                                   _num_cus(dev))
        if cascade:
            splits = int(num_splits)
            if splits <= 0:
                raise ValueError("num_splits must be a positive integer")
        elif num_splits is None:
            # the batch's current lengths tell a uniform batch from a ragged one
            active = cache._host_seq_lens(self.active_request_ids())
            longest = max(active, default=0) + 1
            total = sum(active) + len(active) if len(active) == batch_size else 0
            if total and _is_ragged(active):
                balance = _lib.paged_decode_balance_target(batch_size, cache.num_kv_heads)
            if balance:
                # per-row split counts follow the lengths at every replay
                splits = max(2, min(balance, -(-width * cache.block_size // 32)))
            else:
                splits = _lib.paged_decode_plan(batch_size, num_q_heads, cache.num_kv_heads, cache.head_dim,
                                                min(longest, width * cache.block_size) if total else
                                                width * cache.block_size, total)
        else:
            splits = int(num_splits)
            if splits <= 0:
                raise ValueError("num_splits must be a positive integer")
        _validate_inputs(q_rot[0], cache.k_cache[0], cache.v_cache[0], meta.block_tables, meta.eff_lens,
                         cache.block_size, self.num_warps, self.num_stages, "token_major")
        eligible = (cache.head_dim == 128 and int(rotary_dim) in (64, 128) and not merge and not balance
                     and not cascade and dt in (torch.bfloat16, torch.float16)
                     and num_q_heads // cache.num_kv_heads <= 16)
        if fuse_rope is None:
            fuse_rope = eligible
        elif fuse_rope and not eligible:
            raise ValueError("fuse_rope needs head_dim 128, rotary_dim 64 or 128, a bf16/fp16 cache, <= 16 query "
                             "heads per KV head, no merge and uniform splits")
        fuse_rope = bool(fuse_rope)
        workspace = None
        counters = None
        if splits + prefix_splits > 1:
            ws_splits = splits + prefix_splits
            workspace = (torch.empty((batch_size, num_q_heads, ws_splits, cache.head_dim), device=dev),
                         torch.empty((batch_size, num_q_heads, ws_splits), device=dev),
                         torch.empty((batch_size, num_q_heads, ws_splits), device=dev))
            if merge and not balance:
                # arrival counters, zero before the capture; every launch leaves them at zero
                counters = torch.zeros(batch_size * cache.num_kv_heads * _lib.SPLIT_COUNTER_STRIDE, device=dev,
                                       dtype=torch.int32)
                workspace = workspace + (counters,)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            with torch.cuda.graph(graph, stream=side):
                for layer in range(cache.num_layers):
                    if cascade:
                        from .cascade import paged_decode_attention_cascade_into

                        _fused_rope_kv_append_trusted(q[layer], k[layer], v[layer], cache.k_cache[layer],
                                                      cache.v_cache[layer], meta.block_ids, meta.offsets,
                                                      meta.positions, rotary_dim=rotary_dim, base=base,
                                                      q_out=q_rot[layer], cos_sin_table=cos_sin_table)
                        paged_decode_attention_cascade_into(q_rot[layer], cache.k_cache[layer], cache.v_cache[layer],
                                                            meta.block_tables, meta.eff_lens, out[layer],
                                                            gc.groups, sm_scale=self.sm_scale,
                                                            block_size=cache.block_size, num_splits=splits,
                                                            prefix_splits=prefix_splits, workspace=workspace,
                                                            chunk_rows=chunk_rows)
                        continue
                    if fuse_rope:
                        _decode_with_workspace(q[layer], cache.k_cache[layer], cache.v_cache[layer],
                                               meta.block_tables, meta.eff_lens, out[layer], self.sm_scale,
                                               cache.block_size, splits, workspace[:3] if workspace else None,
                                               cache.max_blocks, kv_reuse=kv_reuse,
                                               append=(k[layer], v[layer], meta.slots),
                                               rope=(int(rotary_dim), float(base), cos_sin_table))
                        continue
                    _fused_rope_kv_append_trusted(q[layer], k[layer], v[layer], cache.k_cache[layer],
                                                  cache.v_cache[layer], meta.block_ids, meta.offsets, meta.positions,
                                                  rotary_dim=rotary_dim, base=base, q_out=q_rot[layer],
                                                  cos_sin_table=cos_sin_table)
                    _decode_with_workspace(q_rot[layer], cache.k_cache[layer], cache.v_cache[layer],
                                           meta.block_tables, meta.eff_lens, out[layer], self.sm_scale,
                                           cache.block_size, splits, workspace[:3] if workspace else None,
                                           cache.max_blocks, balance_target=balance, counters=counters,
                                           kv_reuse=kv_reuse)
        torch.cuda.current_stream(dev).wait_stream(side)
        return DecodeStepGraph(graph=graph, batch_size=batch_size, q=q, k=k, v=v, q_rot=q_rot, out=out,
                               num_splits=splits, rotary_dim=int(rotary_dim), base=float(base), metadata=meta,
                               workspace=workspace, balance_target=balance, kv_reuse=kv_reuse,
                               fused_rope=fuse_rope, cascade=gc, cos_sin_table=cos_sin_table)

    def step_graph(self, transaction, step_graph):
        """Run every layer of the open step by replaying ``step_graph``; returns ``out [L, B, Hq, D]``.

        The transaction must be fresh (no layer run yet), its batch the
        graph's size, and its metadata in the cache's arena.  The replay goes
        on the current stream after the transaction's metadata copy.  An
        error aborts the whole token, as in ``step_layer``.
        """
        state = self._require_open_step(transaction)
        try:
            if not isinstance(step_graph, DecodeStepGraph):
                raise TypeError("step_graph must be a DecodeStepGraph")
            if state.next_layer_idx != 0:
                raise RuntimeError("a step graph runs every layer; this step already ran some")
            if len(state.handle.request_ids) != step_graph.batch_size:
                raise ValueError("transaction batch size does not match the step graph")
            meta = self.cache.transaction_device_metadata(state.cache_transaction)
            if meta.buf.data_ptr() != step_graph.metadata.buf.data_ptr():
                raise RuntimeError("transaction metadata is not in the graph metadata arena")
            if step_graph.cascade is not None:
                self._write_graph_cascade(state.handle.request_ids, step_graph.cascade)
            step_graph.graph.replay()
            self.cache._record_graph_layers(state.cache_transaction)
        except Exception:
            self._close_step(state, "aborted")
            raise
        state.next_layer_idx = self.cache.num_layers
        state.last_output = step_graph.out[-1]
        self._counts.layer_steps += self.cache.num_layers
        return step_graph.out

    def step(self, q, k, v, request_ids=None, layer_idx=0, rotary_dim=None, base=10_000.0):
        """Single-layer append -> decode step; backpressure returns without mutation."""
        self._require_no_open_step("run the single-layer step wrapper")
        if self.cache.num_layers != 1:
            raise RuntimeError("multi-layer caches require begin_step/step_layer/commit_step")
        with self._phase(PROFILE_RANGE_PREFLIGHT):
            ids = self._normalize_active_ids(request_ids)
            self._validate_step_inputs(ids, q, k, v)
            needed = self._needed_new_blocks(ids)
        free = self.cache.num_free_blocks
        if needed > free:
            self._counts.backpressure += 1
            return DecodeStepResult(status=self.STEP_BACKPRESSURE, request_ids=ids, output=None, positions=None,
                                    block_tables=None, seq_lens=None, needed_new_blocks=needed, free_blocks=free,
                                    reason="insufficient_physical_blocks")
        if self._append in ("torch", "fused_hip"):  # a one-layer token transaction
            if int(layer_idx) != 0:
                raise ValueError("single-layer step requires layer_idx=0")
            tx = self.begin_step(ids)
            self.step_layer(tx, 0, q, k, v, rotary_dim=rotary_dim, base=base)
            return self.commit_step(tx)
        from .rope import rope_paged_kv_append

        appended = rope_paged_kv_append(self.cache, layer_idx, ids, q, k, v, rotary_dim=rotary_dim, base=base,
                                        append_backend=self._append)
        output = self._decode(appended.q, appended.block_tables, appended.seq_lens, layer_idx)
        self._counts.steps += 1
        self._counts.tokens += len(ids)
        self._advanced()
        return DecodeStepResult(status=self.STEP_OK, request_ids=ids, output=output, positions=appended.positions,
                                block_tables=appended.block_tables, seq_lens=appended.seq_lens,
                                needed_new_blocks=needed, free_blocks=self.cache.num_free_blocks)

    # --------------------------------------------------------------- status
    def metrics(self):
        """Engine counters together with the cache metrics."""
        statuses = list(self._roster.status.values())
        by_status = {st: statuses.count(st)
                     for st in (self.WAITING, self.ACTIVE, self.FINISHED, self.CANCELLED, self.REJECTED)}
        c = self._counts
        return {
            "waiting_requests": by_status[self.WAITING],
            "active_requests": by_status[self.ACTIVE],
            "finished_requests": by_status[self.FINISHED],
            "cancelled_requests": by_status[self.CANCELLED],
            "rejected_requests": by_status[self.REJECTED],
            "completed_step_count": c.steps,
            "appended_token_count": c.tokens,
            "backpressure_count": c.backpressure,
            "state_version": self._version,
            "cache_state_version": self.cache.state_version,
            # the reference's scheduler-managed mode (policy, outside this data path) is never on
            "scheduler_managed": False,
            "committed_blocks": 0,
            "committed_but_unallocated_blocks": 0,
            "stale_decision_count": 0,
            "applied_decision_count": 0,
            "open_step_transaction_count": int(self._open is not None),
            "transaction_layer_step_count": c.layer_steps,
            "transaction_abort_count": c.aborts,
            "append_backend": self.append_backend,
            "decode_backend": self.decode_backend,
            "cache": self.cache.metrics(),
        }

    def validate_invariants(self):
        """Check engine lifecycle state against cache ownership state."""
        cache = self.cache
        cache.validate_invariants()
        open_step = self._open
        if open_step is None and cache.has_open_transaction:
            raise RuntimeError("cache has an open transaction not owned by DecodeEngine")
        if open_step is not None:
            if not cache.has_open_transaction:
                raise RuntimeError("Engine transaction is open but cache transaction is not")
            view = cache.transaction_view(open_step.cache_transaction)
            if view.request_ids != open_step.handle.request_ids:
                raise RuntimeError("Engine/cache transaction request rows diverged")
            if view.next_layer_idx != open_step.next_layer_idx:
                raise RuntimeError("Engine/cache transaction layer progress diverged")
        for rid, status in self._roster.status.items():
            try:
                cache_status = cache.request_state(rid)["status"]
            except KeyError:
                cache_status = None
            if status in (self.WAITING, self.REJECTED):
                if cache_status is not None:
                    raise RuntimeError("waiting request unexpectedly exists in PagedKVCache")
            elif cache_status != status:
                if cache_status is None:
                    cache.request_state(rid)  # re-raises the cache's own lookup error
                raise RuntimeError("DecodeEngine and PagedKVCache request status diverged")
        return True

    # ------------------------------------------------------------ internals
    def _write_layer(self, state, layer_idx, q, k, v, rotary_dim, base, cos_sin_table=None):
        """Returns (q_rotated, caller view, allocator device metadata or None)."""
        tx = state.cache_transaction
        if self._append == "fused_hip":
            meta = self.cache.transaction_device_metadata(tx)
            prepared = getattr(self.cache, "_write_layer_fused_prepared", None)
            if prepared is not None and self.cache.device.type == "cuda" and _own_method(
                    self.cache, "write_token_layer_fused_cuda"):
                # this package's cache, its fused write not replaced: the step's launch arguments are reused
                q_rot, view = prepared(tx, layer_idx, q, k, v, rotary_dim, base, cos_sin_table)
                return q_rot, view, meta
            # the table keyword goes only where it is used: the call keeps the
            # reference's signature otherwise
            extra = {} if cos_sin_table is None else {"cos_sin_table": cos_sin_table}
            q_rot, view = self.cache.write_token_layer_fused_cuda(tx, layer_idx, q, k, v, rotary_dim=rotary_dim,
                                                                  base=base, **extra)
            return q_rot, view, meta
        from .rope import apply_rope

        cur = self.cache.transaction_view(tx)
        q_rot = apply_rope(q, cur.positions, rotary_dim=rotary_dim, base=base)
        k_rot = apply_rope(k, cur.positions, rotary_dim=rotary_dim, base=base)
        view = self.cache.write_token_layer(tx, layer_idx, k_rot, v)
        return q_rot, view, None

    def _decode_layer(self, q_rot, view, meta, layer_idx):
        ragged = self._open is not None and self._open.ragged
        cascade = self._open.cascade if self._open is not None else None
        kv_reuse = self._open is not None and self._open.kv_reuse
        if meta is not None and cascade is None and self._decode_kind == "hip":
            return self._decode_prepared(self._open, q_rot, meta, layer_idx, ragged, kv_reuse)
        if meta is not None:  # the allocator's own copy, not the caller-visible clone
            return self._decode(q_rot, meta.block_tables, meta.eff_lens, layer_idx, ragged=ragged, cascade=cascade,
                                kv_reuse=kv_reuse)
        return self._decode(q_rot, view.block_tables, view.effective_seq_lens, layer_idx, ragged=ragged,
                            cascade=cascade, kv_reuse=kv_reuse)

    def _fused_layer(self, state, layer_idx, q, k, v, rotary_dim, base, cos_sin_table):
        """Whether this eager layer runs RoPE + K/V write inside its decode launch.

        After the step's first layer went the checked way (the RoPE + append
        kernel, then the prepared decode), later layers with the same RoPE
        setting and shapes take one launch: the decode kernel rotates q and
        the new K at the token's position, stores K/V at the reserved slot
        and attends to it from registers -- the same bits as the two kernels
        (the engine's step graphs do the same), minus a launch per layer.
        Returns ``(view, device metadata)`` once the cache recorded the
        layer, else None.
        """
        if not self.eager_fuse_rope or state.decode_launch is None or state.cascade is not None or state.ragged:
            return None
        cache = self.cache
        if self._append != "fused_hip" or self._decode_kind != "hip" or cache.device.type != "cuda":
            return None
        record = getattr(cache, "_layer_in_fused_decode", None)
        if record is None or not _own_method(cache, "write_token_layer_fused_cuda"):
            return None
        torch = _torch()
        head_dim = q.shape[-1]
        rdim = head_dim if rotary_dim is None else rotary_dim
        if (head_dim != 128 or rdim not in (64, 128) or q.shape[1] // cache.num_kv_heads > 16
                or q.dtype not in (torch.bfloat16, torch.float16)):
            return None
        if not (q.is_contiguous() and k.is_contiguous() and v.is_contiguous()):
            return None
        from . import _lib

        if state.decode_launch[0] != (_lib.current_stream_handle(q.device), tuple(q.shape), q.stride()):
            return None
        view = record(state.cache_transaction, layer_idx, rotary_dim, base, cos_sin_table)
        if view is None:
            return None
        return view, cache.transaction_device_metadata(state.cache_transaction)

    def _decode_fused_layer(self, state, q, k, v, meta, layer_idx, rotary_dim, base, cos_sin_table):
        """Eager decode of one layer with RoPE + K/V write inside the launch (see ``_fused_layer``):
        the step's decode arguments plus the append rows, the reserved slots and the RoPE setting."""
        from . import _lib
        from .paged_decode import _fill_append

        torch = _torch()
        cache = self.cache
        out = torch.empty_like(q)
        from .cache import _rope_key

        # the RoPE setting and the step's decode arguments (q's shape among
        # them) may change between layers: the arguments follow both
        key = (_rope_key(rotary_dim, base, cos_sin_table), state.decode_launch[0])
        if state.fused_launch is None or state.fused_launch[0] != key:
            base_args = state.decode_launch[1]
            args = type(base_args).from_buffer_copy(base_args)
            args.workspace = base_args.workspace
            _fill_append(args, k, v, meta.slots)
            args.rotary_dim = q.shape[-1] if rotary_dim is None else int(rotary_dim)
            args.rope_base = float(base)
            if cos_sin_table is not None:
                args.rope_cos_sin_table = cos_sin_table.data_ptr()
                args.rope_table_rows = cos_sin_table.shape[1]
            state.fused_launch = (key, args)
        else:
            args = state.fused_launch[1]
            args.append_k = k.data_ptr()
            args.append_v = v.data_ptr()
        args.q = q.data_ptr()
        args.out = out.data_ptr()
        layer_bytes = cache.k_cache.stride(0) * cache.k_cache.element_size()
        args.k_cache = cache.k_cache.data_ptr() + layer_idx * layer_bytes
        args.v_cache = cache.v_cache.data_ptr() + layer_idx * layer_bytes
        _lib.paged_decode(args, _lib.current_stream_handle(q.device))
        return out

    def _decode_prepared(self, state, q, meta, layer_idx, ragged, kv_reuse):
        """Eager HIP decode of one layer of the open step (the allocator's metadata).

        The step's first layer goes through ``paged_decode_attention``'s
        validation, split plan and workspace; the later layers of the step
        share them and change only the q, out and per-layer cache pointers
        (every layer's tables, lengths and shapes are the step's), which takes
        the host cost of a layer's decode from ~36 to a few us on MI355X.
        """
        from . import _lib
        from .paged_decode import _decode_args

        layer_idx = int(layer_idx)
        if layer_idx < 0 or layer_idx >= self.cache.num_layers:
            raise ValueError("layer_idx must be in [0, num_layers)")
        torch = _torch()
        cache = self.cache
        out = torch.empty_like(q)
        stream = _lib.current_stream_handle(q.device)
        key = (stream, tuple(q.shape), q.stride())
        if state.decode_launch is None or state.decode_launch[0] != key:
            args, _ = _decode_args(q, cache.k_cache[layer_idx], cache.v_cache[layer_idx], meta.block_tables,
                                   meta.eff_lens, out, self.sm_scale, cache.block_size, self.num_warps,
                                   "token_major", self.num_stages, None, 1, None, None, None, ragged, kv_reuse)
            state.decode_launch = (key, args)
        else:
            args = state.decode_launch[1]
            args.q = q.data_ptr()
            args.out = out.data_ptr()
            layer_bytes = cache.k_cache.stride(0) * cache.k_cache.element_size()
            args.k_cache = cache.k_cache.data_ptr() + layer_idx * layer_bytes
            args.v_cache = cache.v_cache.data_ptr() + layer_idx * layer_bytes
        _lib.paged_decode(args, stream)
        return out

    def _decode(self, q, block_tables, seq_lens, layer_idx=0, ragged=False, cascade=None, kv_reuse=False):
        layer_idx = int(layer_idx)
        if layer_idx < 0 or layer_idx >= self.cache.num_layers:
            raise ValueError("layer_idx must be in [0, num_layers)")
        if self._decode_kind == "reference":
            from .paged_reference import paged_decode_attention_ref

            return paged_decode_attention_ref(q, self.cache.k_cache[layer_idx], self.cache.v_cache[layer_idx],
                                              block_tables, seq_lens, sm_scale=self.sm_scale)
        if cascade is not None:
            from .cascade import paged_decode_attention_cascade

            self._cascade_decode_count += 1
            return paged_decode_attention_cascade(q, self.cache.k_cache[layer_idx], self.cache.v_cache[layer_idx],
                                                  block_tables, seq_lens, groups=cascade, sm_scale=self.sm_scale,
                                                  block_size=self.cache.block_size)
        from .paged_decode import paged_decode_attention

        return paged_decode_attention(q, self.cache.k_cache[layer_idx], self.cache.v_cache[layer_idx], block_tables,
                                      seq_lens, sm_scale=self.sm_scale, block_size=self.cache.block_size,
                                      num_warps=self.num_warps, num_stages=self.num_stages, ragged=ragged,
                                      kv_reuse=kv_reuse)

    def _require_no_open_step(self, action):
        if self._open is not None:
            raise RuntimeError(f"cannot {action} during an open decode step transaction")

    def _require_open_step(self, transaction):
        if not isinstance(transaction, DecodeStepTransaction):
            raise TypeError("transaction must be a DecodeStepTransaction")
        state = self._open
        if state is None:
            raise RuntimeError("DecodeEngine has no open decode step transaction")
        h = state.handle
        if (transaction.transaction_id, transaction.engine_version, transaction.request_ids) != (
                h.transaction_id, h.engine_version, h.request_ids):
            raise RuntimeError("stale or invalid DecodeEngine transaction handle")
        if state.state != "open":
            raise RuntimeError(f"decode step transaction is already {state.state}")
        return state

    def _validate_step_inputs(self, ids, q, k, v):
        if len(ids) == 1:  # one request may pass its K/V row without the batch axis
            k, v = (t.unsqueeze(0) if getattr(t, "dim", lambda: 0)() == 2 else t for t in (k, v))
        for broken, exc, message in _step_input_rules(self, ids, q, k, v):
            if broken():
                raise exc(message)

    def _needed_new_blocks(self, ids):
        """Requests whose next token starts a new block (one block each)."""
        bs = self.cache.block_size
        return sum(n % bs == 0 for n in self.cache._host_seq_lens(ids))

    def _normalize_active_ids(self, request_ids):
        ids = self.active_request_ids() if request_ids is None else self._normalize_ids(request_ids)
        if not ids:
            raise ValueError("at least one active request is required for a decode step")
        for rid in ids:
            self._roster.expect(rid, self.ACTIVE)
        return ids

    @staticmethod
    def _normalize_ids(request_ids):
        ids = _as_id_tuple(request_ids)
        for rid in ids:
            _require_hashable(rid)
        if len(set(ids)) != len(ids):
            raise ValueError("request_ids must be unique")
        return ids
