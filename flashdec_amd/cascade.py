"""Shared-prefix (cascade) paged decode on MI355X through ``libflashdec_hip.so``.

Rows attached to one registered prefix of the paged cache
(``PagedKVCache.attach_prefix``, flashdec/cache.py:225-248) lead their block
tables with the same physical blocks.  The reference's decode kernels read
that prefix once per row (flashdec/kernels/paged_decode.py:330-543); the
cascade launch reads it once per 16 (member, query head) rows of a group
and fills all 16 columns of the MFMA tiles with them (one request of a
GQA group of 8 fills only half):

1. prefix-role workgroups attend a group's prefix for 16 of its rows each,
   writing ``prefix_splits`` partials per row;
2. tail-role workgroups, in the same launch, attend every row's private
   tokens after its prefix (the whole row for rows in no group);
3. the split reducer merges both sets of partials (log-sum-exp).

The result equals :func:`flashdec_amd.paged_decode_attention` on the same
inputs (within floating-point reassociation).  Grouping is host logic over the
block tables (:func:`build_cascade_groups`); the caller rebuilds the groups
when tables change.
"""

from __future__ import annotations

import math
import threading
from dataclasses import dataclass

import numpy as np
import torch

from . import _lib
from .paged_decode import (_auto_workspace, _cache_strides, _fill_common, _fill_workspace, _launch_key,
                           _validate_inputs)

@dataclass(frozen=True)
class CascadeGroups:
    """Prefix groups of a batch (host-built, device-resident index tensors).

    ``members`` int32 ``[num_groups, max_members]`` (row indices, -1 after the
    last member; entry 0 is the lead, whose block-table row supplies the
    prefix's block ids), ``prefix_len`` int32 ``[num_groups]`` (shared tokens,
    whole blocks), ``row_prefix_len`` int32 ``[num_seqs]`` (0 for rows in no
    group).
    ``max_prefix_len``, ``max_tail_len`` and ``total_tail_len`` are host
    figures for split planning.
    """

    members: torch.Tensor
    prefix_len: torch.Tensor
    row_prefix_len: torch.Tensor
    max_prefix_len: int
    max_tail_len: int
    total_tail_len: int

    @property
    def num_groups(self) -> int:
        return int(self.members.shape[0])

    @property
    def max_members(self) -> int:
        return int(self.members.shape[1])


def group_rows(block_tables, seq_lens, block_size, max_members, min_prefix_blocks=1):
    """Host grouping: lists of ``(rows, prefix_blocks)``.

    Rows whose first physical block is the same are candidates; a candidate
    set's prefix is the longest run of leading block ids common to all of
    them, limited to each member's full blocks (a prefix never reaches past a
    member's length).  Sets larger than ``max_members`` are cut into the
    fewest chunks of near-equal size, in row order; sets of one row or with
    fewer than ``min_prefix_blocks`` shared blocks are dropped (those rows
    decode without a prefix pass).
    """
    bt = np.asarray(block_tables)
    sl = np.asarray(seq_lens).astype(np.int64)
    if bt.ndim != 2 or sl.ndim != 1 or sl.shape[0] != bt.shape[0]:
        raise ValueError("block_tables must be [num_seqs, max_blocks_per_seq] and seq_lens [num_seqs]")
    if max_members < 2:
        return []
    full = np.minimum(sl // block_size, bt.shape[1])
    buckets = {}
    for b in range(bt.shape[0]):
        if full[b] >= max(min_prefix_blocks, 1) and bt[b, 0] >= 0:
            buckets.setdefault(int(bt[b, 0]), []).append(b)
    groups = []
    for rows in buckets.values():
        pieces = -(-len(rows) // max_members)
        for part in np.array_split(np.asarray(rows), pieces):
            chunk = [int(r) for r in part]
            if len(chunk) < 2:
                continue
            limit = int(full[chunk].min())
            same = (bt[chunk, :limit] == bt[chunk[0], :limit]).all(axis=0)
            blocks = limit if same.all() else int(np.argmin(same))
            if blocks >= max(min_prefix_blocks, 1):
                groups.append((chunk, blocks))
    return groups


def build_cascade_groups(block_tables, seq_lens, block_size, num_q_heads, num_kv_heads, *, device=None,
                         min_prefix_blocks=1, max_members=None):
    """Find the batch's prefix groups and return them as :class:`CascadeGroups`.

    ``block_tables``/``seq_lens`` may live on any device (they are read on
    the host).  ``max_members`` bounds the rows of one group (default: no
    bound); larger sets of sharers are cut into near-equal groups.
    """
    if num_q_heads % num_kv_heads != 0:
        raise ValueError("num_q_heads must be divisible by num_kv_heads")
    if device is None:
        device = block_tables.device if isinstance(block_tables, torch.Tensor) else "cpu"
    bt = block_tables.cpu().numpy() if isinstance(block_tables, torch.Tensor) else np.asarray(block_tables)
    sl = seq_lens.cpu().numpy() if isinstance(seq_lens, torch.Tensor) else np.asarray(seq_lens)
    groups = group_rows(bt, sl, block_size, max_members or max(2, bt.shape[0]), min_prefix_blocks)
    width = max([len(rows) for rows, _ in groups], default=1)
    members = np.full((len(groups), width), -1, dtype=np.int32)
    prefix = np.zeros(len(groups), dtype=np.int32)
    row_prefix = np.zeros(sl.shape[0], dtype=np.int32)
    for g, (rows, blocks) in enumerate(groups):
        members[g, : len(rows)] = rows
        prefix[g] = blocks * block_size
        row_prefix[rows] = blocks * block_size
    tails = np.maximum(sl.astype(np.int64) - row_prefix, 0)
    return CascadeGroups(
        members=torch.from_numpy(members).to(device),
        prefix_len=torch.from_numpy(prefix).to(device),
        row_prefix_len=torch.from_numpy(row_prefix).to(device),
        max_prefix_len=int(prefix.max(initial=0)),
        max_tail_len=int(tails.max(initial=0)),
        total_tail_len=int(tails.sum()),
    )


def plan_prefix_splits(num_groups, num_kv_heads, chunks, max_prefix_len, num_cus, share=1.0, min_tiles=16):
    """Prefix partials per (group, KV head, chunk of ``FD_CASCADE_CHUNK_ROWS`` rows).

    About ``share`` of the CUs take one prefix-role workgroup each, and a
    split holds at least ``min_tiles`` prefix tiles.  With the defaults, the
    best of a same-box sweep on MI355X (sharers x prefix tokens: prefix splits
    chosen -> cascade vs per-row us/call): 16 x 4096: 8 -> 14.2 vs 14.5;
    32 x 8192: 8 -> 23.4 vs 32.8; 64 x 16384: 4 -> 50.5 vs 96.0; 128 x 16384:
    2 -> 88.7 vs 183.0 (each split's tail count planned on its own).
    :func:`plan_cascade_splits` plans both counts together.
    """
    tiles = max(1, -(-max_prefix_len // 32))
    want = max(1, int(num_cus * share) // max(1, num_groups * num_kv_heads * chunks))
    return int(min(want, -(-tiles // min_tiles), 1024))


def _whole_wave_tail_splits(num_seqs, num_q_heads, num_kv_heads, head_dim, groups, prefix_blocks, num_cus,
                            prefix_tiles=None):
    """(the tails' own plan, the fewest tail splits that make the launch whole waves or None)."""
    base = _lib.paged_decode_plan(num_seqs, num_q_heads, num_kv_heads, head_dim, max(groups.max_tail_len, 1),
                                  max(groups.total_tail_len, 1))
    pairs = num_seqs * num_kv_heads
    low = max(1, (base + 1) // 2)
    if prefix_tiles is not None:
        # a tail-role workgroup may also be as long as a prefix-role one
        tail_tiles = max(1, -(-groups.max_tail_len // 32))
        low = min(low, max(1, -(-tail_tiles // max(1, prefix_tiles))))
    for splits in range(low, base + 1):
        if (prefix_blocks + pairs * splits) % num_cus == 0:
            return base, splits
    return base, None


def plan_tail_splits(num_seqs, num_q_heads, num_kv_heads, head_dim, groups, prefix_blocks, num_cus):
    """Tail splits of a cascade launch: the fewest from half the library's plan for the tails alone
    up to that plan that make the launch (``prefix_blocks`` prefix-role workgroups plus the
    tail-role ones) whole waves of workgroups; the plan where none does.  The lower bound keeps a
    tail-role workgroup at no more than about twice the tokens the plan gives it.

    The tail-role workgroups run after the prefix role's, so the tails' own plan (sized as if they
    had the GPU to themselves) can add a wave: same-box MI355X sweep, us/call by tail splits,
    64 x 16384 (256 prefix-role workgroups, 128 rows x KV heads): 1: 40.2, 2: 39.4, 4: 42.5 (the
    tails' plan), 8: 48.1; 32 x 8192 (256 + 64 per split): 2: 22.9, 4: 22.0, 8: 24.4.
    """
    base, splits = _whole_wave_tail_splits(num_seqs, num_q_heads, num_kv_heads, head_dim, groups, prefix_blocks,
                                           num_cus)
    return base if splits is None else splits


def plan_cascade_splits(num_seqs, num_q_heads, num_kv_heads, head_dim, groups, chunks, num_cus):
    """(prefix splits, tail splits) of a cascade launch over ``chunks`` prefix chunks per (group, KV head).

    The launch's time is its longest workgroup's, and a prefix-role workgroup
    streams its tiles through one CU's vector memory path (the prefix is read
    from L2 by every chunk), so the plan first gives the prefix role about
    three quarters of the CUs, at least 8 tiles a split, and the tail role
    the rest of one wave (a tail-role workgroup no longer than a prefix-role
    one); where no tail split count fills whole waves it falls back to one
    prefix-role workgroup per CU (:func:`plan_prefix_splits`,
    :func:`plan_tail_splits`).  Same-box MI355X sweep, us/call (chunk rows /
    prefix splits / tail splits): 16 x 4096: 16/12/2 13.48 (16/8/4, the
    earlier plan, 14.68; 16/14/1 14.04; 16/10/2 13.96); 32 x 8192: 32/12/1
    18.59, 32/12/2 18.36 (16/8/4, the earlier plan, 22.03); 64 x 16384: 32/8/2
    36.98 (32/6/2 37.48).
    """
    units = max(1, groups.num_groups * num_kv_heads * chunks)
    prefix_tiles = max(1, -(-groups.max_prefix_len // 32))
    for share, min_tiles in ((0.75, 8), (1.0, 16)):
        sp = plan_prefix_splits(groups.num_groups, num_kv_heads, chunks, groups.max_prefix_len, num_cus, share,
                                min_tiles)
        base, st = _whole_wave_tail_splits(num_seqs, num_q_heads, num_kv_heads, head_dim, groups, units * sp,
                                           num_cus, prefix_tiles=-(-prefix_tiles // sp))
        if st is not None:
            return sp, st
    return sp, base


# plan_chunk_rows: group rows (sharers x query heads per KV head) x prefix
# tokens from which a 32-row chunk pays for its doubled per-unit work.  Same-box
# MI355X sweep, best prefix / tail splits each, 16- vs 32-row chunks (us/call):
# 16 x 4096 13.48 vs 16.09; 32 x 8192 21.30 vs 18.36; 64 x 16384 (earlier
# build, best prefix splits) 54.2 vs 46.2; 128 x 16384 91.5 vs 68.8 (Hq16/Hkv2:
# 8 rows per sharer).
_WIDE_CHUNK_MIN_WORK = 1 << 21


def plan_chunk_rows(groups, num_q_heads, num_kv_heads):
    """Rows per prefix-role chunk: 16, or ``FD_CASCADE_MAX_CHUNK_ROWS`` (two MFMA column blocks per wave)
    when the group's rows x prefix tokens are large enough that the halved prefix re-reads pay for the
    doubled work per K/V unit."""
    rows = groups.max_members * (num_q_heads // num_kv_heads)
    return _lib.CASCADE_MAX_CHUNK_ROWS if rows * groups.max_prefix_len >= _WIDE_CHUNK_MIN_WORK else 16


def prefix_chunks(groups, num_q_heads, num_kv_heads, chunk_rows=16):
    """Prefix-role chunks per group and KV head: rows (members x query heads per KV head)
    in chunks of ``chunk_rows``, one prefix-role workgroup each."""
    return -(-groups.max_members * (num_q_heads // num_kv_heads) // chunk_rows)


_NUM_CUS = {}


def _num_cus(device):
    idx = device.index if device.index is not None else torch.cuda.current_device()
    if idx not in _NUM_CUS:
        _NUM_CUS[idx] = torch.cuda.get_device_properties(idx).multi_processor_count
    return _NUM_CUS[idx]


def paged_decode_attention_cascade_into(
    q,
    k_cache,
    v_cache,
    block_tables,
    seq_lens,
    out,
    groups: CascadeGroups,
    sm_scale=None,
    block_size=None,
    num_splits=None,
    prefix_splits=None,
    kv_reuse=True,
    workspace=None,
    chunk_rows=None,
):
    """Write shared-prefix decode attention into ``out``.

    Token-major caches ``[num_blocks, num_kv_heads, block_size, 128]`` with
    up to 16 query heads per KV head; same shapes and meaning as
    :func:`flashdec_amd.paged_decode_attention_into`.  ``groups`` must have
    been built for these ``block_tables``/``seq_lens`` (see
    :func:`build_cascade_groups`).  ``num_splits`` (tail) and
    ``prefix_splits`` default to the library's plan for the tail lengths and
    to :func:`plan_prefix_splits`.  The prefix pass reads its blocks with
    plain loads (the group's chunks re-read them).  ``kv_reuse=False``
    streams the private tails with non-temporal loads instead; the default
    keeps plain loads there too (on MI355X streamed tails took 14.0 vs 15.1 us
    for 16 rows x 4096 shared tokens but 55.4 vs 52.9 us for 64 x 16384).
    ``workspace`` = ``(acc, max, sum)`` fp32 ``[>= B, >= Hq, >= S + S_p, D]`` /
    ``[..., >= S + S_p]`` (equal max/sum strides) replaces the library's own,
    e.g. for graph capture.  ``chunk_rows`` (16 or 32; default
    :func:`plan_chunk_rows`) is how many of a group's rows one prefix-role
    workgroup attends.
    """
    key = None
    last = getattr(_LAST_CASCADE, "entry", None)
    if last is not None and isinstance(q, torch.Tensor) and q.is_cuda and isinstance(groups, CascadeGroups):
        stream = _lib.current_stream_handle(q.device)
        try:
            key = _cascade_key(q, k_cache, v_cache, block_tables, seq_lens, out, groups, workspace,
                               (sm_scale, block_size, num_splits, prefix_splits, kv_reuse, chunk_rows, stream))
        except (AttributeError, TypeError):
            key = None  # an argument that is not a tensor: the full path raises the reference's message
        if key is not None and last[0] == key:
            # the previous call's metadata and settings: only data pointers change
            args, cas = last[1]
            args.q = q.data_ptr()
            args.k_cache = k_cache.data_ptr()
            args.v_cache = v_cache.data_ptr()
            args.block_tables = block_tables.data_ptr()
            args.seq_lens = seq_lens.data_ptr()
            args.out = out.data_ptr()
            if workspace is not None:
                args.split_acc, args.split_max, args.split_sum = (t.data_ptr() for t in workspace)
                args.workspace = tuple(workspace)
            cas.group_members = groups.members.data_ptr()
            cas.group_prefix_len = groups.prefix_len.data_ptr()
            cas.row_prefix_len = groups.row_prefix_len.data_ptr()
            _lib.paged_decode_cascade(args, cas, stream)
            return out
    sm_scale_in, block_size_in, num_splits_in, prefix_splits_in, chunk_rows_in = (sm_scale, block_size, num_splits,
                                                                                   prefix_splits, chunk_rows)
    if block_size is None:
        if k_cache.dim() != 4:
            raise ValueError("k_cache must be a 4D tensor")
        block_size = k_cache.shape[2]
    block_size = int(block_size)
    _validate_inputs(q, k_cache, v_cache, block_tables, seq_lens, block_size, 2, None, "token_major")
    if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError("out must match q in shape, dtype and device")
    num_seqs, num_q_heads, head_dim = q.shape
    num_kv_heads = k_cache.shape[1]
    for name, t in (("members", groups.members), ("prefix_len", groups.prefix_len),
                    ("row_prefix_len", groups.row_prefix_len)):
        if t.dtype != torch.int32 or t.device != q.device or not t.is_contiguous():
            raise ValueError(f"groups.{name} must be a contiguous int32 tensor on q.device")
    if groups.row_prefix_len.shape != (num_seqs,):
        raise ValueError("groups.row_prefix_len must have one entry per sequence")
    if groups.prefix_len.shape != (groups.num_groups,):
        raise ValueError("groups.prefix_len must have one entry per group")
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(head_dim)
    if chunk_rows is None:
        chunk_rows = plan_chunk_rows(groups, num_q_heads, num_kv_heads)
    if chunk_rows not in (16, _lib.CASCADE_MAX_CHUNK_ROWS):
        raise ValueError(f"chunk_rows must be 16 or {_lib.CASCADE_MAX_CHUNK_ROWS}")
    chunks = prefix_chunks(groups, num_q_heads, num_kv_heads, chunk_rows)
    if prefix_splits is None and num_splits is None:
        prefix_splits, num_splits = plan_cascade_splits(num_seqs, num_q_heads, num_kv_heads, head_dim, groups,
                                                        chunks, _num_cus(q.device))
    if prefix_splits is None:
        prefix_splits = plan_prefix_splits(groups.num_groups, num_kv_heads, chunks, groups.max_prefix_len,
                                           _num_cus(q.device))
    if num_splits is None:
        if isinstance(prefix_splits, int) and not isinstance(prefix_splits, bool) and prefix_splits > 0:
            num_splits = plan_tail_splits(num_seqs, num_q_heads, num_kv_heads, head_dim, groups,
                                          groups.num_groups * num_kv_heads * chunks * prefix_splits,
                                          _num_cus(q.device))
        else:
            num_splits = 1  # the check below reports prefix_splits
    for name, v in (("num_splits", num_splits), ("prefix_splits", prefix_splits)):
        if isinstance(v, bool) or not isinstance(v, int) or v <= 0:
            raise ValueError(f"{name} must be a positive integer")
    stream = _lib.current_stream_handle(q.device)
    if workspace is None:
        acc, mx, sm, _ = _auto_workspace(q, num_kv_heads, num_splits + prefix_splits, stream)
    else:
        acc, mx, sm = workspace
        need = num_splits + prefix_splits
        if (any(t.dtype != torch.float32 or t.device != q.device for t in (acc, mx, sm)) or acc.dim() != 4
                or acc.shape[0] < num_seqs or acc.shape[1] < num_q_heads or acc.shape[2] < need
                or acc.shape[3] != head_dim or mx.shape[:3] != acc.shape[:3] or sm.shape != mx.shape
                or sm.stride() != mx.stride() or acc.stride(3) != 1):
            raise ValueError("workspace must be fp32 (acc [>=B, >=Hq, >=S+S_p, D], max/sum [>=B, >=Hq, >=S+S_p]) "
                             "on q.device with equal max/sum strides")

    args = _lib.PagedDecodeArgs()
    _fill_common(args, q, k_cache, v_cache, _cache_strides(k_cache, 2, 3), _cache_strides(v_cache, 2, 3),
                 block_tables, seq_lens, out, num_kv_heads, block_size, sm_scale)
    args.num_blocks = k_cache.shape[0]
    args.max_seq_len = groups.max_prefix_len + groups.max_tail_len
    args.kv_reuse = 1 if kv_reuse else 0
    _fill_workspace(args, acc, mx, sm, num_splits)
    # the cascade always writes partials, also with a single tail split
    args.split_acc = acc.data_ptr()
    args.split_acc_stride[:] = acc.stride()
    args.split_max = mx.data_ptr()
    args.split_sum = sm.data_ptr()
    args.split_stats_stride[:] = mx.stride()
    cas = _lib.CascadeArgs()
    cas.num_groups = groups.num_groups
    cas.max_members = groups.max_members
    cas.prefix_splits = prefix_splits
    cas.group_members = groups.members.data_ptr()
    cas.group_prefix_len = groups.prefix_len.data_ptr()
    cas.row_prefix_len = groups.row_prefix_len.data_ptr()
    cas.max_prefix_len = groups.max_prefix_len
    cas.chunk_rows = chunk_rows
    args.workspace = (acc, mx, sm)  # alive as long as the arguments that point into it
    _lib.paged_decode_cascade(args, cas, stream)
    if key is None:
        key = _cascade_key(q, k_cache, v_cache, block_tables, seq_lens, out, groups, workspace,
                           (sm_scale_in, block_size_in, num_splits_in, prefix_splits_in, kv_reuse, chunk_rows_in,
                            stream))
    _LAST_CASCADE.entry = (key, (args, cas))
    return out


# The last cascade launch of each thread: (metadata key, (PagedDecodeArgs, CascadeArgs)).
_LAST_CASCADE = threading.local()


def _cascade_key(q, k_cache, v_cache, block_tables, seq_lens, out, groups, workspace, settings):
    """What a cascade launch's validation, plans and arguments depend on except data pointers: the
    tensors' metadata, the groups' host figures and index-tensor metadata, and the settings."""
    def meta(t):
        return (t.shape, t.stride(), t.dtype, t.device)

    figures = (groups.num_groups, groups.max_members, groups.max_prefix_len, groups.max_tail_len,
               groups.total_tail_len, meta(groups.members), meta(groups.prefix_len), meta(groups.row_prefix_len))
    return (_launch_key(q, k_cache, v_cache, block_tables, seq_lens, out, workspace, None, None, None, settings),
            figures)


def paged_decode_attention_cascade(q, k_cache, v_cache, block_tables, seq_lens, groups=None, sm_scale=None,
                                   block_size=None, num_splits=None, prefix_splits=None, kv_reuse=True,
                                   chunk_rows=None):
    """Allocating form of :func:`paged_decode_attention_cascade_into`; builds
    the groups from the tables when ``groups`` is None."""
    if block_size is None:
        if k_cache.dim() != 4:
            raise ValueError("k_cache must be a 4D tensor")
        block_size = k_cache.shape[2]
    if groups is None:
        groups = build_cascade_groups(block_tables, seq_lens, int(block_size), q.shape[1], k_cache.shape[1],
                                      device=q.device)
    out = torch.empty_like(q)
    return paged_decode_attention_cascade_into(q, k_cache, v_cache, block_tables, seq_lens, out, groups,
                                               sm_scale=sm_scale, block_size=block_size, num_splits=num_splits,
                                               prefix_splits=prefix_splits, kv_reuse=kv_reuse,
                                               chunk_rows=chunk_rows)
