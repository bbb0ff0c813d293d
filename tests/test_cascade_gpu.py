"""GPU parity of shared-prefix (cascade) decode against the CPU oracle.

Group members lead their block tables with the same physical blocks (the
layout ``PagedKVCache.attach_prefix`` produces, flashdec/cache.py:225-248);
the cascade result must equal plain paged decode of the same tables, so the
oracle is the ordinary paged-decode oracle.  Cases: block sizes 8/16/32,
group sizes 1/8/16, fp16 and bf16, prefixes that end inside a 32-token tile,
rows whose tail is empty, zero-length rows, rows in no group, groups of 32
and 40 members (16 and 20 sixteen-row chunks per KV head), more prefix
splits than prefix tiles, explicit tail split counts, groups whose prefix is
shorter than what the tables share, and padded member lists -- with 16-row
and 32-row prefix chunks (one or two MFMA column blocks per wave).
Tolerance: atol 2e-2 / rtol 1e-2.
"""

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, np32

pytestmark = pytest.mark.gpu


def _cascade():
    from flashdec_amd import cascade

    return cascade


@pytest.fixture
def record():
    from flashdec_amd import _lib

    _lib.record_launches(True)
    yield _lib
    _lib.record_launches(False)


def make_prefix_inputs(groups, singles, hq, hkv, block_size, dtype, seed=3, head_dim=128):
    """groups: list of (prefix_blocks, [tail tokens per member]); singles:
    lengths of rows that share nothing.  Returns q, k, v, table, lens (cuda)
    plus the expected (rows, prefix_blocks) of every group."""
    rng = np.random.default_rng(seed)
    rows = []  # (shared block ids, private tokens)
    expected = []
    next_row = 0
    need = 0
    for pblocks, tails in groups:
        expected.append((list(range(next_row, next_row + len(tails))), pblocks))
        next_row += len(tails)
        need += pblocks + sum(-(-t // block_size) for t in tails)
    need += sum(-(-n // block_size) for n in singles)
    pool = int(need * 1.3) + 4
    perm = rng.permutation(pool)
    cursor = 0

    def take(n):
        nonlocal cursor
        out = perm[cursor : cursor + n]
        cursor += n
        return list(out)

    lens = []
    tables = []
    for pblocks, tails in groups:
        shared = take(pblocks)
        for t in tails:
            tables.append(shared + take(-(-t // block_size)))
            lens.append(pblocks * block_size + t)
    for n in singles:
        tables.append(take(-(-n // block_size)))
        lens.append(n)
    width = max(1, max(len(t) for t in tables))
    table = np.full((len(tables), width), -1, dtype=np.int32)
    for b, t in enumerate(tables):
        table[b, : len(t)] = t
    gen = torch.Generator().manual_seed(seed)
    shape = (pool, hkv, block_size, head_dim)
    k = torch.randn(shape, generator=gen).to(dtype)
    v = torch.randn(shape, generator=gen).to(dtype)
    q = torch.randn((len(lens), hq, head_dim), generator=gen).to(dtype)
    return (q.cuda(), k.cuda(), v.cuda(), torch.from_numpy(table).cuda(),
            torch.tensor(lens, dtype=torch.int32).cuda(), expected)


def _oracle(q, k, v, table, lens):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy())


def _groups_as_sets(groups):
    members = groups.members.cpu().numpy()
    plen = groups.prefix_len.cpu().numpy()
    return sorted((tuple(int(x) for x in m if x >= 0), int(p)) for m, p in zip(members, plen))


@pytest.mark.parametrize("chunk_rows", [16, 32])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize(("hq", "hkv"), [(16, 2), (8, 8), (32, 2)])
def test_shared_prefix_matches_oracle(hq, hkv, block_size, dtype, chunk_rows):
    # prefixes of 13 and 3 blocks (ends inside a 32-token tile for bs 8/16),
    # tails including empty ones, rows in no group, one zero-length row
    groups = [(13, [5, 0, 77, 1, 40]), (3, [9, block_size])]
    q, k, v, table, lens, expected = make_prefix_inputs(groups, [0, 50, 130], hq, hkv, block_size, dtype)
    cas = _cascade()
    g = cas.build_cascade_groups(table, lens, block_size, hq, hkv)
    assert _groups_as_sets(g) == sorted((tuple(r), p * block_size) for r, p in expected)
    out = cas.paged_decode_attention_cascade(q, k, v, table, lens, groups=g, block_size=block_size,
                                             chunk_rows=chunk_rows)
    expected_out = _oracle(q, k, v, table, lens)
    assert_close_to_oracle(out, expected_out)
    assert torch.count_nonzero(out[7]) == 0  # the zero-length row


@pytest.mark.parametrize("dtype", [torch.bfloat16])
def test_group_of_32_members(dtype):
    rng = np.random.default_rng(5)
    tails = [int(x) for x in rng.integers(1, 100, size=32)]
    q, k, v, table, lens, expected = make_prefix_inputs([(64, tails)], [300], 16, 2, 16, dtype, seed=9)
    cas = _cascade()
    g = cas.build_cascade_groups(table, lens, 16, 16, 2)
    assert g.num_groups == 1 and g.max_members == 32 and g.max_prefix_len == 1024
    out = cas.paged_decode_attention_cascade(q, k, v, table, lens, groups=g)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


@pytest.mark.parametrize("chunk_rows", [16, 32])
def test_large_group_spans_many_chunks(chunk_rows):
    # 40 members x 8 query heads per KV head = 320 rows: 20 chunks of 16, or 10 of 32
    rng = np.random.default_rng(8)
    tails = [int(x) for x in rng.integers(0, 70, size=40)]
    q, k, v, table, lens, _ = make_prefix_inputs([(9, tails)], [33], 16, 2, 16, torch.bfloat16, seed=13)
    cas = _cascade()
    g = cas.build_cascade_groups(table, lens, 16, 16, 2)
    assert g.num_groups == 1 and g.max_members == 40
    out = cas.paged_decode_attention_cascade(q, k, v, table, lens, groups=g, chunk_rows=chunk_rows)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


@pytest.mark.parametrize("chunk_rows", [16, 32])
@pytest.mark.parametrize(("num_splits", "prefix_splits"), [(1, 1), (3, 2), (2, 40), (8, 7)])
def test_explicit_split_counts(num_splits, prefix_splits, chunk_rows):
    # prefix of 20 blocks of 16 = 10 tiles: 40 prefix splits leave 30 empty
    q, k, v, table, lens, _ = make_prefix_inputs([(20, [33, 200, 7, 64])], [90, 1], 16, 2, 16, torch.bfloat16,
                                                 seed=11)
    cas = _cascade()
    g = cas.build_cascade_groups(table, lens, 16, 16, 2)
    out = cas.paged_decode_attention_cascade(q, k, v, table, lens, groups=g, num_splits=num_splits,
                                             prefix_splits=prefix_splits, chunk_rows=chunk_rows)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_no_shared_prefix_decodes_every_row_in_the_tail_pass():
    q, k, v, table, lens, _ = make_prefix_inputs([], [40, 0, 513, 96], 16, 2, 32, torch.bfloat16, seed=2)
    cas = _cascade()
    g = cas.build_cascade_groups(table, lens, 32, 16, 2)
    assert g.num_groups == 0 and int(g.row_prefix_len.abs().sum()) == 0
    out = cas.paged_decode_attention_cascade(q, k, v, table, lens, groups=g)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_hand_built_groups_shorter_prefix_and_padding():
    # tables share 12 blocks but the group claims 5; members listed out of
    # order with -1 padding; one row of the shared set left out of the group
    q, k, v, table, lens, _ = make_prefix_inputs([(12, [17, 3, 60, 25])], [77], 16, 2, 16, torch.float16, seed=4)
    cas = _cascade()
    dev = q.device
    groups = cas.CascadeGroups(
        members=torch.tensor([[2, 0, 3, -1, -1, -1]], dtype=torch.int32, device=dev),
        prefix_len=torch.tensor([5 * 16], dtype=torch.int32, device=dev),
        row_prefix_len=torch.tensor([80, 0, 80, 80, 0], dtype=torch.int32, device=dev),
        max_prefix_len=80,
        max_tail_len=int(lens.max()),
        total_tail_len=int(lens.sum()),
    )
    for chunk_rows in (16, 32):
        out = torch.empty_like(q)
        cas.paged_decode_attention_cascade_into(q, k, v, table, lens, out, groups, prefix_splits=3,
                                                chunk_rows=chunk_rows)
        assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_two_calls_reuse_the_workspace():
    cas = _cascade()
    q, k, v, table, lens, _ = make_prefix_inputs([(40, [10, 300, 1])], [5], 16, 2, 16, torch.bfloat16, seed=21)
    g = cas.build_cascade_groups(table, lens, 16, 16, 2)
    first = cas.paged_decode_attention_cascade(q, k, v, table, lens, groups=g).clone()
    q2, k2, v2, table2, lens2, _ = make_prefix_inputs([(6, [3, 8])], [], 16, 2, 16, torch.bfloat16, seed=22)
    g2 = cas.build_cascade_groups(table2, lens2, 16, 16, 2)
    second = cas.paged_decode_attention_cascade(q2, k2, v2, table2, lens2, groups=g2)
    again = cas.paged_decode_attention_cascade(q, k, v, table, lens, groups=g)
    torch.cuda.synchronize()
    assert_close_to_oracle(second, _oracle(q2, k2, v2, table2, lens2))
    assert torch.equal(first, again)


def test_unsupported_shapes_raise():
    cas = _cascade()
    q, k, v, table, lens, _ = make_prefix_inputs([(4, [3, 8])], [], 8, 2, 16, torch.bfloat16, head_dim=64)
    g = cas.build_cascade_groups(table, lens, 16, 8, 2)
    with pytest.raises(RuntimeError, match="head_dim 128"):
        cas.paged_decode_attention_cascade(q, k, v, table, lens, groups=g)


def test_repeated_cascade_calls_reuse_arguments_but_follow_every_pointer():
    """The cascade entry keeps the last call's arguments when only data pointers change: two input sets
    with their own groups objects, alternated, and a caller workspace swapped between calls, each give
    their own result."""
    cas = _cascade()
    groups_def = [(13, [5, 0, 77, 1, 40]), (3, [9, 32])]
    sets = []
    for seed in (31, 32):
        q, k, v, table, lens, _ = make_prefix_inputs(groups_def, [0, 50, 130], 16, 2, 32, torch.bfloat16, seed=seed)
        sets.append((q, k, v, table, lens, cas.build_cascade_groups(table, lens, 32, 16, 2)))
    wss = [(torch.empty((10, 16, 24, 128), device="cuda"), torch.empty((10, 16, 24), device="cuda"),
            torch.empty((10, 16, 24), device="cuda")) for _ in range(2)]
    for rnd in range(3):
        for i, (q, k, v, table, lens, g) in enumerate(sets):
            expected = _oracle(q, k, v, table, lens)
            out = torch.empty_like(q)
            cas.paged_decode_attention_cascade_into(q, k, v, table, lens, out, g)
            assert_close_to_oracle(out, expected)
            out2 = torch.empty_like(q)
            cas.paged_decode_attention_cascade_into(q, k, v, table, lens, out2, g, num_splits=4, prefix_splits=8,
                                                    workspace=wss[(i + rnd) % 2])
            assert_close_to_oracle(out2, expected)


@pytest.mark.parametrize("packed", [True, False])
def test_rows_without_a_prefix_ignore_poisoned_prefix_slots(packed, record):
    """Rows in no group (and zero-length rows) have no prefix partials: the merge must not read
    them.  With a packed workspace the preloaded cascade merge loads every split before the row's
    prefix length arrives and masks the prefix splits by selection, so NaN left in those slots
    must not reach the output; a strided workspace takes the other merge.  Both must equal the
    oracle on a workspace poisoned with NaN before every call."""
    cas = _cascade()
    groups_def = [(20, [7, 0, 300]), (5, [64, 1])]
    q, k, v, table, lens, _ = make_prefix_inputs(groups_def, [0, 90, 513, 1], 16, 2, 32, torch.bfloat16, seed=71)
    g = cas.build_cascade_groups(table, lens, 32, 16, 2)
    b, hq = q.shape[:2]
    tail, pre = 3, 4
    if packed:
        ws = (torch.full((b, hq, tail + pre, 128), float("nan"), device="cuda"),
              torch.full((b, hq, tail + pre), float("nan"), device="cuda"),
              torch.full((b, hq, tail + pre), float("nan"), device="cuda"))
    else:
        # statistics with a split stride of 2: not the packed layout
        big = torch.full((b, hq, tail + pre + 2, 136), float("nan"), device="cuda")
        st = torch.full((b, hq, 2 * (tail + pre)), float("nan"), device="cuda")
        ws = (big[:, :, 1:tail + pre + 1, :128], st[:, :, ::2], st.clone()[:, :, ::2])
    expected = _oracle(q, k, v, table, lens)
    for rep in range(2):
        for t in ws:
            t.fill_(float("nan"))
        out = torch.empty_like(q)
        cas.paged_decode_attention_cascade_into(q, k, v, table, lens, out, g, num_splits=tail, prefix_splits=pre,
                                                workspace=ws)
        torch.cuda.synchronize()
        reducer = record.last_launch()[-1]
        assert ("split_reduce_cascade_pre_kernel" in reducer) == packed, reducer
        assert_close_to_oracle(out, expected)
