"""Host logic of shared-prefix decode: grouping rows by their leading blocks.

Pinned by hand-worked tables: the expected groups follow from which leading
block ids the rows hold in common and from each row's count of full blocks.
"""

import numpy as np
import torch

from flashdec_amd import cascade


def test_groups_follow_common_leading_blocks():
    bt = np.array([
        [7, 8, 9, 40, -1],   # row 0: shares 7, 8, 9 with rows 1 and 3
        [7, 8, 9, 41, 42],
        [50, 51, -1, -1, -1],
        [7, 8, 9, 43, -1],
        [60, 61, 62, -1, -1],  # row 4: shares 60, 61 with row 5
        [60, 61, 70, -1, -1],
    ], dtype=np.int32)
    sl = np.array([60, 80, 20, 64, 48, 33], dtype=np.int32)  # block size 16
    groups = cascade.group_rows(bt, sl, 16, max_members=8)
    assert sorted(groups) == [([0, 1, 3], 3), ([4, 5], 2)]


def test_prefix_stops_at_a_members_full_blocks():
    bt = np.array([[1, 2, 3, 4], [1, 2, 3, 4], [1, 2, 3, 5]], dtype=np.int32)
    # row 1 holds 2 full blocks of 8 (tokens 0..19): the prefix stops there
    sl = np.array([32, 20, 30], dtype=np.int32)
    assert cascade.group_rows(bt, sl, 8, max_members=4) == [([0, 1, 2], 2)]
    # a row with no full block joins no group
    sl2 = np.array([32, 7, 30], dtype=np.int32)
    assert cascade.group_rows(bt, sl2, 8, max_members=4) == [([0, 2], 3)]


def test_large_sets_are_cut_and_singletons_dropped():
    bt = np.array([[9, i + 10] for i in range(5)], dtype=np.int32)
    sl = np.full(5, 20, dtype=np.int32)
    # 5 sharers, at most 2 per group: three chunks [0, 1], [2, 3], [4]; the
    # lone row is dropped
    assert cascade.group_rows(bt, sl, 16, max_members=2) == [([0, 1], 1), ([2, 3], 1)]
    assert cascade.group_rows(bt, sl, 16, max_members=2, min_prefix_blocks=2) == []
    assert cascade.group_rows(bt, sl, 16, max_members=1) == []


def test_build_cascade_groups_tensors():
    bt = torch.tensor([[3, 4, 5], [3, 4, 6], [8, -1, -1], [3, 4, 7]], dtype=torch.int32)
    sl = torch.tensor([40, 48, 5, 35], dtype=torch.int32)
    g = cascade.build_cascade_groups(bt, sl, 16, num_q_heads=16, num_kv_heads=2)
    assert g.num_groups == 1 and g.max_members == 3
    assert g.members.tolist() == [[0, 1, 3]]
    assert g.prefix_len.tolist() == [32]
    assert g.row_prefix_len.tolist() == [32, 32, 0, 32]
    assert g.members.dtype == torch.int32 and g.row_prefix_len.dtype == torch.int32
    assert g.max_prefix_len == 32
    assert g.max_tail_len == 16 and g.total_tail_len == 8 + 16 + 5 + 3


def test_group_size_bound():
    n = 40
    bt = torch.tensor([[1, 100 + i] for i in range(n)], dtype=torch.int32)
    sl = torch.full((n,), 20, dtype=torch.int32)
    g = cascade.build_cascade_groups(bt, sl, 16, num_q_heads=16, num_kv_heads=2)  # no bound: one group
    assert g.num_groups == 1 and g.max_members == 40
    g = cascade.build_cascade_groups(bt, sl, 16, num_q_heads=16, num_kv_heads=2, max_members=16)
    assert g.num_groups == 3 and g.max_members == 14  # 40 rows: 14 + 13 + 13
    assert sorted(len([x for x in m if x >= 0]) for m in g.members.tolist()) == [13, 13, 14]
    # 40 members x 8 query heads per KV head = 320 rows: 20 chunks of 16 rows, 10 of 32
    g = cascade.build_cascade_groups(bt, sl, 16, 16, 2)
    assert cascade.prefix_chunks(g, 16, 2) == 20
    assert cascade.prefix_chunks(g, 16, 2, chunk_rows=32) == 10


def test_chunk_rows_plan():
    # 32-row chunks once group rows x prefix tokens reach 2^21 (32 sharers x 8 heads x 8192 tokens)
    def groups(members, prefix):
        return cascade.CascadeGroups(members=torch.zeros((1, members), dtype=torch.int32),
                                     prefix_len=torch.zeros(1, dtype=torch.int32),
                                     row_prefix_len=torch.zeros(members, dtype=torch.int32), max_prefix_len=prefix,
                                     max_tail_len=1, total_tail_len=1)

    assert cascade.plan_chunk_rows(groups(16, 4096), 16, 2) == 16
    assert cascade.plan_chunk_rows(groups(32, 8192), 16, 2) == 32  # exactly 2^21
    assert cascade.plan_chunk_rows(groups(31, 8192), 16, 2) == 16
    assert cascade.plan_chunk_rows(groups(64, 16384), 16, 2) == 32
    assert cascade.plan_chunk_rows(groups(128, 16384), 16, 2) == 32
    assert cascade.plan_chunk_rows(groups(64, 8192), 16, 2) == 32


def test_prefix_split_plan():
    # about one prefix-role workgroup per CU, at least 16 prefix tiles per split
    assert cascade.plan_prefix_splits(1, 2, 8, 4096, 256) == 8     # 16 sharers x 4096
    assert cascade.plan_prefix_splits(1, 2, 16, 8192, 256) == 8    # 32 x 8192
    assert cascade.plan_prefix_splits(1, 2, 32, 16384, 256) == 4   # 64 x 16384
    assert cascade.plan_prefix_splits(1, 2, 64, 16384, 256) == 2   # 128 x 16384
    assert cascade.plan_prefix_splits(8, 8, 8, 4096, 256) == 1
    assert cascade.plan_prefix_splits(0, 2, 1, 0, 256) == 1
