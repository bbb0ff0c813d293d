"""CPU checks of the library's split plan (``fd_paged_decode_plan``).

Without a GPU the library plans for 256 CUs (MI355X's count).  Each case is
worked by hand from the plan's rules: one workgroup per CU at least
(ceil(256 / pairs)), the balance bound from the batch's total length, whole
waves of 256 workgroups where a count up to twice the start gives them, else
the count from the balance bound up whose last wave is fullest (ties: fewer
workgroups), then the cap of one 16-token unit per wave (one split where that
cap is two).  No counterpart in the reference, whose split count is per
launch (flashdec/kernels/paged_decode.py:408-411).
"""

import pytest

CASES = [
    # (num_seqs, Hq, Hkv, D, max_len, total_len) -> splits
    # C2: 16 pairs, 16 splits = 256 workgroups
    ((8, 16, 2, 128, 2048, 0), 16),
    # ctx1024: 16 pairs want 16, the cap (2 * 32 tiles / 8 waves) gives 8
    ((8, 16, 2, 128, 1024, 0), 8),
    # C5 layer: 128 pairs, 2 splits
    ((64, 16, 2, 128, 8192, 64 * 8192), 2),
    # B16 x 8192, G8: 32 pairs, 8 splits
    ((16, 16, 2, 128, 8192, 16 * 8192), 8),
    # B16 x 8192, G32: one head block of 32 heads, so 32 pairs, 8 splits
    ((16, 64, 2, 128, 8192, 16 * 8192), 8),
    # MQA G71 D64: 3 head blocks, 48 pairs.  Start 6 (288 workgroups); no
    # count in [6, 12] fills whole waves; from the balance bound 5 up, 5
    # (240 of 256) and 10 (480 of 512) are fullest: 5
    ((16, 71, 1, 64, 8192, 16 * 8192), 5),
    # 6 pairs of 32768 tokens: start 43 (258 workgroups, a second wave of 2);
    # 85 splits fill 510 of 512
    ((3, 16, 2, 128, 32768, 3 * 32768), 85),
    # C1's shape: 8 pairs want 32, the cap (2 * 16 tiles / 8 waves) gives 4
    ((4, 8, 2, 64, 512, 4 * 512), 4),
    # rows of 8 tiles: the cap would be 2 (one unit per wave); one split, no reducer
    ((8, 16, 2, 128, 256, 8 * 256), 1),
    ((64, 16, 2, 128, 256, 64 * 256), 1),
    # 12 tiles: cap 3 (one 32-token unit per wave of 4)
    ((8, 16, 2, 128, 384, 8 * 384), 3),
]


@pytest.mark.parametrize(("shape", "splits"), CASES)
def test_plan_cases(shape, splits):
    from flashdec_amd import _lib

    assert _lib.paged_decode_plan(*shape) == splits


def test_plan_fills_whole_waves_when_it_can():
    # every pair count that divides 256 gets a grid of whole waves
    from flashdec_amd import _lib

    for pairs_b in (1, 2, 4, 8, 16, 32, 64, 128):
        s = _lib.paged_decode_plan(pairs_b, 16, 2, 128, 65536, pairs_b * 65536)
        assert (pairs_b * 2 * s) % 256 == 0, (pairs_b, s)


# Cascade tail splits (flashdec_amd.cascade.plan_tail_splits): the fewest in
# [ceil(plan / 2), plan] that make prefix-role plus tail-role workgroups whole
# waves of 256, else the tails' own plan.  Tails ~ U{1..512} on the bench's
# shared-prefix sizes: (rows, prefix-role workgroups, max tail, total tail).
TAIL_CASES = [
    # 64 rows on 16384 tokens: 256 prefix-role workgroups, 128 pairs; plan 4, 2 gives 512
    ((64, 256, 512, 64 * 256), 4, 2),
    # 128 rows: 256 + 256 per split; plan 2, 1 gives 512
    ((128, 256, 512, 128 * 256), 2, 1),
    # 32 rows: 256 + 64 per split; plan 4, and only 4 in [2, 4] gives whole waves
    ((32, 256, 512, 32 * 256), 4, 4),
    # 16 rows: 128 + 32 per split; 4 gives 256
    ((16, 128, 512, 16 * 256), 4, 4),
    # 8 rows of 8192-token tails beside 240 prefix-role workgroups: 1 split would fill the
    # wave but holds 8192 tokens a workgroup; none in [8, 16] does, so the plan (16)
    ((8, 240, 8192, 8 * 8192), 16, 16),
]


@pytest.mark.parametrize(("shape", "plan", "splits"), TAIL_CASES)
def test_cascade_tail_split_cases(shape, plan, splits):
    from types import SimpleNamespace

    from flashdec_amd import _lib, cascade

    rows, prefix_blocks, max_tail, total_tail = shape
    groups = SimpleNamespace(max_tail_len=max_tail, total_tail_len=total_tail)
    assert _lib.paged_decode_plan(rows, 16, 2, 128, max_tail, total_tail) == plan
    assert cascade.plan_tail_splits(rows, 16, 2, 128, groups, prefix_blocks, 256) == splits


# Cascade prefix and tail splits together (flashdec_amd.cascade.plan_cascade_splits), worked by
# hand for 256 CUs, Hq16/Hkv2/D128, tails ~ U{1..512} (max 512 tokens, mean 256), one group:
# (sharers, prefix tokens, chunk rows) -> (prefix splits, tail splits)
CASCADE_CASES = [
    # 8 chunks x 2 KV heads = 16 prefix units; 3/4 of the CUs: 192 // 16 = 12 splits of ceil(128 / 12)
    # = 11 tiles; the tails' plan is 4, and 32 pairs x 2 fill the wave: 192 + 64 = 256
    ((16, 4096, 16), (12, 2)),
    # 32-row chunks: 8 chunks x 2 = 16 units -> 12 splits of 22 tiles; one tail split (16 tiles, no
    # longer than a prefix-role workgroup) fills the wave: 192 + 64 = 256
    ((32, 8192, 32), (12, 1)),
    # 16 chunks x 2 = 32 units: 192 // 32 = 6 splits leave 64 CUs that 128 pairs cannot fill in whole
    # waves; one workgroup per CU instead: 8 splits, 2 tail splits -> 256 + 256
    ((64, 16384, 32), (8, 2)),
    # 64 units: 3 splits leave no whole wave; 4 splits + 1 tail split -> 256 + 256
    ((128, 16384, 32), (4, 1)),
]


@pytest.mark.parametrize(("shape", "splits"), CASCADE_CASES)
def test_cascade_split_plan_cases(shape, splits):
    from types import SimpleNamespace

    from flashdec_amd import cascade

    sharers, prefix, rows = shape
    groups = SimpleNamespace(num_groups=1, max_members=sharers, max_prefix_len=prefix, max_tail_len=512,
                             total_tail_len=sharers * 256)
    assert cascade.plan_chunk_rows(groups, 16, 2) == rows
    chunks = cascade.prefix_chunks(groups, 16, 2, rows)
    assert cascade.plan_cascade_splits(sharers, 16, 2, 128, groups, chunks, 256) == splits
