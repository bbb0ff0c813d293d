"""GPU parity of the HIP paged-decode path against the CPU oracle.

Cases follow the reference's kernel tests (cysong2025/flashdec
tests/test_paged_decode.py): variable lengths over every head_dim / block
size / layout, GQA and MQA maps, zero-length rows, custom scale, strided NHD
views, unused invalid table entries, explicit split counts, fused current-
token append, and the unchecked vLLM launcher with graph-padding rows.
Tolerance: atol 2e-2 / rtol 1e-2 against the fp32 oracle; appended K/V
bytes bit-exact.
"""

import math

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, bits16, make_paged_inputs, np32

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _fd():
    import flashdec_amd

    return flashdec_amd


def _oracle(q, k, v, table, lens, sm_scale=None, kv_layout="token_major"):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy(), sm_scale=sm_scale,
                         kv_layout=kv_layout)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("kv_layout", ["token_major", "dim_major"])
def test_variable_lengths_match_oracle(kv_layout, block_size, head_dim, dtype):
    q, k, v, table, lens = make_paged_inputs([33, 1, 47], 4, 4, head_dim, block_size, dtype, kv_layout=kv_layout)
    out = _fd().decode(q, k, v, table, lens, block_size=block_size, kv_layout=kv_layout)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens, kv_layout=kv_layout))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("kv_layout", ["token_major", "dim_major"])
@pytest.mark.parametrize(("hq", "hkv", "head_dim"), [(32, 2, 64), (16, 1, 64), (16, 2, 128), (32, 2, 128),
                                                     (64, 2, 128)])
def test_gqa_and_mqa_maps(hq, hkv, head_dim, kv_layout, block_size, dtype):
    q, k, v, table, lens = make_paged_inputs([16, 31, 45], hq, hkv, head_dim, block_size, dtype,
                                             kv_layout=kv_layout, seed=7)
    out = _fd().decode(q, k, v, table, lens, block_size=block_size, kv_layout=kv_layout)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens, kv_layout=kv_layout))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
def test_zero_length_row_is_zero(dtype, head_dim):
    q, k, v, table, lens = make_paged_inputs([0, 17, 0], 8, 2, head_dim, 16, dtype)
    out = _fd().decode(q, k, v, table, lens)
    assert torch.count_nonzero(out[0]) == 0 and torch.count_nonzero(out[2]) == 0
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


@pytest.mark.parametrize("dtype", DTYPES)
def test_custom_scale(dtype):
    q, k, v, table, lens = make_paged_inputs([19, 70], 16, 2, 128, 32, dtype, seed=3)
    out = _fd().decode(q, k, v, table, lens, sm_scale=0.25)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens, sm_scale=0.25))


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_nhd_view(dtype):
    q, k, v, table, lens = make_paged_inputs([17, 31], 16, 2, 128, 16, dtype, seed=5)
    k_view = k.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    v_view = v.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    assert not k_view.is_contiguous()
    out = torch.empty_like(q)
    returned = _fd().paged_decode_attention_into(q, k_view, v_view, table, lens, out, block_size=16)
    assert returned is out
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_unused_invalid_table_entries_are_never_read():
    q, k, v, table, lens = make_paged_inputs([7], 2, 1, 64, 8, torch.float16, seed=9)
    wide = torch.full((1, 64), 2**30, device="cuda", dtype=torch.int32)
    wide[:, : table.shape[1]] = table
    out = _fd().decode(q, k, v, wide, lens, block_size=8)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


@pytest.mark.parametrize("num_splits", [2, 8, 16])
@pytest.mark.parametrize("dtype", DTYPES)
def test_explicit_split_kv(num_splits, dtype):
    q, k, v, table, lens = make_paged_inputs([257, 193], 16, 2, 128, 16, dtype, seed=11)
    ws = (torch.empty((2, 16, 16, 128), device="cuda"), torch.empty((2, 16, 16), device="cuda"),
          torch.empty((2, 16, 16), device="cuda"))
    out = torch.empty_like(q)
    _fd().paged_decode_attention_into(q, k, v, table, lens, out, block_size=16, split_kv_workspace=ws,
                                      num_splits=num_splits)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def _slots(table, lens, block_size):
    slots = []
    for b, n in enumerate(lens.tolist()):
        if n == 0:
            slots.append(-1)
            continue
        blk = int(table[b, (n - 1) // block_size])
        slots.append(blk * block_size + (n - 1) % block_size)
    return slots


@pytest.mark.parametrize("num_splits", [1, 8])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("prior", [(0, 17), (256, 193), (31, 63)])
@pytest.mark.parametrize("block_size", [16, 32])
def test_fused_current_token_append(prior, num_splits, dtype, block_size, head_dim=128):
    lens_after = [p + 1 for p in prior]
    q, k, v, table, lens = make_paged_inputs(lens_after, 16, 2, head_dim, block_size, dtype, seed=13)
    expected = _oracle(q, k, v, table, lens)  # cache already holding the new token
    slots = _slots(table, lens.cpu(), block_size)
    append_k = torch.empty((2, 2, head_dim), device="cuda", dtype=dtype)
    append_v = torch.empty_like(append_k)
    k_expected = k.clone()
    v_expected = v.clone()
    for b, s in enumerate(slots):
        blk, off = divmod(s, block_size)
        append_k[b] = k[blk, :, off]
        append_v[b] = v[blk, :, off]
        k[blk, :, off] = float("nan")  # must come from append_k, never from the cache
        v[blk, :, off] = float("nan")
    ws = (torch.empty((2, 16, 16, head_dim), device="cuda"), torch.empty((2, 16, 16), device="cuda"),
          torch.empty((2, 16, 16), device="cuda"))
    out = torch.empty_like(q)
    _fd().paged_decode_attention_into(q, k, v, table, lens, out, block_size=block_size, split_kv_workspace=ws,
                                      num_splits=num_splits, append_k=append_k, append_v=append_v,
                                      slot_mapping=torch.tensor(slots, device="cuda", dtype=torch.int64))
    assert_close_to_oracle(out, expected)
    assert np.array_equal(bits16(k), bits16(k_expected))
    assert np.array_equal(bits16(v), bits16(v_expected))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("num_splits", "cache_layout", "in_launch_merge"),
                         [(1, "NHD", False), (8, "NHD", False), (8, "HND", False), (8, "NHD", True),
                          (16, "HND", True)])
def test_vllm_launcher_full_cache_and_graph_padding(num_splits, cache_layout, in_launch_merge, dtype):
    """Rows: 2 active, 1 padding (slot -1) inside the grid, 1 beyond num_reqs."""
    bs = 16
    q_act, k, v, table_act, lens_act = make_paged_inputs([1, 257], 16, 2, 128, bs, dtype, seed=17)
    expected = _oracle(q_act, k, v, table_act, lens_act)
    slots = _slots(table_act, lens_act.cpu(), bs)
    nb = k.shape[0]
    full = torch.stack((k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)), dim=1).contiguous()  # [NB,2,bs,Hkv,D]
    expected_cache = full.clone()
    if cache_layout == "HND":
        storage = torch.empty((nb, 2, 2, bs, 128), device="cuda", dtype=dtype)
        cache = storage.permute(0, 1, 3, 2, 4)
        cache.copy_(full)
        assert not cache.is_contiguous()
    else:
        cache = full
    append_k = torch.randn((4, 2, 128), device="cuda").to(dtype)
    append_v = torch.randn((4, 2, 128), device="cuda").to(dtype)
    for b, s in enumerate(slots):
        blk, off = divmod(s, bs)
        append_k[b] = expected_cache[blk, 0, off]
        append_v[b] = expected_cache[blk, 1, off]
        cache[blk, :, off].zero_()
    q = torch.cat((q_act, torch.randn((2, 16, 128), device="cuda").to(dtype)))
    table = torch.cat((table_act, torch.zeros_like(table_act[:1])))
    lens_storage = torch.zeros((3, 2), device="cuda", dtype=torch.int32)
    lens_storage[:2, 1] = lens_act
    lens_storage[2, 1] = 17
    lens = lens_storage[:, 1]
    slot_mapping = torch.tensor([*slots, -1], device="cuda", dtype=torch.int64)
    ws = (torch.empty((4, 16, 16, 128), device="cuda"), torch.empty((4, 16, 16), device="cuda"),
          torch.empty((4, 16, 16), device="cuda"))
    out = torch.full_like(q, 37)
    from flashdec_amd.paged_decode import _vllm_paged_decode_attention_into

    counters = torch.zeros(8 * 64, device="cuda", dtype=torch.int32) if in_launch_merge else None
    returned = _vllm_paged_decode_attention_into(q, append_k, append_v, cache, table, lens, out, slot_mapping, *ws,
                                                 num_reqs=3, num_q_heads=16, num_kv_heads=2, head_dim=128,
                                                 block_size=bs, sm_scale=1.0 / math.sqrt(128),
                                                 num_splits=num_splits, split_counters=counters,
                                                 max_seq_len=int(lens_act.max()) if in_launch_merge else None)
    assert returned is out
    if counters is not None:
        assert torch.count_nonzero(counters) == 0
    assert_close_to_oracle(out[:2], expected)
    assert torch.count_nonzero(out[2]) == 0
    assert bool(torch.all(out[3] == 37))
    assert np.array_equal(bits16(cache), bits16(expected_cache))


@pytest.mark.parametrize("ctx", [1024, 2048])
def test_qwen_b8_shape_matches_oracle(ctx):
    """The headline shape: B8, Hq16/Hkv2, D128, bf16, bs32, all seq_lens = ctx."""
    q, k, v, table, lens = make_paged_inputs([ctx] * 8, 16, 2, 128, 32, torch.bfloat16, seed=20260830 + 8 + ctx)
    out = _fd().decode(q, k, v, table, lens, sm_scale=1.0 / math.sqrt(128))
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens, sm_scale=1.0 / math.sqrt(128)))


def test_ragged_long_context_matches_oracle():
    """Ragged long context (scaled to 8 rows): L ~ logU[128, 32768]."""
    rng = np.random.default_rng(1701)
    lens = [int(round(math.exp(x))) for x in rng.uniform(math.log(128), math.log(32768), size=8)]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, 128, 32, torch.bfloat16, seed=1701)
    out = _fd().decode(q, k, v, table, sl)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


def test_int64_tables_and_lengths():
    q, k, v, table, lens = make_paged_inputs([40, 5], 16, 2, 128, 32, torch.bfloat16, seed=23)
    out = _fd().decode(q, k, v, table.to(torch.int64), lens.to(torch.int64))
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_graph_capture_replays_match_eager():
    q, k, v, table, lens = make_paged_inputs([300, 1000, 64], 16, 2, 128, 32, torch.bfloat16, seed=29)
    fd = _fd()
    out = torch.empty_like(q)
    fd.paged_decode_attention_into(q, k, v, table, lens, out)
    eager = out.clone()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph):
            fd.paged_decode_attention_into(q, k, v, table, lens, out)
    torch.cuda.current_stream().wait_stream(stream)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


def test_in_launch_merge_matches_the_reducer_and_leaves_counters_zero():
    """C2 through the in-launch merge (split counters given): five calls in a row equal the
    reducer-kernel path bit for bit, and each leaves every arrival counter at zero."""
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    q, k, v, table, lens = make_paged_inputs([2048] * 8, 16, 2, 128, 32, torch.bfloat16, seed=31)
    splits = _lib.paged_decode_plan(8, 16, 2, 128, 2048)
    assert splits > 1
    ws = (torch.empty((8, 16, splits, 128), device="cuda"), torch.empty((8, 16, splits), device="cuda"),
          torch.empty((8, 16, splits), device="cuda"))
    counters = torch.zeros(8 * 2 * _lib.SPLIT_COUNTER_STRIDE, device="cuda", dtype=torch.int32)
    scale = 1.0 / math.sqrt(128)
    reducer = torch.empty_like(q)
    pd._decode_with_workspace(q, k, v, table, lens, reducer, scale, 32, splits, ws, k.shape[0])
    for _ in range(5):
        merged = torch.full_like(q, float("nan"))
        pd._decode_with_workspace(q, k, v, table, lens, merged, scale, 32, splits, ws, k.shape[0], counters=counters)
        torch.cuda.synchronize()
        assert torch.equal(merged, reducer)
        assert torch.count_nonzero(counters) == 0
    assert_close_to_oracle(merged, _oracle(q, k, v, table, lens))


@pytest.mark.parametrize("num_splits", [2, 16, 64, 100])
def test_explicit_splits_reducer_kernel_many_splits(num_splits):
    q, k, v, table, lens = make_paged_inputs([4000, 37, 0], 16, 2, 128, 32, torch.bfloat16, seed=37)
    ws = (torch.empty((3, 16, num_splits, 128), device="cuda"), torch.empty((3, 16, num_splits), device="cuda"),
          torch.empty((3, 16, num_splits), device="cuda"))
    out = torch.empty_like(q)
    _fd().paged_decode_attention_into(q, k, v, table, lens, out, split_kv_workspace=ws, num_splits=num_splits)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("num_splits", [2, 4, 5, 8, 16, 32, 40])
def test_packed_and_strided_workspaces_merge_to_the_same_bits(num_splits, head_dim):
    """The plain merge runs one kernel on a packed [B, Hq, S, D] workspace (addressing
    preloaded, empty rows told by their zero denominators) and another on any other
    workspace strides (reading each row's length and slot).  With NaN in both workspaces
    beforehand, zero-length rows and a padding slot, the two give the same bits; 2, 4, 8,
    16 and 32 splits take the whole-chunk kernel (immediate-offset loads), 40 the four-wave
    merge.  At 32 splits the whole chunk's one maximum and the other kernel's two chunks of
    16 (rescaled between them) round differently: there the two agree within a bf16 ulp."""
    dtype = torch.bfloat16
    hq, hkv, bs = 16, 2, 32
    lens_after = [0, 1, 37, 300, 1100, 65]
    q, k, v, table, lens = make_paged_inputs(lens_after, hq, hkv, head_dim, bs, dtype, seed=29)
    expected = _oracle(q, k, v, table, lens)
    slots = _slots(table, lens.cpu(), bs)
    slots[4] = -1  # a graph-padding row: zero output, nothing appended
    expected[4] = 0.0
    append_k = torch.empty((len(lens_after), hkv, head_dim), device="cuda", dtype=dtype)
    append_v = torch.empty_like(append_k)
    for b, s in enumerate(slots):
        if s >= 0:
            blk, off = divmod(s, bs)
            append_k[b] = k[blk, :, off]
            append_v[b] = v[blk, :, off]
    slot_t = torch.tensor(slots, device="cuda", dtype=torch.int64)
    nb = len(lens_after)

    from flashdec_amd.paged_decode import _decode_with_workspace

    def run(shape):
        # through the C ABI: the public API keeps the reference's refusal of a fused append at head_dim 64
        ws = (torch.full(shape, float("nan"), device="cuda"), torch.full(shape[:3], float("nan"), device="cuda"),
              torch.full(shape[:3], float("nan"), device="cuda"))
        out = torch.full_like(q, float("nan"))
        _decode_with_workspace(q, k, v, table, lens, out, 1.0 / math.sqrt(head_dim), bs, num_splits, ws, k.shape[0],
                               append=(append_k, append_v, slot_t))
        torch.cuda.synchronize()
        return out

    packed = run((nb, hq, num_splits, head_dim))
    strided = run((nb + 1, hq + 3, num_splits + 2, head_dim + 8))  # as0 != hq * as1: the length-reading kernel
    if num_splits <= 16 or num_splits > 32:
        assert torch.equal(packed, strided)
    else:
        # within one bf16 ulp of each other (2^-8 relative)
        torch.testing.assert_close(packed.float(), strided.float(), atol=1e-6, rtol=2.0**-7)
    assert torch.count_nonzero(packed[0]) == 0 and torch.count_nonzero(packed[4]) == 0
    assert_close_to_oracle(packed, expected)


@pytest.mark.parametrize("in_launch_merge", [False, True])
@pytest.mark.parametrize("hint", [1, 100, 700, 5000])
def test_max_seq_len_is_only_a_hint(hint, in_launch_merge):
    """Rows longer or shorter than the max_seq_len hint are attended in full."""
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    bs, splits = 16, 8
    q, k, v, table, lens = make_paged_inputs([700, 1, 333, 1500], 16, 2, 128, bs, torch.bfloat16, seed=41)
    ws = (torch.empty((4, 16, splits, 128), device="cuda"), torch.empty((4, 16, splits), device="cuda"),
          torch.empty((4, 16, splits), device="cuda"))
    counters = torch.zeros(4 * 2 * 64, device="cuda", dtype=torch.int32) if in_launch_merge else None
    out = torch.empty_like(q)
    args = _lib.PagedDecodeArgs()
    pd._fill_common(args, q, k, v, pd._cache_strides(k, 2, 3), pd._cache_strides(v, 2, 3), table, lens, out, 2, bs,
                    1.0 / math.sqrt(128))
    args.num_blocks = k.shape[0]
    args.max_seq_len = hint
    pd._fill_workspace(args, *ws, splits, counters)
    _lib.paged_decode(args, _lib.current_stream_handle(q.device))
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))
    if counters is not None:
        assert torch.count_nonzero(counters) == 0


def test_graph_replay_after_rows_grow_past_the_captured_hint():
    """vLLM's pattern: capture with the current max_seq_len, replay after rows grew in place."""
    from flashdec_amd.paged_decode import _vllm_paged_decode_attention_into

    bs, full_lens = 16, [900, 400, 1200, 64]
    q, k, v, table, lens_full = make_paged_inputs(full_lens, 16, 2, 128, bs, torch.bfloat16, seed=43)
    cache = torch.stack((k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)), dim=1).contiguous()
    append_k = cache[:, 0].new_empty((4, 2, 128))
    append_v = torch.empty_like(append_k)
    lens = torch.tensor([300, 100, 500, 10], device="cuda", dtype=torch.int32)
    slot_mapping = torch.empty(4, device="cuda", dtype=torch.int64)
    splits = 8
    ws = (torch.empty((4, 16, splits, 128), device="cuda"), torch.empty((4, 16, splits), device="cuda"),
          torch.empty((4, 16, splits), device="cuda"))
    out = torch.empty_like(q)

    def set_rows(lengths):
        lens.copy_(torch.tensor(lengths, device="cuda", dtype=torch.int32))
        sl = _slots(table, lens.cpu(), bs)
        slot_mapping.copy_(torch.tensor(sl, device="cuda", dtype=torch.int64))
        for b, s in enumerate(sl):  # the newest token's K/V, as vLLM's separate update leaves them
            blk, off = divmod(s, bs)
            append_k[b] = cache[blk, 0, off]
            append_v[b] = cache[blk, 1, off]

    def launch():
        _vllm_paged_decode_attention_into(q, append_k, append_v, cache, table, lens, out, slot_mapping, *ws,
                                          num_reqs=4, num_q_heads=16, num_kv_heads=2, head_dim=128, block_size=bs,
                                          sm_scale=1.0 / math.sqrt(128), num_splits=splits, max_seq_len=500)

    set_rows([300, 100, 500, 10])
    launch()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph):
            launch()
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    for lengths in ([301, 101, 501, 11], [900, 400, 1200, 64], [17, 399, 1100, 63]):
        set_rows(lengths)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


@pytest.mark.parametrize("num_splits", [None, 1, 3, 16])
@pytest.mark.parametrize("lens", [[2048] * 8, [1, 31, 32, 33, 700, 5000]])
def test_head_dim_64_long_rows_match_oracle(lens, num_splits):
    """head_dim 64 on the MFMA kernel (Qwen2.5-0.5B heads: 14 query, 2 KV), 32-token units on short
    splits and 16-token units on long ones.  The public API plans the splits itself at head_dim 64
    (the reference's split-KV path is head_dim 128 only), so explicit counts go through the C ABI."""
    from flashdec_amd.paged_decode import _decode_with_workspace

    q, k, v, table, sl = make_paged_inputs(lens, 14, 2, 64, 32, torch.bfloat16, seed=64 + len(lens))
    if num_splits is None:
        out = _fd().decode(q, k, v, table, sl)
    else:
        ws = None
        if num_splits > 1:
            ws = (torch.empty((len(lens), 14, num_splits, 64), device="cuda"),
                  torch.empty((len(lens), 14, num_splits), device="cuda"),
                  torch.empty((len(lens), 14, num_splits), device="cuda"))
        out = torch.empty_like(q)
        _decode_with_workspace(q, k, v, table, sl, out, 1.0 / 8.0, 32, num_splits, ws, k.shape[0])
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("num_splits", [1, 8])
@pytest.mark.parametrize("block_size", [16, 32])
def test_head_dim_64_fused_append_through_the_abi(num_splits, block_size):
    """The C ABI's fused append at head_dim 64 (the public API keeps the reference's refusal)."""
    from flashdec_amd.paged_decode import _decode_with_workspace

    prior = (0, 17, 256, 31)
    lens_after = [p + 1 for p in prior]
    q, k, v, table, lens = make_paged_inputs(lens_after, 16, 2, 64, block_size, torch.float16, seed=17)
    expected = _oracle(q, k, v, table, lens)
    slots = _slots(table, lens.cpu(), block_size)
    append_k = torch.empty((4, 2, 64), device="cuda", dtype=torch.float16)
    append_v = torch.empty_like(append_k)
    k_expected, v_expected = k.clone(), v.clone()
    for b, s in enumerate(slots):
        blk, off = divmod(s, block_size)
        append_k[b] = k[blk, :, off]
        append_v[b] = v[blk, :, off]
        k[blk, :, off] = float("nan")
        v[blk, :, off] = float("nan")
    ws = None
    if num_splits > 1:
        ws = (torch.empty((4, 16, num_splits, 64), device="cuda"), torch.empty((4, 16, num_splits), device="cuda"),
              torch.empty((4, 16, num_splits), device="cuda"))
    out = torch.empty_like(q)
    _decode_with_workspace(q, k, v, table, lens, out, 1.0 / 8.0, block_size, num_splits, ws, k.shape[0],
                           append=(append_k, append_v, torch.tensor(slots, device="cuda", dtype=torch.int64)))
    assert_close_to_oracle(out, expected)
    assert np.array_equal(bits16(k), bits16(k_expected))
    assert np.array_equal(bits16(v), bits16(v_expected))


@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize(("hq", "hkv", "head_dim"), [(32, 2, 128), (48, 2, 128), (24, 1, 64), (71, 1, 64),
                                                     (64, 1, 128), (34, 2, 128), (66, 2, 128), (40, 1, 64),
                                                     (17, 1, 64)])
def test_groups_above_16_heads_take_head_blocks(hq, hkv, head_dim, dtype, block_size):
    """More than 16 query heads per KV head: ceil(G / 32) head blocks of two 16-column blocks on the MFMA
    kernel (G 17 and 33: a last column block with a single head), every block size."""
    lens = [1, 100, 2048, 3000]
    q, k, v, table, sl = make_paged_inputs(lens, hq, hkv, head_dim, block_size, dtype, seed=hq + head_dim)
    out = _fd().decode(q, k, v, table, sl, block_size=block_size)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("block_size", [8, 32])
@pytest.mark.parametrize(("hq", "hkv", "head_dim"), [(40, 2, 128), (34, 1, 64), (80, 2, 128)])
@pytest.mark.parametrize("num_splits", [1, 5])
def test_groups_above_16_fused_append_written_once(num_splits, hq, hkv, head_dim, block_size):
    """Every head block attends to the appended token; the cache holds it exactly."""
    from flashdec_amd.paged_decode import _decode_with_workspace

    lens_after = [18, 257, 64]
    q, k, v, table, lens = make_paged_inputs(lens_after, hq, hkv, head_dim, block_size, torch.bfloat16, seed=41)
    expected = _oracle(q, k, v, table, lens)
    slots = _slots(table, lens.cpu(), block_size)
    ak = torch.empty((3, hkv, head_dim), device="cuda", dtype=torch.bfloat16)
    av = torch.empty_like(ak)
    k_expected, v_expected = k.clone(), v.clone()
    for b, s in enumerate(slots):
        blk, off = divmod(s, block_size)
        ak[b] = k[blk, :, off]
        av[b] = v[blk, :, off]
        k[blk, :, off] = float("nan")
        v[blk, :, off] = float("nan")
    ws = None
    if num_splits > 1:
        ws = (torch.empty((3, hq, num_splits, head_dim), device="cuda"),
              torch.empty((3, hq, num_splits), device="cuda"), torch.empty((3, hq, num_splits), device="cuda"))
    out = torch.empty_like(q)
    _decode_with_workspace(q, k, v, table, lens, out, 1.0 / math.sqrt(head_dim), block_size, num_splits, ws,
                           k.shape[0], append=(ak, av, torch.tensor(slots, device="cuda", dtype=torch.int64)))
    assert_close_to_oracle(out, expected)
    assert np.array_equal(bits16(k), bits16(k_expected))
    assert np.array_equal(bits16(v), bits16(v_expected))


def test_stream_handle_is_the_current_stream_on_every_stream_and_under_capture():
    """The launchers take torch's current stream through its raw-stream query: the same handle as
    torch.cuda.current_stream(...).cuda_stream on the default stream, on a side stream and under
    graph capture, and a decode captured there replays as the eager call computes it."""
    from flashdec_amd import _lib

    dev = torch.device("cuda", torch.cuda.current_device())
    assert _lib.current_stream_handle(dev) == torch.cuda.current_stream(dev).cuda_stream
    assert _lib.current_stream_handle(torch.device("cuda")) == torch.cuda.current_stream().cuda_stream
    side = torch.cuda.Stream(dev)
    with torch.cuda.stream(side):
        assert _lib.current_stream_handle(dev) == side.cuda_stream
    q, k, v, table, lens = make_paged_inputs([300, 37], 16, 2, 128, 32, torch.bfloat16, seed=21)
    ref = torch.empty_like(q)
    out = torch.empty_like(q)
    _fd().paged_decode_attention_into(q, k, v, table, lens, ref)
    side.wait_stream(torch.cuda.current_stream(dev))
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        _fd().paged_decode_attention_into(q, k, v, table, lens, out)  # the side stream's workspace, outside capture
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            assert _lib.current_stream_handle(dev) == side.cuda_stream
            _fd().paged_decode_attention_into(q, k, v, table, lens, out)
    torch.cuda.current_stream(dev).wait_stream(side)
    for _ in range(3):
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, ref)
    assert_close_to_oracle(ref, _oracle(q, k, v, table, lens))


def test_repeated_calls_reuse_arguments_but_follow_every_pointer():
    """paged_decode_attention_into keeps the last call's validated arguments when only data pointers change:
    alternating inputs, caller workspaces and fused-append rows of one shape, then another shape, must each
    give their own result."""
    from flashdec_amd.paged_decode import paged_decode_attention_into

    sets = [make_paged_inputs([300, 2048, 1], 16, 2, 128, 32, torch.bfloat16, seed=s) for s in (71, 72)]
    other = make_paged_inputs([100, 40], 8, 2, 64, 16, torch.bfloat16, seed=73)
    wss = [(torch.empty((3, 16, 4, 128), device="cuda"), torch.empty((3, 16, 4), device="cuda"),
            torch.empty((3, 16, 4), device="cuda")) for _ in range(2)]
    for rnd in range(3):
        for i, (q, k, v, table, sl) in enumerate(sets):
            out = torch.empty_like(q)
            paged_decode_attention_into(q, k, v, table, sl, out)
            assert_close_to_oracle(out, _oracle(q, k, v, table, sl))
            out2 = torch.empty_like(q)
            paged_decode_attention_into(q, k, v, table, sl, out2, split_kv_workspace=wss[(i + rnd) % 2], num_splits=4)
            assert_close_to_oracle(out2, _oracle(q, k, v, table, sl))
        q, k, v, table, sl = other
        out = torch.empty_like(q)
        paged_decode_attention_into(q, k, v, table, sl, out)
        assert_close_to_oracle(out, _oracle(q, k, v, table, sl))
    # fused append: each call's rows land at each call's slots
    for s in (74, 75):
        q, k, v, table, sl = make_paged_inputs([64, 257], 16, 2, 128, 32, torch.bfloat16, seed=s)
        expected = _oracle(q, k, v, table, sl)
        slots = torch.tensor(_slots(table, sl.cpu(), 32), device="cuda", dtype=torch.int64)
        blk, off = slots // 32, slots % 32
        ak, av = k[blk, :, off].clone(), v[blk, :, off].clone()
        k_expected, v_expected = k.clone(), v.clone()
        k[blk, :, off] = float("nan")
        v[blk, :, off] = float("nan")
        out = torch.empty_like(q)
        paged_decode_attention_into(q, k, v, table, sl, out, append_k=ak, append_v=av, slot_mapping=slots)
        assert_close_to_oracle(out, expected)
        assert np.array_equal(bits16(k), bits16(k_expected))
        assert np.array_equal(bits16(v), bits16(v_expected))
