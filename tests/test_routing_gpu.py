"""Which kernels each public path launches, from the library's launch record.

The parity tests elsewhere check results; these check that each path takes
the kernel the design says it does (a wrong route would still pass parity on
a kernel that happens to be correct, and then the performance claims would be
about another kernel).  No counterpart in the reference.  Every call is also
checked against the oracle, so a routed call is a correct one.
"""

import math

import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, make_paged_inputs, np32

pytestmark = pytest.mark.gpu

MFMA = "fd::decode_mfma_kernel<__bf16, {bs}, {fuse}, {merge}, {unit}, {nt}, {d}, {ncb}>"


def mfma(bs=32, fuse=0, merge="false", unit=32, nt="true", d=128, ncb=1):
    return MFMA.format(bs=bs, fuse=fuse, merge=merge, unit=unit, nt=nt, d=d, ncb=ncb)


@pytest.fixture(autouse=True)
def record():
    from flashdec_amd import _lib

    _lib.record_launches(True)
    yield _lib
    _lib.record_launches(False)


def _oracle(q, k, v, table, lens, kv_layout="token_major"):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy(), kv_layout=kv_layout)


def test_c2_shape_row_kernel_and_preloaded_reducer(record):
    import flashdec_amd as fd

    q, k, v, table, sl = make_paged_inputs([2048] * 8, 16, 2, 128, 32, seed=1)
    out = fd.decode(q, k, v, table, sl)
    # an output in row order: the reducer takes its pointer preloaded and no strides; the
    # library's contiguous workspace with 16 splits: immediate-offset partial loads
    assert record.last_launch() == [mfma(unit=32), "fd::split_reduce_pre_kernel<__bf16, 128, 1, true, 16>"]
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("d", [64, 128])
def test_output_view_out_of_row_order_takes_the_strided_store(d, record):
    """A packed split workspace with an output whose rows are not in order (a view with a
    wider head stride, and a transposed view): the preloaded reducer reads the output
    strides, and every row lands where the view puts it."""
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    q, k, v, table, sl = make_paged_inputs([2048, 900, 0, 1500], 16, 2, d, 32, seed=4)
    splits = _lib.paged_decode_plan(4, 16, 2, d, 2048)
    assert splits > 1
    ws = (torch.empty((4, 16, splits, d), device="cuda"), torch.empty((4, 16, splits), device="cuda"),
          torch.empty((4, 16, splits), device="cuda"))
    expected = _oracle(q, k, v, table, sl)
    wide = torch.full((4, 16, d + 24), float("nan"), device="cuda", dtype=q.dtype)
    transposed = torch.full((16, 4, d), float("nan"), device="cuda", dtype=q.dtype).transpose(0, 1)
    for out in (wide[..., :d], transposed):
        pd._decode_with_workspace(q, k, v, table, sl, out, 1.0 / math.sqrt(d), 32, splits, ws, k.shape[0])
        torch.cuda.synchronize()
        assert record.last_launch()[1] == f"fd::split_reduce_pre_kernel<__bf16, {d}, 1, false, 0>"
        assert_close_to_oracle(out, expected)
    assert torch.isnan(wide[..., d:]).all()  # nothing written past the view


def test_misaligned_whole_chunk_views_take_the_general_merge_with_the_same_bits(record):
    """The whole-chunk reducer at head_dim 128 loads 8 bytes per split and stores 4 bytes per
    lane.  An output in row order that starts 2 bytes into its buffer, or a workspace that
    starts 4 bytes into its buffer, takes the general row-order merge instead, and every
    layout gives the aligned one's bits."""
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    d = 128
    q, k, v, table, sl = make_paged_inputs([2048, 900, 0, 1500], 16, 2, d, 32, seed=9)
    splits = _lib.paged_decode_plan(4, 16, 2, d, 2048)
    assert splits == 16
    n_acc, n_st = 4 * 16 * splits * d, 4 * 16 * splits

    def workspace(shift):
        flat = torch.full((n_acc + 2 * n_st + shift,), float("nan"), device="cuda")
        acc = flat[shift:shift + n_acc].view(4, 16, splits, d)
        mx = flat[shift + n_acc:shift + n_acc + n_st].view(4, 16, splits)
        sm = flat[shift + n_acc + n_st:shift + n_acc + 2 * n_st].view(4, 16, splits)
        return acc, mx, sm

    outs = {}
    for name, out_shift, ws_shift in (("aligned", 0, 0), ("output", 1, 0), ("workspace", 0, 1)):
        buf = torch.full((4 * 16 * d + out_shift,), float("nan"), device="cuda", dtype=q.dtype)
        out = buf[out_shift:].view(4, 16, d)
        ws = workspace(ws_shift)
        pd._decode_with_workspace(q, k, v, table, sl, out, 1.0 / math.sqrt(d), 32, splits, ws, k.shape[0])
        torch.cuda.synchronize()
        fch = 16 if name == "aligned" else 0
        assert record.last_launch()[1] == f"fd::split_reduce_pre_kernel<__bf16, {d}, 1, true, {fch}>", name
        outs[name] = out.clone()
    assert_close_to_oracle(outs["aligned"], _oracle(q, k, v, table, sl))
    for name in ("output", "workspace"):
        assert torch.equal(outs[name], outs["aligned"]), name


@pytest.mark.parametrize(("hq", "d", "ncb"), [(16, 128, 1), (64, 128, 2), (40, 64, 2)])
@pytest.mark.parametrize("kv_reuse", [False, True])
def test_long_rows_16_token_units_and_column_blocks(hq, d, ncb, kv_reuse, record):
    import flashdec_amd as fd

    # 8 rows, 16 splits of 16 tiles: 16-token units
    q, k, v, table, sl = make_paged_inputs([8192] * 4 + [6000] * 4, hq, 2, d, 32, seed=2)
    out = fd.decode(q, k, v, table, sl, kv_reuse=kv_reuse)
    names = record.last_launch()
    assert names[0] == mfma(unit=16, d=d, ncb=ncb, nt="false" if kv_reuse else "true"), names
    assert names[1].startswith(f"fd::split_reduce_pre_kernel<__bf16, {d}, "), names
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


def test_ragged_flag_takes_per_row_splits(record):
    import flashdec_amd as fd

    q, k, v, table, sl = make_paged_inputs([4000, 10, 250, 0, 1500, 33, 7, 900, 60], 16, 2, 128, 32, seed=3)
    out = fd.decode(q, k, v, table, sl, ragged=True)
    names = record.last_launch()
    assert names[0] == "fd::decode_balanced_kernel<__bf16, 32, true>", names
    assert names[1].startswith("fd::split_reduce_kernel<__bf16, 128, 2, "), names
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("d", [64, 128])
def test_dim_major_mfma_kernel(d, record):
    import flashdec_amd as fd

    q, k, v, table, sl = make_paged_inputs([4096, 77], 16, 2, d, 16, seed=4, kv_layout="dim_major")
    out = fd.decode(q, k, v, table, sl, kv_layout="dim_major")
    names = record.last_launch()
    assert names[0] == f"fd::decode_dm_kernel<__bf16, 16, true, {d}, 0>", names
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl, kv_layout="dim_major"))


def test_misaligned_views_take_the_generic_kernel(record):
    import flashdec_amd as fd

    q, k, v, table, sl = make_paged_inputs([300, 31], 16, 2, 128, 16, seed=5)
    # the same values one element into a larger buffer: a 2-byte aligned base
    kb = torch.empty(k.numel() + 1, dtype=k.dtype, device="cuda")
    vb = torch.empty(v.numel() + 1, dtype=v.dtype, device="cuda")
    k_off, v_off = kb[1:].view(k.shape), vb[1:].view(v.shape)
    k_off.copy_(k)
    v_off.copy_(v)
    out = fd.decode(q, k_off, v_off, table, sl)
    names = record.last_launch()
    assert names[0] == "fd::decode_generic_kernel<__bf16, 128>", names
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize(("kv_reuse", "nt"), [(True, "false"), (False, "true")])
def test_cascade_launch_and_reducer(kv_reuse, nt, record):
    from flashdec_amd import cascade
    from tests.test_cascade_gpu import make_prefix_inputs

    groups = [(512, [5, 300, 77, 1, 40, 700, 12, 64] * 8)]
    q, k, v, table, sl, _ = make_prefix_inputs(groups, [], 16, 2, 32, torch.bfloat16, seed=6)
    g = cascade.build_cascade_groups(table, sl, 32, 16, 2)
    out = cascade.paged_decode_attention_cascade(q, k, v, table, sl, groups=g, kv_reuse=kv_reuse)
    names = record.last_launch()
    # 64 rows on a 16384-token prefix: 32-row chunks (two column blocks per wave)
    # the library's packed workspace: the cascade merge with preloaded arguments
    assert names == [f"fd::cascade_decode_kernel<__bf16, 32, 16, {nt}, 2>",
                     "fd::split_reduce_cascade_pre_kernel<__bf16, 128>"], names
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


def test_in_launch_merge_is_one_dispatch(record):
    from flashdec_amd import _lib
    from flashdec_amd.paged_decode import _decode_with_workspace

    q, k, v, table, sl = make_paged_inputs([2048] * 8, 16, 2, 128, 32, seed=7)
    ws = (torch.empty((8, 16, 16, 128), device="cuda"), torch.empty((8, 16, 16), device="cuda"),
          torch.empty((8, 16, 16), device="cuda"))
    counters = torch.zeros(8 * 2 * _lib.SPLIT_COUNTER_STRIDE, device="cuda", dtype=torch.int32)
    out = torch.empty_like(q)
    _decode_with_workspace(q, k, v, table, sl, out, 1.0 / math.sqrt(128), 32, 16, ws, k.shape[0], counters=counters)
    assert record.last_launch() == [mfma(unit=32, merge="true")]
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))
    assert torch.count_nonzero(counters) == 0


def test_fused_rope_in_the_decode_launch(record):
    from flashdec_amd.paged_decode import _decode_with_workspace

    q, k, v, table, sl = make_paged_inputs([4096] * 4, 16, 2, 128, 32, seed=8)
    ak = torch.zeros((4, 2, 128), device="cuda", dtype=torch.bfloat16)
    pos = sl.to(torch.int64) - 1
    slots = table.gather(1, (pos // 32).view(-1, 1)).view(-1).to(torch.int64) * 32 + pos % 32
    ws = (torch.empty((4, 16, 8, 128), device="cuda"), torch.empty((4, 16, 8), device="cuda"),
          torch.empty((4, 16, 8), device="cuda"))
    out = torch.empty_like(q)
    _decode_with_workspace(q, k, v, table, sl, out, None, 32, 8, ws, k.shape[0], append=(ak, ak, slots),
                           rope=(128, 1e6))
    names = record.last_launch()
    assert names[0] == mfma(fuse=2, unit=16), names


def test_rope_append_and_kv_append_kernels(record):
    from flashdec_amd import _kv_append, fused_rope_kv_append

    q, k, v, table, sl = make_paged_inputs([64, 40], 16, 2, 128, 32, seed=9)
    ak = torch.randn((2, 2, 128), device="cuda").to(torch.bfloat16)
    blk = table[:, 0].to(torch.int64)
    off = torch.tensor([3, 5], device="cuda", dtype=torch.int64)
    fused_rope_kv_append(q, ak, ak, k, v, blk, off, off, base=1e6)
    assert record.last_launch() == ["fd::rope_append_vec_kernel<__bf16>"]
    _kv_append.cuda_kv_append(k, v, blk, off, ak, ak)
    assert record.last_launch() == ["fd::kv_append_kernel<__bf16>"]


def test_eager_engine_layers_after_the_first_take_one_launch(record):
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine

    cache = PagedKVCache(num_layers=3, num_kv_heads=2, head_dim=128, block_size=32, max_blocks=64,
                         dtype=torch.bfloat16, device="cuda")
    engine = DecodeEngine(cache)
    for rid in ("a", "b"):
        engine.add_request(rid)
    engine.admit()
    tx = engine.begin_step(["a", "b"])
    g = torch.Generator().manual_seed(10)
    launched = []
    for layer in range(3):
        q = torch.randn((2, 16, 128), generator=g).to(torch.bfloat16).cuda()
        kv = torch.randn((2, 2, 128), generator=g).to(torch.bfloat16).cuda()
        engine.step_layer(tx, layer, q, kv, kv, base=1e6)
        launched.append(record.last_launch())
    engine.commit_step(tx)
    # layer 0: the RoPE + append kernel, then the decode (the last call); later layers: one fused decode call
    assert launched[0][0].startswith("fd::decode_mfma_kernel<__bf16, 32, 0, false, ")
    for names in launched[1:]:
        assert names[0].startswith("fd::decode_mfma_kernel<__bf16, 32, 2, false, "), names
