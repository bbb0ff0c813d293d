"""GPU parity of the dim-major MFMA decode kernel against the CPU oracle.

Dim-major caches (``[blocks, kv_heads, head_dim, block_size]``, the
reference's ``kv_layout="dim_major"``, flashdec/paged_reference.py:19-125)
with 64- or 128-dim heads run the MFMA kernel that stages
K through LDS.  These cases cover what that kernel adds over the token-major
one: lengths that end inside a unit, a block or a quarter of a unit, head
blocks (G > 16), explicit and planned splits, strided views, non-finite
values past a row's end, table padding past the used range, streamed
against cached K/V loads (bit-identical), the fused current-token append
(output against the oracle, cache bytes bit-exact, inert rows), and hipGraph
replays with new inputs against eager calls.  Views whose strides or alignment
the kernel does not take run the generic kernel and must agree as well.
Tolerance: atol 2e-2 / rtol 1e-2 against the fp32 oracle.
"""

import math

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, make_paged_inputs, np32

pytestmark = pytest.mark.gpu

DTYPES = [torch.float16, torch.bfloat16]


def _fd():
    import flashdec_amd

    return flashdec_amd


def _oracle(q, k, v, table, lens, sm_scale=None):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy(), sm_scale=sm_scale,
                         kv_layout="dim_major")


def _workspace(b, hq, splits, head_dim=128):
    return (torch.empty((b, hq, splits, head_dim), device="cuda"), torch.empty((b, hq, splits), device="cuda"),
            torch.empty((b, hq, splits), device="cuda"))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize("lens", [[1, 7, 8, 9], [15, 16, 17, 31], [32, 33, 63, 64], [65, 100, 129, 0]])
def test_lengths_end_inside_units(lens, block_size, head_dim, dtype):
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, head_dim, block_size, dtype, kv_layout="dim_major",
                                           seed=21)
    out = _fd().decode(q, k, v, table, sl, block_size=block_size, kv_layout="dim_major")
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("block_size", [8, 16, 32])
@pytest.mark.parametrize(("hq", "hkv", "head_dim"), [(8, 8, 128), (4, 1, 128), (16, 2, 128), (32, 2, 128),
                                                     (40, 2, 128), (64, 1, 128), (14, 2, 64), (71, 1, 64),
                                                     (32, 32, 64)])
def test_group_sizes_and_head_blocks(hq, hkv, head_dim, block_size, dtype):
    q, k, v, table, sl = make_paged_inputs([300, 77, 1024], hq, hkv, head_dim, block_size, dtype,
                                           kv_layout="dim_major", seed=23)
    out = _fd().decode(q, k, v, table, sl, block_size=block_size, kv_layout="dim_major")
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("num_splits", [1, 3, 16, 40])
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("dtype", DTYPES)
def test_explicit_splits(num_splits, head_dim, dtype):
    lens = [2049, 1500, 33, 4096]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, head_dim, 32, dtype, kv_layout="dim_major", seed=25)
    out = torch.empty_like(q)
    _fd().paged_decode_attention_into(q, k, v, table, sl, out, block_size=32, kv_layout="dim_major",
                                      split_kv_workspace=_workspace(4, 16, 40, head_dim), num_splits=num_splits)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("block_size", [8, 16, 32])
def test_long_rows_planned_splits(block_size, head_dim, dtype):
    lens = [8192, 6000, 8191, 3]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, head_dim, block_size, dtype, kv_layout="dim_major",
                                           seed=27)
    out = _fd().decode(q, k, v, table, sl, block_size=block_size, kv_layout="dim_major")
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("block_size", [8, 16, 32])
def test_non_finite_values_past_row_end_are_masked(block_size, head_dim):
    lens = [45, 70, 5]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, head_dim, block_size, torch.bfloat16,
                                           kv_layout="dim_major", seed=29)
    ref = _oracle(q, k, v, table, sl)
    # every token slot past a row's length in its last block holds NaN / Inf
    for b, n in enumerate(lens):
        blk = int(table[b, (n - 1) // block_size])
        tail = n % block_size
        if tail:
            k[blk, :, :, tail:] = float("nan")
            v[blk, :, :, tail:] = float("inf")
    out = _fd().decode(q, k, v, table, sl, block_size=block_size, kv_layout="dim_major")
    assert_close_to_oracle(out, ref)


def test_table_padding_past_used_range_is_never_read():
    q, k, v, table, sl = make_paged_inputs([40, 90], 16, 2, 128, 16, torch.float16, kv_layout="dim_major",
                                           seed=31, table_width=64, pad_value=2**30)
    out = _fd().decode(q, k, v, table, sl, block_size=16, kv_layout="dim_major")
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("dtype", DTYPES)
def test_strided_dim_major_view(dtype):
    # a [blocks, head_dim, kv_heads, block_size] allocation viewed as dim-major:
    # head stride block_size, dim stride kv_heads * block_size
    q, k, v, table, sl = make_paged_inputs([130, 61], 16, 2, 128, 32, dtype, kv_layout="dim_major", seed=33)
    k_view = k.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    v_view = v.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3)
    assert not k_view.is_contiguous() and k_view.stride(3) == 1
    out = _fd().decode(q, k_view, v_view, table, sl, block_size=32, kv_layout="dim_major")
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


def test_misaligned_view_takes_the_generic_kernel_and_agrees():
    q, k, v, table, sl = make_paged_inputs([200, 33], 16, 2, 128, 16, torch.bfloat16, kv_layout="dim_major",
                                           seed=35)
    # the same values one element into a larger buffer: 2-byte aligned base
    kb = torch.empty(k.numel() + 1, dtype=k.dtype, device="cuda")
    vb = torch.empty(v.numel() + 1, dtype=v.dtype, device="cuda")
    k_off = kb[1:].view(k.shape)
    v_off = vb[1:].view(v.shape)
    k_off.copy_(k)
    v_off.copy_(v)
    out_fast = _fd().decode(q, k, v, table, sl, block_size=16, kv_layout="dim_major")
    out_gen = _fd().decode(q, k_off, v_off, table, sl, block_size=16, kv_layout="dim_major")
    ref = _oracle(q, k, v, table, sl)
    assert_close_to_oracle(out_fast, ref)
    assert_close_to_oracle(out_gen, ref)


@pytest.mark.parametrize("block_size", [8, 16, 32])
def test_kv_reuse_is_bit_identical(block_size):
    q, k, v, table, sl = make_paged_inputs([700, 1300, 64], 16, 2, 128, block_size, torch.bfloat16,
                                           kv_layout="dim_major", seed=37)
    a = _fd().decode(q, k, v, table, sl, block_size=block_size, kv_layout="dim_major")
    b = _fd().paged_decode_attention(q, k, v, table, sl, block_size=block_size, kv_layout="dim_major",
                                     kv_reuse=True)
    assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert_close_to_oracle(a, _oracle(q, k, v, table, sl))


def test_matches_token_major_layout_of_the_same_cache():
    # one cache in both layouts: both MFMA kernels agree with the oracle and,
    # within the tolerance, with each other
    q, k, v, table, sl = make_paged_inputs([511, 1025, 2048], 16, 2, 128, 32, torch.bfloat16, seed=39)
    kd = k.permute(0, 1, 3, 2).contiguous()
    vd = v.permute(0, 1, 3, 2).contiguous()
    tok = _fd().decode(q, k, v, table, sl, block_size=32)
    dim = _fd().decode(q, kd, vd, table, sl, block_size=32, kv_layout="dim_major")
    ref = oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), sl.cpu().numpy())
    assert_close_to_oracle(tok, ref)
    assert_close_to_oracle(dim, ref)
    assert np.abs(np32(tok) - np32(dim)).max() <= 2e-2


def _slots(table, lens, block_size):
    slots = []
    for b, n in enumerate(lens.tolist()):
        if n == 0:
            slots.append(-1)
            continue
        blk = int(table[b, (n - 1) // block_size])
        slots.append(blk * block_size + (n - 1) % block_size)
    return slots


@pytest.mark.parametrize("num_splits", [0, 1, 8])
@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("prior", [(0, 17, 31), (256, 193, 1000), (31, 63, 8)])
@pytest.mark.parametrize("block_size", [16, 32])
def test_fused_current_token_append(prior, num_splits, dtype, block_size):
    # the new token's K/V come from append_k/v (its cache slot holds NaN before
    # the call); the cache afterwards holds them at that slot, bit for bit
    lens_after = [p + 1 for p in prior]
    q, k, v, table, lens = make_paged_inputs(lens_after, 16, 2, 128, block_size, dtype, kv_layout="dim_major",
                                             seed=41)
    expected = _oracle(q, k, v, table, lens)
    slots = _slots(table, lens.cpu(), block_size)
    append_k = torch.empty((3, 2, 128), device="cuda", dtype=dtype)
    append_v = torch.empty_like(append_k)
    k_expected = k.clone()
    v_expected = v.clone()
    for b, s in enumerate(slots):
        blk, off = divmod(s, block_size)
        append_k[b] = k[blk, :, :, off]
        append_v[b] = v[blk, :, :, off]
        k[blk, :, :, off] = float("nan")
        v[blk, :, :, off] = float("nan")
    out = torch.empty_like(q)
    kwargs = {}
    if num_splits:
        kwargs = {"split_kv_workspace": _workspace(3, 16, 8), "num_splits": num_splits}
    _fd().paged_decode_attention_into(q, k, v, table, lens, out, block_size=block_size, kv_layout="dim_major",
                                      append_k=append_k, append_v=append_v,
                                      slot_mapping=torch.tensor(slots, device="cuda", dtype=torch.int64), **kwargs)
    assert_close_to_oracle(out, expected)
    assert torch.equal(k.view(torch.int16), k_expected.view(torch.int16))
    assert torch.equal(v.view(torch.int16), v_expected.view(torch.int16))


def test_fused_append_inert_rows():
    # slot -1 and seq_len 0 rows: zero output, no cache write
    q, k, v, table, lens = make_paged_inputs([40, 0, 70], 16, 2, 128, 32, torch.bfloat16, kv_layout="dim_major",
                                             seed=43)
    slots = _slots(table, lens.cpu(), 32)
    slots[2] = -1
    before_k, before_v = k.clone(), v.clone()
    append_k = torch.randn((3, 2, 128), device="cuda").to(torch.bfloat16)
    append_v = torch.randn((3, 2, 128), device="cuda").to(torch.bfloat16)
    blk, off = divmod(slots[0], 32)
    exp_k, exp_v = before_k.clone(), before_v.clone()
    exp_k[blk, :, :, off] = append_k[0]
    exp_v[blk, :, :, off] = append_v[0]
    out = torch.empty_like(q)
    _fd().paged_decode_attention_into(q, k, v, table, lens, out, block_size=32, kv_layout="dim_major",
                                      append_k=append_k, append_v=append_v,
                                      slot_mapping=torch.tensor(slots, device="cuda", dtype=torch.int32))
    assert torch.count_nonzero(out[1]) == 0 and torch.count_nonzero(out[2]) == 0
    assert torch.equal(k.view(torch.int16), exp_k.view(torch.int16))
    assert torch.equal(v.view(torch.int16), exp_v.view(torch.int16))
    ref = _oracle(q[:1], exp_k, exp_v, table[:1], lens[:1])
    assert_close_to_oracle(out[:1], ref)


@pytest.mark.parametrize("block_size", [8, 32])
def test_graph_replays_match_eager_with_new_inputs(block_size):
    # one captured dim-major launch replayed with new q and lengths written
    # into its buffers between replays (eager work and synchronisations in
    # between), each replay checked against an eager call on the same inputs
    q, k, v, table, lens = make_paged_inputs([600, 900, 64], 16, 2, 128, block_size, torch.bfloat16,
                                             kv_layout="dim_major", seed=47)
    fd = _fd()
    ws = _workspace(3, 16, 8)
    out = torch.empty_like(q)

    def call(o):
        fd.paged_decode_attention_into(q, k, v, table, lens, o, block_size=block_size, kv_layout="dim_major",
                                       split_kv_workspace=ws, num_splits=8)

    call(out)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        with torch.cuda.graph(graph):
            call(out)
    torch.cuda.current_stream().wait_stream(stream)
    gen = torch.Generator(device="cuda")
    gen.manual_seed(5)
    for step in range(3):
        q.copy_(torch.randn(q.shape, device="cuda", generator=gen).to(q.dtype))
        lens.copy_(torch.tensor([600 - 100 * step, 900 - step, 64 - 3 * step], device="cuda", dtype=lens.dtype))
        expected = torch.empty_like(q)
        call(expected)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), expected.view(torch.int16)), step
        assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def _fused_abi_call(q, k, v, table, lens, slots, append_k, append_v, block_size, num_splits):
    """fd_paged_decode on a dim-major cache with the fused append, through the C ABI (the Python
    API takes the fused append only for the reference's grouped shapes)."""
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    out = torch.empty_like(q)
    args = _lib.PagedDecodeArgs()
    pd._fill_common(args, q, k, v, pd._cache_strides(k, 3, 2), pd._cache_strides(v, 3, 2), table, lens, out,
                    k.shape[1], block_size, 1.0 / math.sqrt(q.shape[2]))
    args.num_blocks = k.shape[0]
    args.max_seq_len = int(lens.max())
    b, hq, d = q.shape
    ws = None
    if num_splits > 1:
        ws = (torch.empty((b, hq, num_splits, d), device="cuda"), torch.empty((b, hq, num_splits), device="cuda"),
              torch.empty((b, hq, num_splits), device="cuda"))
    pd._fill_workspace(args, *(ws or (None, None, None)), num_splits)
    pd._fill_append(args, append_k, append_v, torch.tensor(slots, device="cuda", dtype=torch.int64))
    _lib.paged_decode(args, _lib.current_stream_handle(q.device))
    return out


@pytest.mark.parametrize("num_splits", [1, 4])
@pytest.mark.parametrize(("hq", "head_dim", "block_size", "lens_after"), [
    # 8-token blocks: the appended token in each quarter of a 32-token unit (pos % 32 = 4, 10, 22, 24)
    (16, 128, 8, [101, 75, 55, 121]),
    (16, 64, 8, [101, 75, 55, 121]),
    # head_dim 64 on 16- and 32-token blocks
    (16, 64, 16, [33, 1, 200, 64]),
    (16, 64, 32, [33, 1, 200, 64]),
    # groups of 32 and 40 query heads per KV head: head blocks past the first splice the new token
    # from registers without storing it
    (64, 128, 32, [33, 300, 64, 2]),
    (80, 128, 32, [33, 300, 64, 2]),
    (80, 128, 8, [101, 75, 55, 121]),
])
def test_fused_append_dim_major_beyond_the_python_shapes(hq, head_dim, block_size, lens_after, num_splits):
    q, k, v, table, lens = make_paged_inputs(lens_after, hq, 2, head_dim, block_size, torch.bfloat16,
                                             kv_layout="dim_major", seed=53)
    expected = _oracle(q, k, v, table, lens)
    slots = _slots(table, lens.cpu(), block_size)
    append_k = torch.empty((len(lens_after), 2, head_dim), device="cuda", dtype=torch.bfloat16)
    append_v = torch.empty_like(append_k)
    k_expected, v_expected = k.clone(), v.clone()
    for b, s in enumerate(slots):
        blk, off = divmod(s, block_size)
        append_k[b] = k[blk, :, :, off]
        append_v[b] = v[blk, :, :, off]
        k[blk, :, :, off] = float("nan")
        v[blk, :, :, off] = float("nan")
    out = _fused_abi_call(q, k, v, table, lens, slots, append_k, append_v, block_size, num_splits)
    assert_close_to_oracle(out, expected)
    assert torch.equal(k.view(torch.int16), k_expected.view(torch.int16))
    assert torch.equal(v.view(torch.int16), v_expected.view(torch.int16))
