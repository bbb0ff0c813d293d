"""fd_paged_decode_noalloc against fd_paged_decode, through the C ABI.

The no-allocation entry point runs the same kernels with the split partials
in the library's per-GPU scratch array instead of a caller workspace, so its
output must equal fd_paged_decode's bit for bit (and the oracle within the
attention tolerance).  Two calls in a row, the second smaller, check that a
call never depends on what the previous one left in the scratch; the largest
launch the scratch holds runs too.  Calls on two streams with no ordering
between them each use their stream's own scratch slot, and a stream past the
slots is refused (that test runs last: it leaves every slot taken).
"""

import math

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, bits16, make_paged_inputs, np32

pytestmark = pytest.mark.gpu


def _args(q, k, v, table, lens, out, bs, hkv, splits, ws=None, append=None):
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    args = _lib.PagedDecodeArgs()
    pd._fill_common(args, q, k, v, pd._cache_strides(k, 2, 3), pd._cache_strides(v, 2, 3), table, lens, out, hkv, bs,
                    1.0 / math.sqrt(q.shape[2]))
    args.num_blocks = k.shape[0]
    args.max_seq_len = int(lens.max())
    if ws is not None:
        pd._fill_workspace(args, *ws, splits)
    else:
        args.num_splits = splits
    if append is not None:
        pd._fill_append(args, *append)
    return args


def _workspace(b, hq, splits, d):
    return (torch.empty((b, hq, splits, d), device="cuda"), torch.empty((b, hq, splits), device="cuda"),
            torch.empty((b, hq, splits), device="cuda"))


def _both(q, k, v, table, lens, bs, hkv, splits):
    """(fd_paged_decode output, fd_paged_decode_noalloc output) on the same inputs."""
    from flashdec_amd import _lib

    stream = _lib.current_stream_handle(q.device)
    ref = torch.empty_like(q)
    _lib.paged_decode(_args(q, k, v, table, lens, ref, bs, hkv, splits, _workspace(*q.shape[:2], splits, q.shape[2])),
                      stream)
    out = torch.full_like(q, float("nan"))
    _lib.paged_decode_noalloc(_args(q, k, v, table, lens, out, bs, hkv, splits), stream)
    torch.cuda.synchronize()
    return ref, out


def _oracle(q, k, v, table, lens):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy())


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_two_calls_in_a_row_match_the_workspace_entry_point(dtype):
    from flashdec_amd import _lib

    # C2's shape with the library's split plan, then a smaller ragged batch
    lens_big = [2048] * 8
    splits = _lib.paged_decode_plan(8, 16, 2, 128, 2048)
    assert splits > 1
    q, k, v, table, lens = make_paged_inputs(lens_big, 16, 2, 128, 32, dtype, seed=20260830 + 8 + 2048)
    ref, out = _both(q, k, v, table, lens, 32, 2, splits)
    assert torch.equal(ref, out)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))

    q, k, v, table, lens = make_paged_inputs([700, 1, 333], 16, 2, 128, 16, dtype, seed=5)
    ref, out = _both(q, k, v, table, lens, 16, 2, 8)
    assert torch.equal(ref, out)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_largest_launch_the_scratch_holds():
    from flashdec_amd import _lib

    b, hq, d = 8, 16, 128
    splits = _lib.NOALLOC_SCRATCH_BYTES // (b * hq * (d + 2) * 4)
    assert b * hq * splits * (d + 2) * 4 <= _lib.NOALLOC_SCRATCH_BYTES < b * hq * (splits + 1) * (d + 2) * 4
    q, k, v, table, lens = make_paged_inputs([4000, 37, 2048, 0, 1, 3999, 100, 64], hq, 2, d, 32, seed=17)
    ref, out = _both(q, k, v, table, lens, 32, 2, splits)
    assert torch.equal(ref, out)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))
    # and a smaller call right after it
    q, k, v, table, lens = make_paged_inputs([5, 90], 8, 2, 64, 8, seed=19)
    ref, out = _both(q, k, v, table, lens, 8, 2, 3)
    assert torch.equal(ref, out)
    assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_fused_append_writes_the_same_cache_bytes():
    from flashdec_amd import _lib

    bs, hkv, splits = 32, 2, 8
    lens_l = [517, 64, 1]
    q, k, v, table, lens = make_paged_inputs(lens_l, 16, hkv, 128, bs, seed=23)
    gen = torch.Generator().manual_seed(29)
    ak = torch.randn((3, hkv, 128), generator=gen).to(torch.bfloat16).cuda()
    av = torch.randn((3, hkv, 128), generator=gen).to(torch.bfloat16).cuda()
    slots = []
    for b, n in enumerate(lens_l):
        blk = int(table[b, (n - 1) // bs])
        slots.append(blk * bs + (n - 1) % bs)
    slot = torch.tensor(slots, device="cuda", dtype=torch.int64)
    for b, s in enumerate(slots):  # poison the slots: the kernels must take the new token from registers
        k[s // bs, :, s % bs] = float("nan")
        v[s // bs, :, s % bs] = float("nan")
    stream = _lib.current_stream_handle(q.device)
    k1, v1, k2, v2 = k.clone(), v.clone(), k.clone(), v.clone()
    ref = torch.empty_like(q)
    out = torch.empty_like(q)
    _lib.paged_decode(_args(q, k1, v1, table, lens, ref, bs, hkv, splits, _workspace(3, 16, splits, 128),
                            (ak, av, slot)), stream)
    _lib.paged_decode_noalloc(_args(q, k2, v2, table, lens, out, bs, hkv, splits, None, (ak, av, slot)), stream)
    torch.cuda.synchronize()
    assert torch.equal(ref, out)
    assert np.array_equal(bits16(k1), bits16(k2)) and np.array_equal(bits16(v1), bits16(v2))
    for b, s in enumerate(slots):
        assert torch.equal(k2[s // bs, :, s % bs], ak[b]) and torch.equal(v2[s // bs, :, s % bs], av[b])
    assert_close_to_oracle(out, _oracle(q, k2, v2, table, lens))


def test_captured_noalloc_launch_replays_like_the_workspace_entry_point():
    """fd_paged_decode_noalloc captured into a hipGraph (after fd_paged_decode_noalloc_prepare
    resolved the scratch address outside the capture): every replay, with new inputs copied
    into the captured buffers and eager work of the program's own between the replays, equals
    fd_paged_decode on the same inputs bit for bit, and the oracle within tolerance."""
    from flashdec_amd import _lib

    b, hq, hkv, d, bs = 8, 16, 2, 128, 32
    splits = _lib.paged_decode_plan(b, hq, hkv, d, 1024)
    assert splits > 1
    q, k, v, table, lens = make_paged_inputs([1024, 999, 1, 512, 1024, 77, 640, 1000], hq, hkv, d, bs, seed=41)
    out = torch.full_like(q, float("nan"))
    args = _args(q, k, v, table, lens, out, bs, hkv, splits)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.stream(side):
        stream = _lib.current_stream_handle(q.device)
        _lib.paged_decode_noalloc_prepare(stream)
        with torch.cuda.graph(graph, stream=side):
            _lib.paged_decode_noalloc(args, _lib.current_stream_handle(q.device))
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    ws = _workspace(b, hq, splits, d)
    for rep in range(3):
        print(f"noalloc graph replay {rep}", flush=True)
        q2, k2, v2, _, lens2 = make_paged_inputs([1024, 999, 1, 512, 1024, 77, 640, 1000], hq, hkv, d, bs,
                                                  seed=100 + rep)
        q.copy_(q2)
        k.copy_(k2)
        v.copy_(v2)
        lens.copy_(torch.clamp(lens2 - rep * 100, min=0))
        out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        ref = torch.empty_like(q)
        _lib.paged_decode(_args(q, k, v, table, lens, ref, bs, hkv, splits, ws), _lib.current_stream_handle(q.device))
        # the program's own eager work between the replays: a different noalloc launch
        _both(*make_paged_inputs([300, 5], 8, 2, 64, 16, seed=7 + rep), 16, 2, 4)
        torch.cuda.synchronize()
        assert torch.equal(ref, out), rep
        assert_close_to_oracle(out, _oracle(q, k, v, table, lens))


def test_prepare_needs_no_launch_and_is_idempotent():
    from flashdec_amd import _lib

    stream = _lib.current_stream_handle(torch.device("cuda"))
    for _ in range(3):
        _lib.paged_decode_noalloc_prepare(stream)
    _lib.paged_decode_noalloc_prepare(0)  # the null stream: the current device


def test_two_streams_without_ordering_use_their_own_slots():
    """Two streams enqueue no-allocation calls back to back with nothing ordering one stream
    against the other; every output equals fd_paged_decode's on the same inputs, bit for bit,
    because each stream's partials go to a scratch slot of its own."""
    from flashdec_amd import _lib

    splits = 16
    inputs = [make_paged_inputs([2048] * 8, 16, 2, 128, 32, seed=200 + i) for i in range(2)]
    refs = []
    for q, k, v, table, lens in inputs:
        ref = torch.empty_like(q)
        _lib.paged_decode(_args(q, k, v, table, lens, ref, 32, 2, splits, _workspace(8, 16, splits, 128)),
                          _lib.current_stream_handle(q.device))
        refs.append(ref)
    outs = [[torch.full_like(inputs[i][0], float("nan")) for _ in range(6)] for i in range(2)]
    torch.cuda.synchronize()
    streams = (torch.cuda.Stream(), torch.cuda.Stream())
    for rep in range(6):
        for i, side in enumerate(streams):
            q, k, v, table, lens = inputs[i]
            with torch.cuda.stream(side):
                _lib.paged_decode_noalloc(_args(q, k, v, table, lens, outs[i][rep], 32, 2, splits),
                                          _lib.current_stream_handle(q.device))
    torch.cuda.synchronize()
    for i in range(2):
        for rep in range(6):
            assert torch.equal(outs[i][rep], refs[i]), (i, rep)


def test_zz_a_stream_past_the_slots_is_refused_before_anything_runs():
    """New streams take the free scratch slots; the first stream past them gets the
    library's error (and its output is untouched), while a stream that owns a slot still runs.
    Runs last in this file: afterwards every slot of the GPU is taken."""
    from flashdec_amd import _lib

    q, k, v, table, lens = make_paged_inputs([512, 300], 8, 2, 128, 32, seed=9)
    owner = _lib.current_stream_handle(q.device)
    _lib.paged_decode_noalloc_prepare(owner)
    refused = None
    for n in range(48):  # more than torch's stream pool: its handles repeat
        side = torch.cuda.Stream()
        out = torch.full_like(q, float("nan"))
        with torch.cuda.stream(side):
            try:
                _lib.paged_decode_noalloc(_args(q, k, v, table, lens, out, 32, 2, 4),
                                          _lib.current_stream_handle(q.device))
            except RuntimeError as exc:
                refused = str(exc)
                torch.cuda.synchronize()
                assert torch.isnan(out).all()
                break
    assert refused is not None and "scratch slots" in refused, refused
    ref, out = _both(q, k, v, table, lens, 32, 2, 4)  # the owner's slot still serves it
    assert torch.equal(ref, out)
