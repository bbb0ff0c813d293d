"""Views whose base is not 16-byte aligned: outputs, split workspaces and q.

The reference takes any strided ``out``, ``q`` and split workspace
(flashdec/kernels/paged_decode.py:28-121, 330-642 index every tensor through
its strides; its validation checks shapes, dtypes and devices only, :645-725,
1076-1096), so a caller may hand over a view that starts one element into a
buffer.  The MFMA kernel stores an output row's eight elements and a split
partial's dims as 16-byte vectors, and reads q as 16-byte vectors: each case
here runs on a view one element (2 or 4 bytes) past an aligned base and is
checked against the oracle, and the launch record names the kernel it took.
"""

import math

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, make_paged_inputs, np32

pytestmark = pytest.mark.gpu


def _oracle(q, k, v, table, lens):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy())


def _shifted(shape, dtype, fill=float("nan")):
    """A contiguous view of ``shape`` one element past a 256-byte aligned buffer start."""
    n = math.prod(shape)
    buf = torch.full((n + 8,), fill, device="cuda", dtype=dtype)
    view = buf[1:1 + n].view(shape)
    assert view.data_ptr() % 16 != 0
    return view


@pytest.fixture
def record():
    from flashdec_amd import _lib

    _lib.record_launches(True)
    yield _lib
    _lib.record_launches(False)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("lens", [[2048] * 4, [40, 7, 120], [600, 1, 0, 333]])
@pytest.mark.parametrize("head_dim", [64, 128])
def test_unaligned_out(lens, head_dim, dtype, record):
    import flashdec_amd as fd

    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, head_dim, 32, dtype, seed=len(lens) + head_dim)
    out = _shifted(tuple(q.shape), dtype)
    fd.paged_decode_attention_into(q, k, v, table, sl, out)
    assert record.last_launch()[0].startswith("fd::decode_mfma_kernel<"), record.last_launch()
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("num_splits", [1, 8])
def test_unaligned_out_with_fused_append(num_splits, record):
    import flashdec_amd as fd

    lens = [300, 65, 1024]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, 128, 16, torch.bfloat16, seed=77)
    expected = _oracle(q, k, v, table, sl)
    append_k = torch.empty((3, 2, 128), device="cuda", dtype=torch.bfloat16)
    append_v = torch.empty_like(append_k)
    slots = []
    for b, n in enumerate(lens):
        blk, off = int(table[b, (n - 1) // 16]), (n - 1) % 16
        append_k[b], append_v[b] = k[blk, :, off], v[blk, :, off]
        k[blk, :, off] = float("nan")
        v[blk, :, off] = float("nan")
        slots.append(blk * 16 + off)
    out = _shifted((3, 16, 128), torch.bfloat16)
    ws = None
    if num_splits > 1:
        ws = (torch.empty((3, 16, num_splits, 128), device="cuda"), torch.empty((3, 16, num_splits), device="cuda"),
              torch.empty((3, 16, num_splits), device="cuda"))
    fd.paged_decode_attention_into(q, k, v, table, sl, out, split_kv_workspace=ws, num_splits=num_splits,
                                   append_k=append_k, append_v=append_v,
                                   slot_mapping=torch.tensor(slots, device="cuda", dtype=torch.int64))
    assert record.last_launch()[0].startswith("fd::decode_mfma_kernel<__bf16, 16, 1, "), record.last_launch()
    assert_close_to_oracle(out, expected)


@pytest.mark.parametrize("num_splits", [4, 40])
def test_unaligned_split_workspace(num_splits, record):
    import flashdec_amd as fd

    q, k, v, table, sl = make_paged_inputs([3000, 900, 17], 16, 2, 128, 32, torch.bfloat16, seed=5)
    ws = (_shifted((3, 16, num_splits, 128), torch.float32), _shifted((3, 16, num_splits), torch.float32),
          _shifted((3, 16, num_splits), torch.float32))
    out = torch.empty_like(q)
    fd.paged_decode_attention_into(q, k, v, table, sl, out, split_kv_workspace=ws, num_splits=num_splits)
    names = record.last_launch()
    assert names[0].startswith("fd::decode_mfma_kernel<") and len(names) == 2, names
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


def test_unaligned_out_with_in_launch_merge(record):
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    q, k, v, table, sl = make_paged_inputs([2048] * 8, 16, 2, 128, 32, torch.bfloat16, seed=8)
    splits = 16
    ws = (torch.empty((8, 16, splits, 128), device="cuda"), torch.empty((8, 16, splits), device="cuda"),
          torch.empty((8, 16, splits), device="cuda"))
    counters = torch.zeros(8 * 2 * _lib.SPLIT_COUNTER_STRIDE, device="cuda", dtype=torch.int32)
    out = _shifted((8, 16, 128), torch.bfloat16)
    pd._decode_with_workspace(q, k, v, table, sl, out, 1.0 / math.sqrt(128), 32, splits, ws, k.shape[0],
                              counters=counters)
    assert record.last_launch() == ["fd::decode_mfma_kernel<__bf16, 32, 0, true, 32, true, 128, 1>"]
    assert int(counters.count_nonzero()) == 0
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("layout", ["token_major", "dim_major"])
def test_unaligned_q_takes_the_generic_kernel(layout, record):
    import flashdec_amd as fd

    q, k, v, table, sl = make_paged_inputs([500, 64], 16, 2, 128, 16, torch.bfloat16, seed=9, kv_layout=layout)
    q_view = _shifted(tuple(q.shape), torch.bfloat16)
    q_view.copy_(q)
    out = _shifted(tuple(q.shape), torch.bfloat16)
    fd.paged_decode_attention_into(q_view, k, v, table, sl, out, kv_layout=layout)
    assert record.last_launch()[0].startswith("fd::decode_generic_kernel<"), record.last_launch()
    expected = oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), sl.cpu().numpy(), kv_layout=layout)
    assert_close_to_oracle(out, expected)


def test_vllm_launcher_with_unaligned_out():
    from flashdec_amd.paged_decode import _vllm_paged_decode_attention_into

    bs, lens = 16, [700, 20, 1500]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, 128, bs, torch.bfloat16, seed=12)
    cache = torch.stack((k.permute(0, 2, 1, 3), v.permute(0, 2, 1, 3)), dim=1).contiguous()
    expected = _oracle(q, k, v, table, sl)
    append_k = torch.empty((3, 2, 128), device="cuda", dtype=torch.bfloat16)
    append_v = torch.empty_like(append_k)
    slots = []
    for b, n in enumerate(lens):
        blk, off = int(table[b, (n - 1) // bs]), (n - 1) % bs
        append_k[b], append_v[b] = cache[blk, 0, off], cache[blk, 1, off]
        slots.append(blk * bs + off)
    splits = 8
    ws = (torch.empty((3, 16, splits, 128), device="cuda"), torch.empty((3, 16, splits), device="cuda"),
          torch.empty((3, 16, splits), device="cuda"))
    out = _shifted((3, 16, 128), torch.bfloat16)
    _vllm_paged_decode_attention_into(q, append_k, append_v, cache, table, sl, out,
                                      torch.tensor(slots, device="cuda", dtype=torch.int64), *ws, num_reqs=3,
                                      num_q_heads=16, num_kv_heads=2, head_dim=128, block_size=bs,
                                      sm_scale=1.0 / math.sqrt(128), num_splits=splits)
    assert_close_to_oracle(out, expected)
    assert np.isfinite(np32(out)).all()
