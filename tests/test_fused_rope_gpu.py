"""Decode with RoPE + append fused into the attention launch.

``rope=(rotary_dim, base)`` on the fused-append decode takes q and append_k
unrotated and rotates both at position seq_len - 1.  It must give the same
bits as the two-kernel path it replaces -- ``fused_rope_kv_append`` at those
positions, then decode of the rotated q -- for the output and for every byte
of both caches, and match the oracles (RoPE oracle, then attention oracle)
within atol 2e-2 / rtol 1e-2 against fp32.  Bad combinations are refused
before any launch.
"""

import math

import numpy as np
import pytest
import torch

from flashdec_amd._fused_rope_kv_append import fused_rope_kv_append
from flashdec_amd.paged_decode import _decode_with_workspace, paged_decode_attention_into
from oracle import attention as oa
from oracle import rope as orope
from tests.helpers import assert_close_to_oracle, bits16, make_paged_inputs

pytestmark = pytest.mark.gpu


def _locations(table, lens, bs):
    """Block id, offset and slot of each row's newest token (index seq_len - 1)."""
    blk, off, slot = [], [], []
    for b, n in enumerate(lens.tolist()):
        t = n - 1
        blk.append(int(table[b, t // bs]))
        off.append(t % bs)
        slot.append(blk[-1] * bs + t % bs)
    i64 = dict(device="cuda", dtype=torch.int64)
    return torch.tensor(blk, **i64), torch.tensor(off, **i64), torch.tensor(slot, **i64)


def _workspace(b, hq, splits):
    if splits == 1:
        return None
    return (torch.empty((b, hq, splits, 128), device="cuda"), torch.empty((b, hq, splits), device="cuda"),
            torch.empty((b, hq, splits), device="cuda"))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("rotary_dim", [64, 128])
@pytest.mark.parametrize("block_size", [16, 32])
@pytest.mark.parametrize(("lens", "splits"), [([1, 17, 300, 2049], 8), ([4096] * 8, 16), ([33, 64, 65], 1),
                                              ([700, 9000], 4)])
def test_fused_rope_matches_two_kernel_path_bit_for_bit(lens, splits, block_size, rotary_dim, dtype):
    base = 1e6
    hq, hkv = 16, 2
    q, k, v, table, sl = make_paged_inputs(lens, hq, hkv, 128, block_size, dtype, seed=len(lens) + block_size)
    gen = torch.Generator().manual_seed(rotary_dim + block_size)
    ak = torch.randn((len(lens), hkv, 128), generator=gen).to(dtype).cuda()
    av = torch.randn((len(lens), hkv, 128), generator=gen).to(dtype).cuda()
    blk, off, slot = _locations(table.cpu(), sl.cpu(), block_size)
    pos = sl.to(torch.int64) - 1
    scale = 1.0 / math.sqrt(128)

    # two kernels: RoPE + append into the caches, then decode of the rotated q
    k2, v2 = k.clone(), v.clone()
    q_rot = fused_rope_kv_append(q, ak, av, k2, v2, blk, off, pos, rotary_dim=rotary_dim, base=base)
    ref = torch.empty_like(q)
    _decode_with_workspace(q_rot, k2, v2, table, sl, ref, scale, block_size, splits, _workspace(len(lens), hq, splits),
                           k.shape[0])

    # one launch
    k1, v1 = k.clone(), v.clone()
    out = torch.empty_like(q)
    _decode_with_workspace(q, k1, v1, table, sl, out, scale, block_size, splits, _workspace(len(lens), hq, splits),
                           k.shape[0], append=(ak, av, slot), rope=(rotary_dim, base))
    torch.cuda.synchronize()
    assert np.array_equal(bits16(out), bits16(ref))
    assert np.array_equal(bits16(k1), bits16(k2))
    assert np.array_equal(bits16(v1), bits16(v2))

    # and the oracles: rotated q and K, then attention over the updated cache
    odt = "bfloat16" if dtype == torch.bfloat16 else "float16"
    q_o = orope.apply_rope(q.float().cpu().numpy(), pos.cpu().numpy(), rotary_dim=rotary_dim, base=base,
                           out_dtype=odt)
    expected = oa.paged_decode_attention(q_o, k2.float().cpu().numpy(), v2.float().cpu().numpy(),
                                         table.cpu().numpy(), sl.cpu().numpy(), sm_scale=scale)
    assert_close_to_oracle(out, expected)
    k_o = orope.apply_rope(ak.float().cpu().numpy(), pos.cpu().numpy(), rotary_dim=rotary_dim, base=base,
                           out_dtype=odt)
    got = k1[blk.cpu(), :, off.cpu()].float().cpu().numpy()
    assert np.array_equal(got, k_o)


def test_fused_rope_refusals():
    q, k, v, table, sl = make_paged_inputs([40, 50], 16, 2, 128, 32, torch.bfloat16, seed=3)
    ak = torch.zeros((2, 2, 128), device="cuda", dtype=torch.bfloat16)
    blk, off, slot = _locations(table.cpu(), sl.cpu(), 32)
    out = torch.empty_like(q)
    ws = _workspace(2, 16, 4)
    with pytest.raises(RuntimeError, match="rotary_dim needs the fused append"):
        _decode_with_workspace(q, k, v, table, sl, out, 0.1, 32, 4, ws, k.shape[0], rope=(128, 1e4))
    with pytest.raises(RuntimeError, match="rotary_dim must be 0, 64 or 128"):
        _decode_with_workspace(q, k, v, table, sl, out, 0.1, 32, 4, ws, k.shape[0], append=(ak, ak, slot),
                               rope=(96, 1e4))
    with pytest.raises(RuntimeError, match="rope_base must be a positive finite number"):
        _decode_with_workspace(q, k, v, table, sl, out, 0.1, 32, 4, ws, k.shape[0], append=(ak, ak, slot),
                               rope=(128, float("nan")))
    counters = torch.zeros(2 * 2 * 64, device="cuda", dtype=torch.int32)
    with pytest.raises(RuntimeError, match="in-launch merge"):
        _decode_with_workspace(q, k, v, table, sl, out, 0.1, 32, 4, ws, k.shape[0], counters=counters,
                               append=(ak, ak, slot), rope=(128, 1e4))
    q64, k64, v64, t64, sl64 = make_paged_inputs([40, 50], 16, 2, 64, 32, torch.bfloat16, seed=4)
    ak64 = torch.zeros((2, 2, 64), device="cuda", dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="fused RoPE needs head_dim 128"):
        _decode_with_workspace(q64, k64, v64, t64, sl64, torch.empty_like(q64), 0.1, 32, 1, None, k64.shape[0],
                               append=(ak64, ak64, slot), rope=(64, 1e4))
    q32, k32, v32, t32, sl32 = make_paged_inputs([40, 50], 64, 2, 128, 32, torch.bfloat16, seed=5)
    with pytest.raises(RuntimeError, match="<= 16 query heads per KV head"):
        _decode_with_workspace(q32, k32, v32, t32, sl32, torch.empty_like(q32), 0.1, 32, 1, None, k32.shape[0],
                               append=(ak, ak, slot), rope=(128, 1e4))
    # nothing above launched: the caches are untouched
    q2, k2, v2, _, _ = make_paged_inputs([40, 50], 16, 2, 128, 32, torch.bfloat16, seed=3)
    assert torch.equal(k, k2) and torch.equal(v, v2)
