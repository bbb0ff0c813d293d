"""The K/V read policy (``kv_reuse``) changes only how K/V are loaded.

Streaming (non-temporal) and plain loads must give bit-identical outputs on
every kernel that takes the switch: the row kernel (one and several units per
wave, one and two column blocks per wave, fused append), the dim-major
kernel, per-row (balanced) splits, the cascade launch and the vLLM
launcher.  (The plain-load kernels also read block ids through the scalar
cache, the streaming ones through vector loads.)  Both are also checked against the fp32 oracle.  A value other
than 0 or 1 is rejected before any launch.
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


@pytest.mark.parametrize("lens", [[2048] * 8, [40, 5, 3000, 777], [16384, 9000]])
@pytest.mark.parametrize("block_size", [16, 32])
@pytest.mark.parametrize(("hq", "head_dim"), [(16, 128), (64, 128), (40, 64)])
def test_row_kernel_same_bits_either_policy(lens, block_size, hq, head_dim):
    # G 8 (one column block), G 32 and G 20 (two column blocks per wave)
    import flashdec_amd as fd

    q, k, v, table, sl = make_paged_inputs(lens, hq, 2, head_dim, block_size, torch.bfloat16, seed=5 + len(lens))
    streamed = fd.decode(q, k, v, table, sl)
    cached = fd.decode(q, k, v, table, sl, kv_reuse=True)
    assert torch.equal(streamed.view(torch.int16), cached.view(torch.int16))
    assert_close_to_oracle(streamed, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("block_size", [8, 32])
def test_dim_major_same_bits_either_policy(block_size, head_dim):
    import flashdec_amd as fd

    lens = [4096, 1000, 33]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, head_dim, block_size, torch.bfloat16, seed=9,
                                           kv_layout="dim_major")
    streamed = fd.decode(q, k, v, table, sl, kv_layout="dim_major")
    cached = fd.decode(q, k, v, table, sl, kv_layout="dim_major", kv_reuse=True)
    assert torch.equal(streamed.view(torch.int16), cached.view(torch.int16))
    expected = oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), sl.cpu().numpy(), kv_layout="dim_major")
    assert_close_to_oracle(streamed, expected)


def test_balanced_splits_same_bits_either_policy():
    import flashdec_amd as fd

    rng = np.random.default_rng(1701)
    lens = [int(round(math.exp(x))) for x in rng.uniform(math.log(128), math.log(32768), size=12)]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, 128, 32, torch.bfloat16, seed=1701)
    streamed = fd.decode(q, k, v, table, sl, ragged=True)
    cached = fd.decode(q, k, v, table, sl, ragged=True, kv_reuse=True)
    assert torch.equal(streamed.view(torch.int16), cached.view(torch.int16))
    assert_close_to_oracle(streamed, _oracle(q, k, v, table, sl))


def test_fused_append_same_bits_either_policy():
    from flashdec_amd.paged_decode import paged_decode_attention_into

    lens = [300, 64, 1000]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, 128, 32, torch.bfloat16, seed=77)
    gen = torch.Generator().manual_seed(78)
    ak = torch.randn((3, 2, 128), generator=gen).to(torch.bfloat16).cuda()
    av = torch.randn((3, 2, 128), generator=gen).to(torch.bfloat16).cuda()
    pos = sl.to(torch.int64) - 1
    slots = table.gather(1, (pos // 32).view(-1, 1)).view(-1).to(torch.int64) * 32 + pos % 32
    outs, caches = [], []
    for reuse in (False, True):
        kc, vc = k.clone(), v.clone()
        out = torch.empty_like(q)
        paged_decode_attention_into(q, kc, vc, table, sl, out, append_k=ak, append_v=av, slot_mapping=slots,
                                    kv_reuse=reuse)
        outs.append(out)
        caches.append((kc, vc))
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    assert torch.equal(caches[0][0].view(torch.int16), caches[1][0].view(torch.int16))
    assert torch.equal(caches[0][1].view(torch.int16), caches[1][1].view(torch.int16))


def test_cascade_same_bits_either_policy():
    from flashdec_amd.cascade import build_cascade_groups, paged_decode_attention_cascade

    gen = torch.Generator().manual_seed(91)
    prefix_blocks, bs, rows = 40, 32, 6
    tails = [1, 100, 33, 512, 7, 64]
    pool = prefix_blocks + sum((t + bs - 1) // bs for t in tails) + 4
    perm = torch.randperm(pool, generator=gen).to(torch.int32)
    width = prefix_blocks + max((t + bs - 1) // bs for t in tails)
    table = torch.full((rows, width), -1, dtype=torch.int32)
    cursor = prefix_blocks
    for r, t in enumerate(tails):
        n = (t + bs - 1) // bs
        table[r, :prefix_blocks] = perm[:prefix_blocks]
        table[r, prefix_blocks:prefix_blocks + n] = perm[cursor:cursor + n]
        cursor += n
    sl = torch.tensor([prefix_blocks * bs + t for t in tails], dtype=torch.int32)
    k = torch.randn((pool, 2, bs, 128), generator=gen).to(torch.bfloat16).cuda()
    v = torch.randn((pool, 2, bs, 128), generator=gen).to(torch.bfloat16).cuda()
    q = torch.randn((rows, 16, 128), generator=gen).to(torch.bfloat16).cuda()
    table, sl = table.cuda(), sl.cuda()
    groups = build_cascade_groups(table, sl, bs, 16, 2, device=q.device)
    # the cascade's own default is kv_reuse=True: the streamed run asks for it
    streamed = paged_decode_attention_cascade(q, k, v, table, sl, groups=groups, kv_reuse=False)
    cached = paged_decode_attention_cascade(q, k, v, table, sl, groups=groups, kv_reuse=True)
    assert torch.equal(streamed.view(torch.int16), cached.view(torch.int16))
    assert_close_to_oracle(streamed, _oracle(q, k, v, table, sl))


def test_bad_policy_value_is_rejected():
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    q, k, v, table, sl = make_paged_inputs([64, 64], 16, 2, 128, 32, torch.bfloat16, seed=3)
    out = torch.empty_like(q)
    args = _lib.PagedDecodeArgs()
    pd._fill_common(args, q, k, v, pd._cache_strides(k, 2, 3), pd._cache_strides(v, 2, 3), table, sl, out, 2, 32,
                    1.0 / math.sqrt(128))
    args.num_blocks = k.shape[0]
    pd._fill_workspace(args, None, None, None, 1)
    args.kv_reuse = 2
    with pytest.raises(RuntimeError, match="kv_reuse must be 0 or 1"):
        _lib.paged_decode(args, _lib.current_stream_handle(q.device))
