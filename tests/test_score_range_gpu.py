"""GPU parity when the running softmax maximum moves far and often.

The decode kernels keep a per-column reference maximum that moves only when a
unit's scores exceed it by more than 2^8 (base 2); the probabilities of a unit
are taken against that reference.  N(0,1) inputs never move it after the first
unit, so these cases shape the scores instead:

- ``steps``: the scores climb by about 12 (base 2) every 64 tokens, with noise
  of about 1 inside each step, so the maximum moves past the slack every few
  units, each move rescaling the accumulator by about 2^-12, and the result
  mixes the last step's tokens;
- ``large``: q and K of standard deviation 3.5 (scores of standard deviation
  about 12), whose maximum drifts up by more than the slack over a split;
- ``falling``: the first tokens hold the maximum and the rest decay, so the
  reference maximum never moves and later probabilities underflow.

Every kernel family runs them: the row kernel (planned splits and explicit
long splits, head_dim 64 and 128), the dim-major kernel, per-row (ragged)
splits and the shared-prefix cascade with 16- and 32-row chunks.  Oracle: the
paged-decode oracle (flashdec/paged_reference.py:19-125, float64 softmax), so
a rescale that dropped or double-applied a factor fails by far more than the
tolerance.  Tolerance: atol 2e-2 / rtol 1e-2.
"""

import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, make_paged_inputs, np32
from tests.test_cascade_gpu import make_prefix_inputs

pytestmark = pytest.mark.gpu

PROFILES = ["steps", "large", "falling"]


def _shape_scores(profile, q, k, v, table, lens, block_size, seed):
    """Rewrite q and the live K rows (token-major caches) for a score profile.
    The level of token t's K row is a function of t, so rows sharing a
    prefix block give it the same level."""
    gen = torch.Generator().manual_seed(seed)
    d = q.shape[-1]
    if profile == "large":
        qn = torch.randn(q.shape, generator=gen) * 3.5
        kn = torch.randn(k.shape, generator=gen) * 3.5
        q.copy_(qn.to(q.dtype))
        k.copy_(kn.to(k.dtype))
        return
    # q = 0.5 + N(0, 0.25): q . 1 is about d/2 for every head, so a K row of
    # level a * 1 + N(0,1) scores about a * d / (2 sqrt(d)) plus noise of ~0.7
    qn = 0.5 + 0.5 * torch.randn(q.shape, generator=gen)
    q.copy_(qn.to(q.dtype))
    tab = table.cpu()
    ln = lens.cpu()
    kc = k.cpu().float()
    step = 8.3 / (0.5 * d**0.5)  # ~12 (base 2) of score per level
    for b in range(tab.shape[0]):
        n = int(ln[b])
        if n == 0:
            continue
        t = torch.arange(n)
        if profile == "steps":
            level = (t // 64).float() * step
        else:  # falling: the first 16 tokens on top, then 12 (base 2) lower per 16 tokens
            level = -(t // 16).float() * step
        blocks = tab[b, t // block_size].long()
        offs = (t % block_size).long()
        # K of token t: its level plus noise drawn from a fixed seed
        noise = torch.randn((n, 1, d), generator=torch.Generator().manual_seed(seed + 1)).expand(n, k.shape[1], d)
        kc[blocks, :, offs, :] = level[:, None, None] + noise
    k.copy_(kc.to(k.dtype))


def _oracle(q, k, v, table, lens, kv_layout="token_major"):
    return oracle_decode(np32(q), np32(k), np32(v), table.cpu().numpy(), lens.cpu().numpy(), kv_layout=kv_layout)


def _workspace(b, hq, splits, head_dim):
    return (torch.empty((b, hq, splits, head_dim), device="cuda"), torch.empty((b, hq, splits), device="cuda"),
            torch.empty((b, hq, splits), device="cuda"))


@pytest.mark.parametrize("profile", PROFILES)
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_row_kernel_planned_splits(profile, dtype):
    # C2's shape plus ragged neighbours: about one 32-token unit per wave
    import flashdec_amd as fd

    lens = [2048, 1500, 700, 3000]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, 128, 32, dtype, seed=91)
    _shape_scores(profile, q, k, v, table, sl, 32, 91)
    out = fd.decode(q, k, v, table, sl)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("profile", PROFILES)
@pytest.mark.parametrize(("hq", "hkv", "head_dim"), [(16, 2, 128), (8, 2, 64), (32, 2, 128)])
@pytest.mark.parametrize("num_splits", [1, 3])
def test_row_kernel_long_splits(num_splits, hq, hkv, head_dim, profile):
    # one or three splits over up to 4096 tokens: 16-token units, many per wave
    import flashdec_amd as fd

    lens = [4096, 2500, 33, 1024]
    q, k, v, table, sl = make_paged_inputs(lens, hq, hkv, head_dim, 16, torch.bfloat16, seed=93)
    _shape_scores(profile, q, k, v, table, sl, 16, 93)
    out = torch.empty_like(q)
    fd.paged_decode_attention_into(q, k, v, table, sl, out, split_kv_workspace=_workspace(4, hq, 3, head_dim),
                                   num_splits=num_splits)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("profile", PROFILES)
@pytest.mark.parametrize("head_dim", [64, 128])
@pytest.mark.parametrize("block_size", [8, 32])
def test_dim_major_kernel(block_size, head_dim, profile):
    import flashdec_amd as fd

    lens = [4096, 999, 2048]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, head_dim, block_size, torch.bfloat16, seed=95)
    _shape_scores(profile, q, k, v, table, sl, block_size, 95)
    kd = k.permute(0, 1, 3, 2).contiguous()
    vd = v.permute(0, 1, 3, 2).contiguous()
    out = torch.empty_like(q)
    fd.paged_decode_attention_into(q, kd, vd, table, sl, out, block_size=block_size, kv_layout="dim_major",
                                   split_kv_workspace=_workspace(3, 16, 2, head_dim), num_splits=2)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("profile", PROFILES)
def test_ragged_splits(profile):
    import flashdec_amd as fd

    lens = [6000, 10, 250, 0, 1500, 33, 7, 3000, 60]
    q, k, v, table, sl = make_paged_inputs(lens, 16, 2, 128, 32, torch.bfloat16, seed=97)
    _shape_scores(profile, q, k, v, table, sl, 32, 97)
    out = fd.decode(q, k, v, table, sl, ragged=True)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))


@pytest.mark.parametrize("profile", PROFILES)
@pytest.mark.parametrize("chunk_rows", [16, 32])
def test_cascade(chunk_rows, profile):
    from flashdec_amd import cascade

    # 12 rows on a 96-block (3072-token) prefix with tails, 5 rows on a
    # 20-block one, two rows in no group
    groups = [(96, [5, 0, 300, 77, 1, 40, 700, 12, 64, 65, 9, 31]), (20, [100, 1, 0, 33, 500])]
    q, k, v, table, sl, _ = make_prefix_inputs(groups, [1200, 64], 16, 2, 32, torch.bfloat16, seed=99)
    _shape_scores(profile, q, k, v, table, sl, 32, 99)
    g = cascade.build_cascade_groups(table, sl, 32, 16, 2)
    out = cascade.paged_decode_attention_cascade(q, k, v, table, sl, groups=g, chunk_rows=chunk_rows)
    assert_close_to_oracle(out, _oracle(q, k, v, table, sl))
