"""Seeded random sweep of decode configurations against the oracle.

Each case draws the batch, head counts, head_dim, block size, layout, dtype,
row lengths (zero-length and one-token rows included), explicit or planned
split counts, the load policy and, where the reference allows it (grouped
GQA, head_dim 128, block size 16 or 32), the fused current-token append into
a NaN-poisoned slot.  The draws are fixed by the case's seed, so a failure
names a reproducible configuration.  Oracle: the paged-decode oracle
(flashdec/paged_reference.py:19-125); appended K/V bytes bit for bit.
Tolerance: atol 2e-2 / rtol 1e-2.
"""

import numpy as np
import pytest
import torch

from oracle.attention import paged_decode_attention as oracle_decode
from tests.helpers import assert_close_to_oracle, bits16, make_paged_inputs, np32

pytestmark = pytest.mark.gpu

SEEDS = list(range(48))


def draw(seed):
    rng = np.random.default_rng(1000 + seed)
    # about a third of the cases fuse the current token's append, on the shapes the reference takes it for
    fuse = bool(rng.random() < 0.3)
    hkv = int(rng.choice([1, 2, 4, 8]))
    group = int(rng.choice([4, 8, 16] if fuse else [1, 2, 4, 7, 8, 12, 16, 20, 32, 40]))
    head_dim = 128 if fuse else int(rng.choice([64, 128]))
    block_size = int(rng.choice([16, 32] if fuse else [8, 16, 32]))
    layout = "token_major" if fuse or rng.random() >= 0.25 else "dim_major"
    dtype = torch.bfloat16 if rng.random() < 0.6 else torch.float16
    batch = int(rng.integers(1, 7))
    lens = []
    for _ in range(batch):
        r = rng.random()
        lens.append(0 if r < 0.08 and not fuse else 1 if r < 0.15 else int(rng.integers(2, 2500)))
    splits = int(rng.choice([0, 1, 2, 3, 7, 16]))  # 0: the library's plan
    kv_reuse = bool(rng.random() < 0.3)
    return dict(hq=hkv * group, hkv=hkv, head_dim=head_dim, block_size=block_size, layout=layout, dtype=dtype,
                lens=lens, splits=splits, kv_reuse=kv_reuse, fuse=fuse)


@pytest.mark.parametrize("seed", SEEDS)
def test_random_configuration_matches_oracle(seed):
    from flashdec_amd.paged_decode import paged_decode_attention_into

    c = draw(seed)
    print(f"random decode seed={seed} {c}", flush=True)
    q, k, v, table, sl = make_paged_inputs(c["lens"], c["hq"], c["hkv"], c["head_dim"], c["block_size"], c["dtype"],
                                           seed=seed, kv_layout=c["layout"])
    b, hq, d = q.shape
    kwargs = {}
    if c["splits"]:
        s = c["splits"]
        kwargs["num_splits"] = s
        kwargs["split_kv_workspace"] = (torch.empty((b, hq, s, d), device="cuda"),
                                        torch.empty((b, hq, s), device="cuda"), torch.empty((b, hq, s), device="cuda"))
    k_expected = v_expected = None
    if c["fuse"]:
        bs = c["block_size"]
        pos = sl.to(torch.int64) - 1
        slots = table.gather(1, (pos // bs).view(-1, 1).to(torch.int64)).view(-1).to(torch.int64) * bs + pos % bs
        blk, off = slots // bs, slots % bs
        ak = k[blk, :, off].clone()
        av = v[blk, :, off].clone()
        k_expected, v_expected = k.clone(), v.clone()
        k[blk, :, off] = float("nan")
        v[blk, :, off] = float("nan")
        kwargs.update(append_k=ak, append_v=av, slot_mapping=slots)
    expected = oracle_decode(np32(q), np32(k_expected if c["fuse"] else k), np32(v_expected if c["fuse"] else v),
                             table.cpu().numpy(), sl.cpu().numpy(), kv_layout=c["layout"])
    out = torch.empty_like(q)
    paged_decode_attention_into(q, k, v, table, sl, out, block_size=c["block_size"], kv_layout=c["layout"],
                                kv_reuse=c["kv_reuse"], **kwargs)
    assert_close_to_oracle(out, expected)
    if c["fuse"]:
        assert np.array_equal(bits16(k), bits16(k_expected))
        assert np.array_equal(bits16(v), bits16(v_expected))
    for row, n in enumerate(c["lens"]):
        if n == 0:
            assert torch.count_nonzero(out[row]) == 0


def test_the_sweep_covers_the_paths():
    # the draws above reach every family of launch at least once
    cases = [draw(s) for s in SEEDS]
    assert any(c["layout"] == "dim_major" for c in cases)
    assert any(c["fuse"] for c in cases)
    assert any(c["hq"] // c["hkv"] > 16 for c in cases)
    assert any(c["splits"] == 0 for c in cases) and any(c["splits"] > 1 for c in cases)
    assert any(0 in c["lens"] for c in cases) and any(1 in c["lens"] for c in cases)
    assert any(c["block_size"] == 8 for c in cases) and any(c["head_dim"] == 64 for c in cases)
    assert any(c["kv_reuse"] for c in cases)
