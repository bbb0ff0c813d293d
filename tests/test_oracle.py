"""Pins the CPU oracle before it is trusted as the GPU parity checker.

Each oracle function is checked against (1) the reference's own known-answer
values (tests/golden/reference_kats.json, cited per entry), (2) closed forms
and invariants the mathematics fixes, and (3) planted mistakes: plausible
wrong variants of the oracle, built here on the CPU, must fail the same
checks, which shows that the checks are sensitive to them.
"""

import json
import math
import pathlib

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from oracle import split_policy as osp
from tests.helpers import rope_pair_bound

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def random_paged(seq_lens, hq, hkv, d, bs, seed, layout="token_major"):
    rng = np.random.default_rng(seed)
    nblk = [(n + bs - 1) // bs for n in seq_lens]
    pool = sum(nblk) + 3
    perm = rng.permutation(pool)
    width = max(1, max(nblk))
    table = np.full((len(seq_lens), width), -1, dtype=np.int32)
    c = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[c:c + n]
        c += n
    shape = (pool, hkv, bs, d) if layout == "token_major" else (pool, hkv, d, bs)
    k = rng.standard_normal(shape).astype(np.float32)
    v = rng.standard_normal(shape).astype(np.float32)
    q = rng.standard_normal((len(seq_lens), hq, d)).astype(np.float32)
    return q, k, v, table, np.array(seq_lens, dtype=np.int32)


def dense_single_block(kat):
    """A reference dense fixture [B, L, Hkv, D] as a paged cache with one block per sequence."""
    k = np.array(kat["k"], dtype=np.float32)  # [B, L, Hkv, D]
    v = np.array(kat["v"], dtype=np.float32)
    kc = k.transpose(0, 2, 1, 3)  # [B(blocks), Hkv, L(bs), D]
    vc = v.transpose(0, 2, 1, 3)
    table = np.arange(k.shape[0], dtype=np.int32)[:, None]
    return np.array(kat["q"], dtype=np.float32), kc, vc, table, np.array(kat["seq_lens"])


# ------------------------------------------------------------- attention
def test_attention_padding_kat_closed_form():
    kat = KATS["dense_decode_padding"]
    q, kc, vc, table, lens = dense_single_block(kat)
    out = oa.paged_decode_attention(q, kc, vc, table, lens, sm_scale=kat["sm_scale"])
    p0 = math.e / (math.e + 1.0)
    expected = np.array([[[10.0 * p0, 20.0 * (1.0 - p0)]]])
    np.testing.assert_allclose(out, expected, rtol=1e-6)  # the padded 1000s never enter
    dense = oa.dense_attention_f64(np.array(kat["q"]), np.array(kat["k"]), np.array(kat["v"]), lens, kat["sm_scale"])
    np.testing.assert_allclose(dense, expected, rtol=1e-12)


def test_attention_mqa_kat_closed_form():
    kat = KATS["dense_decode_mqa"]
    q, kc, vc, table, lens = dense_single_block(kat)
    out = oa.paged_decode_attention(q, kc, vc, table, lens, sm_scale=1.0)
    keys = np.array(kat["k"], dtype=np.float64)[0, :, 0]
    vals = np.array(kat["v"], dtype=np.float64)[0, :, 0]
    for h, qh in enumerate(np.array(kat["q"], dtype=np.float64)[0]):
        w = np.exp(keys @ qh)
        np.testing.assert_allclose(out[0, h], (w / w.sum()) @ vals, rtol=1e-6)


@pytest.mark.parametrize("layout", ["token_major", "dim_major"])
@pytest.mark.parametrize("hq,hkv", [(4, 4), (8, 2), (6, 1)])
def test_attention_matches_float64_brute_force(layout, hq, hkv):
    lens = [1, 7, 16, 33, 0]
    q, k, v, table, sl = random_paged(lens, hq, hkv, 8, 4, seed=hq * 10 + hkv, layout=layout)
    out = oa.paged_decode_attention(q, k, v, table, sl, kv_layout=layout)
    kd, vd = oa.paged_to_dense(k, v, table, sl, kv_layout=layout)
    ref = oa.dense_attention_f64(q, kd, vd, sl)
    np.testing.assert_allclose(out, ref, atol=2e-6, rtol=2e-6)
    assert not out[4].any()  # empty sequence -> zero row


def test_paged_to_dense_agrees_with_hand_indexing():
    q, k, v, table, sl = random_paged([5, 9], 2, 2, 4, 4, seed=3)
    kd, _ = oa.paged_to_dense(k, v, table, sl)
    # token 6 of sequence 1 lives in logical block 1, offset 2
    np.testing.assert_array_equal(kd[1, 6], k[table[1, 1], :, 2])
    assert not kd[0, 5:].any()


def test_attention_invariants():
    q, k, v, table, sl = random_paged([13, 4], 4, 2, 8, 4, seed=11)
    base = oa.paged_decode_attention(q, k, v, table, sl)
    # relabelling physical blocks changes nothing
    perm = np.random.default_rng(0).permutation(k.shape[0])
    inv = np.argsort(perm)
    t2 = np.where(table >= 0, inv[np.maximum(table, 0)], -1)
    np.testing.assert_array_equal(oa.paged_decode_attention(q, k[perm], v[perm], t2, sl), base)
    # constant V rows -> the output is that constant (weights sum to one)
    vc = np.ones_like(v) * 0.75
    np.testing.assert_allclose(oa.paged_decode_attention(q, k, vc, table, sl), 0.75, rtol=1e-6)
    # one token -> output equals that token's V for every head of its group
    one = oa.paged_decode_attention(q, k, v, table, np.array([1, 1]))
    np.testing.assert_allclose(one[0, 0], v[table[0, 0], 0, 0], rtol=1e-6)
    np.testing.assert_allclose(one[0, 3], v[table[0, 0], 1, 0], rtol=1e-6)
    # NaN past seq_len inside the last block, and garbage in unused table slots, are never read
    k2, v2 = k.copy(), v.copy()
    k2[table[0, 3], :, 1:] = np.nan  # sequence 0 holds 13 tokens: block 3 keeps only offset 0
    v2[table[0, 3], :, 1:] = np.nan
    t3 = table.copy()
    t3[1, 1:] = 10 ** 6
    np.testing.assert_array_equal(oa.paged_decode_attention(q, k2, v2, t3, sl), base)


def test_attention_rejects_invalid_block_in_used_range():
    q, k, v, table, sl = random_paged([5], 2, 1, 4, 4, seed=1)
    bad = table.copy()
    bad[0, 1] = -1
    with pytest.raises(ValueError, match="invalid physical block"):
        oa.paged_decode_attention(q, k, v, bad, sl)


def test_attention_output_rounding():
    q, k, v, table, sl = random_paged([9], 2, 1, 8, 4, seed=2)
    f32 = oa.paged_decode_attention(q, k, v, table, sl)
    bf = oa.paged_decode_attention(q, k, v, table, sl, out_dtype="bfloat16")
    assert np.array_equal(bf, torch.from_numpy(f32).to(torch.bfloat16).float().numpy())


def _planted_gqa_modulo(q, k, v, table, sl):
    """Plausible mistake: query head h reads KV head h % Hkv instead of h // group."""
    hq, hkv = q.shape[1], k.shape[1]
    perm = [h % hkv for h in range(hq)]
    kd, vd = oa.paged_to_dense(k, v, table, sl)
    kx = np.stack([kd[:, :, j] for j in perm], axis=2)
    vx = np.stack([vd[:, :, j] for j in perm], axis=2)
    return oa.dense_attention_f64(q, kx, vx, sl)


def test_planted_attention_mistakes_are_detected():
    q, k, v, table, sl = random_paged([11, 6], 8, 2, 8, 4, seed=21)
    kd, vd = oa.paged_to_dense(k, v, table, sl)
    truth = oa.dense_attention_f64(q, kd, vd, sl)
    wrong = {
        "gqa h%Hkv": _planted_gqa_modulo(q, k, v, table, sl),
        "no scale": oa.dense_attention_f64(q, kd, vd, sl, sm_scale=1.0),
        "off-by-one length": oa.dense_attention_f64(q, kd, vd, sl - 1),
        "K/V swapped": oa.dense_attention_f64(q, vd, kd, sl),
    }
    for name, w in wrong.items():
        assert not np.allclose(w, truth, atol=2e-2, rtol=1e-2), name


def test_algorithmic_bytes_closed_form():
    # B8 ctx2048 Hq16 Hkv2 D128 bs32, bf16: KV = 8*2048*2*128*2*2 bytes
    n = oa.algorithmic_bytes([2048] * 8, 16, 2, 128, 32)
    assert n == 8 * 2048 * 2 * 128 * 2 * 2 + 2 * 8 * 16 * 128 * 2 + 4 * 8 * 64 + 4 * 8


# ------------------------------------------------------------------ rope
def test_round_to_bf16_known_bits_and_torch_agreement():
    vals = np.array([1.0, 1 + 2 ** -8, 1 + 3 * 2 ** -8, -2.5, 65504.0, 1e-40, np.inf, -0.0], dtype=np.float32)
    bits = orope.bf16_bits(orope.round_to(vals, "bfloat16"))
    assert [hex(b) for b in bits[:3]] == ["0x3f80", "0x3f80", "0x3f82"]  # ties to even
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(20000) * 10.0 ** rng.integers(-30, 30, 20000)).astype(np.float32)
    x = np.concatenate([x, vals])
    ours = orope.round_to(x, "bfloat16")
    theirs = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ours.view(np.uint32), theirs.view(np.uint32))
    assert np.isnan(orope.round_to(np.array([np.nan], dtype=np.float32), "bfloat16")).all()
    h = orope.round_to(x, "float16")
    assert np.array_equal(h, torch.from_numpy(x).half().float().numpy(), equal_nan=True)


def test_rope_hand_calculation_kat():
    kat = KATS["rope_hand_calculation"]
    x = np.array([[kat["x"]], [kat["x"]]], dtype=np.float32)
    out = orope.apply_rope(x, np.array(kat["positions"]), base=kat["base"])
    np.testing.assert_array_equal(out[0], x[0])  # position 0 is the identity
    c1, s1, c2, s2 = math.cos(1.0), math.sin(1.0), math.cos(0.01), math.sin(0.01)
    expected = [1 * c1 - 3 * s1, 2 * c2 - 4 * s2, 3 * c1 + 1 * s1, 4 * c2 + 2 * s2]
    np.testing.assert_allclose(out[1, 0], expected, atol=kat["tolerance"], rtol=0)


def test_rope_cos_sin_match_the_float64_closed_form():
    """cos/sin of frequency i at position p against the float64 closed form cos(p * base^(-2i/R)):
    the fp32 algorithm rounds the frequency and the angle once each (relative 2^-24 apiece) and
    the result once more, so it may be off by at most angle * 2^-22 + 2^-23.  A frequency index
    off by one, or another base, moves the angle by a fraction of itself and fails the same
    bound at the positions tested."""
    pos = np.array([1, 7, 1000, 8191, 131071])
    rotary_dim, base = 128, 1e6
    half = rotary_dim // 2

    def exact(p, shift=0, b=base):
        theta = np.exp(-2.0 * (np.arange(half) + shift) / rotary_dim * math.log(b))
        ang = p[:, None].astype(np.float64) * theta[None, :]
        return np.cos(ang), np.sin(ang), ang

    cos, sin = orope.rope_cos_sin(pos, rotary_dim, base=base)
    ec, es, ang = exact(pos)
    tol = ang * 2.0**-22 + 2.0**-23
    assert (np.abs(cos - ec) <= tol).all() and (np.abs(sin - es) <= tol).all()
    # position 0 is the identity rotation, exactly
    c0, s0 = orope.rope_cos_sin(np.array([0]), rotary_dim, base=base)
    assert (c0 == 1.0).all() and (s0 == 0.0).all()
    # planted mistakes: the oracle's values must miss each wrong closed form somewhere
    for shift, b in ((1, base), (-1, base), (0, 1e4)):
        wc, ws, _ = exact(pos, shift, b)
        assert (np.abs(cos - wc) > tol).any() or (np.abs(sin - ws) > tol).any()


def test_rope_invariants():
    rng = np.random.default_rng(5)
    x = rng.standard_normal((6, 3, 16)).astype(np.float32)
    pos = np.array([0, 1, 5, 77, 4095, 100000])
    out = orope.apply_rope(x, pos)
    # rotation preserves each (i, i + D/2) pair's norm
    n_in = x[..., :8] ** 2 + x[..., 8:] ** 2
    n_out = out[..., :8] ** 2 + out[..., 8:] ** 2
    np.testing.assert_allclose(n_out, n_in, rtol=2e-5, atol=1e-6)
    # partial rotary: tail copied bit for bit, head equals rotating the head alone
    part = orope.apply_rope(x, pos, rotary_dim=8)
    np.testing.assert_array_equal(part[..., 8:], x[..., 8:])
    np.testing.assert_array_equal(part[..., :8], orope.apply_rope(x[..., :8], pos))
    # rotating by p then by -p (inverse rotation) returns the input
    cos, sin = orope.rope_cos_sin(pos, 16)
    lo, hi = out[..., :8], out[..., 8:]
    back_lo = lo * cos[:, None] + hi * sin[:, None]
    np.testing.assert_allclose(back_lo, x[..., :8], atol=2e-4)
    with pytest.raises(ValueError):
        orope.apply_rope(x, -pos - 1)


def test_rope_matches_torch_reference_order_per_frequency():
    from flashdec_amd.rope import apply_rope as torch_rope

    rng = np.random.default_rng(9)
    x = rng.standard_normal((8, 4, 64)).astype(np.float32)
    pos = rng.integers(0, 32768, 8)
    ours = orope.apply_rope(x, pos, base=1e6)
    theirs = torch_rope(torch.from_numpy(x), torch.from_numpy(pos), base=1e6).numpy()
    assert (np.abs(ours - theirs) <= rope_pair_bound(x, pos, 64, 1e6)).all()
    steps = torch.arange(0, 64, 2, dtype=torch.float32)
    torch_inv = torch.pow(1e6, -steps / 64).numpy()
    oracle_inv = np.array([np.float32(math.pow(1e6, float(np.float32(-s / np.float32(64))))) for s in steps.numpy()])
    assert (np.abs(torch_inv - oracle_inv) <= np.spacing(oracle_inv)).all()


def test_rope_frequencies_match_the_closed_form():
    """Rotating unit vectors recovers each frequency's angle; against theta_i = exp(-2i/R * ln base)
    (float64), it is off by no more than the fp32 algorithm's own rounding: (pos + 1) * theta_i *
    2^-22 + 2^-22.  A wrong frequency (index off by one, a different base, a dropped factor 2)
    changes the angle by a fraction of pos * theta_i and fails at every position tested."""
    def angles(fn, pos, rotary_dim, base):
        half = rotary_dim // 2
        x = np.zeros((len(pos), 1, rotary_dim), dtype=np.float32)
        x[..., :half] = 1.0  # lo = cos(angle), hi = sin(angle)
        out = fn(x, pos, rotary_dim, base)
        return np.arctan2(out[:, 0, half:].astype(np.float64), out[:, 0, :half].astype(np.float64))

    pos = np.array([1, 2, 3, 17, 100, 1000, 8191, 32767])
    for rotary_dim, base in ((128, 1e6), (64, 1e4), (128, 10000.0)):
        half = rotary_dim // 2
        theta = np.exp(-2.0 * np.arange(half) / rotary_dim * math.log(base))
        exact = np.mod(pos[:, None] * theta[None, :] + math.pi, 2 * math.pi) - math.pi
        tol = (pos[:, None] + 1) * theta[None, :] * 2.0**-22 + 2.0**-22

        def wrapped(a, b):
            return np.abs(np.mod(a - b + math.pi, 2 * math.pi) - math.pi)

        def oracle(x, p, r, bs):
            return orope.apply_rope(x, p, rotary_dim=r, base=bs)

        assert (wrapped(angles(oracle, pos, rotary_dim, base), exact) <= tol).all()
        # planted mistakes in the frequency formula: each must fail the same check
        for wrong_base, wrong_shift, wrong_scale in ((base * 10, 0, 1.0), (base, 1, 1.0), (base, 0, 0.5)):
            theta_w = np.exp(-2.0 * (np.arange(half) + wrong_shift) / rotary_dim * math.log(wrong_base)) * wrong_scale
            cos_w, sin_w = np.cos(pos[:, None] * theta_w), np.sin(pos[:, None] * theta_w)

            def planted(x, p, r, bs, cos_w=cos_w, sin_w=sin_w):
                out = x.copy()
                out[..., :half] = x[..., :half] * cos_w[:, None] - x[..., half:r] * sin_w[:, None]
                out[..., half:r] = x[..., half:r] * cos_w[:, None] + x[..., :half] * sin_w[:, None]
                return out

            assert (wrapped(angles(planted, pos, rotary_dim, base), exact) > tol).any()


def test_planted_rope_mistakes_are_detected():
    kat = KATS["rope_hand_calculation"]
    x = np.array([[kat["x"]]], dtype=np.float32)
    truth = orope.apply_rope(x, np.array([1]), base=kat["base"])
    c1, s1, c2, s2 = math.cos(1.0), math.sin(1.0), math.cos(0.01), math.sin(0.01)
    interleaved = [1 * c1 - 2 * s1, 2 * c1 + 1 * s1, 3 * c2 - 4 * s2, 4 * c2 + 3 * s2]  # GPT-J pairing
    sign_flip = [1 * c1 + 3 * s1, 2 * c2 + 4 * s2, 3 * c1 - 1 * s1, 4 * c2 - 2 * s2]
    for wrong in (interleaved, sign_flip):
        assert not np.allclose(truth[0, 0], wrong, atol=1e-3)


def test_rope_kv_append_and_kv_append_write_only_their_slots():
    rng = np.random.default_rng(4)
    nb, hkv, bs, d = 5, 2, 4, 8
    kc = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    vc = rng.standard_normal((nb, hkv, bs, d)).astype(np.float32)
    q = rng.standard_normal((3, 4, d)).astype(np.float32)
    k = rng.standard_normal((3, hkv, d)).astype(np.float32)
    v = rng.standard_normal((3, hkv, d)).astype(np.float32)
    blk, off, pos = np.array([4, 0, 2]), np.array([3, 0, 1]), np.array([19, 0, 9])
    q_out, kc2, vc2 = orope.rope_kv_append(q, k, v, kc, vc, blk, off, pos, dtype="float32")
    np.testing.assert_array_equal(q_out, orope.apply_rope(q, pos))
    mask = np.zeros(kc.shape, dtype=bool)
    for b in range(3):
        mask[blk[b], :, off[b]] = True
        np.testing.assert_array_equal(kc2[blk[b], :, off[b]], orope.apply_rope(k, pos)[b])
        np.testing.assert_array_equal(vc2[blk[b], :, off[b]], v[b])
    np.testing.assert_array_equal(kc2[~mask], kc[~mask])
    np.testing.assert_array_equal(vc2[~mask], vc[~mask])
    kc3, vc3 = orope.kv_append(k, v, kc, vc, blk, off)
    np.testing.assert_array_equal(vc3, vc2)
    np.testing.assert_array_equal(kc3[~mask], kc[~mask])


# ----------------------------------------------------------- split policy
def test_split_policy_kats():
    kat = KATS["split_policy"]
    a = kat["auto_by_num_reqs"]
    for num_reqs, expected in a["cases"]:
        assert osp.select_num_splits(0, num_reqs=num_reqs, num_kv_heads=a["num_kv_heads"],
                                     logical_blocks=a["logical_blocks"]) == expected
    b = kat["auto_by_logical_blocks"]
    for blocks, expected in b["cases"]:
        assert osp.select_num_splits(0, num_reqs=b["num_reqs"], num_kv_heads=b["num_kv_heads"],
                                     logical_blocks=blocks) == expected
    c = kat["explicit"]
    for requested, blocks, expected in c["cases"]:
        assert osp.select_num_splits(requested, num_reqs=c["num_reqs"], num_kv_heads=c["num_kv_heads"],
                                     logical_blocks=blocks) == expected
    for value in kat["valid_requests"]:
        assert osp.parse_requested_splits(value) == int(value)
    for value in kat["invalid_requests"]:
        with pytest.raises(ValueError, match=r"0, 1, 2, 4, 8, or 16 \(0 selects auto\)"):
            osp.parse_requested_splits(value)


def test_torch_loop_restatement_matches_the_numpy_oracle():
    """The torch-CPU loop form (bench.py's CPU baseline) against the independently pinned numpy
    oracle: fp32 C1-shaped inputs with an empty row and ragged lengths, and bf16 inputs."""
    from oracle.torch_loop import paged_decode_attention_loop

    q, k, v, table, lens = random_paged([37, 0, 512, 1, 300], 8, 2, 64, 32, seed=61)
    got = paged_decode_attention_loop(torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v),
                                      torch.from_numpy(table), torch.from_numpy(lens), 0.125).numpy()
    want = oa.paged_decode_attention(q, k, v, table, lens, sm_scale=0.125)
    np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-6)
    assert (got[1] == 0).all()
    bf = [torch.from_numpy(x).to(torch.bfloat16) for x in (q, k, v)]
    got = paged_decode_attention_loop(*bf, torch.from_numpy(table), torch.from_numpy(lens), 0.125)
    assert got.dtype == torch.bfloat16
    want = oa.paged_decode_attention(*(x.float().numpy() for x in bf), table, lens, sm_scale=0.125,
                                     out_dtype="bfloat16")
    np.testing.assert_allclose(got.float().numpy(), want, rtol=1e-2, atol=1e-2)
