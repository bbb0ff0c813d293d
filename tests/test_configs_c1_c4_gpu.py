"""The C1 and C4-shared-prefix configurations at their own sizes, on the HIP path.

C1 (the reference's CPU-runnable case): B4, Hq8 / Hkv2 (group 4), head_dim 64,
32-token blocks, seq_lens ~ U{1..512}, a 128-block pool whose table rows are
consecutive slices of a seeded ``randperm(128)``, N(0,1) q/K/V, scale 1/8,
seed 61.  The reference's decode kernels take fp16/bf16 only
(flashdec/kernels/paged_decode.py:678-679), so the fp32 draw is cast to each.

C4 shared prefix: 16 requests attached to one registered 128-block
(4096-token) prefix with private tails ~ U{1..512} (seed 1701;
flashdec/cache.py:192-248), decoded through ``DecodeEngine`` with the cascade
on (and a per-row engine beside it) and through
``paged_decode_attention_cascade`` on a pool with the same table structure.

Bar: atol 2e-2 / rtol 1e-2 against the fp32 oracle; appended K/V bytes of
the engine steps equal between the cascade and per-row engines.
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from tests.helpers import assert_close_to_oracle, np32

pytestmark = pytest.mark.gpu


def c1_inputs():
    """C1's seeded fp32 inputs (CPU tensors)."""
    gen = torch.Generator().manual_seed(61)
    lens = torch.randint(1, 513, (4,), generator=gen)
    perm = torch.randperm(128, generator=gen)
    nblk = [(int(n) + 31) // 32 for n in lens]
    table = torch.full((4, max(nblk)), -1, dtype=torch.int32)
    cursor = 0
    for b, n in enumerate(nblk):
        table[b, :n] = perm[cursor:cursor + n].to(torch.int32)
        cursor += n
    k = torch.randn((128, 2, 32, 64), generator=gen)
    v = torch.randn((128, 2, 32, 64), generator=gen)
    q = torch.randn((4, 8, 64), generator=gen)
    return q, k, v, table, lens.to(torch.int32)


@pytest.mark.parametrize("kv_layout", ["token_major", "dim_major"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_c1_matches_oracle(dtype, kv_layout):
    import flashdec_amd as fd

    q, k, v, table, lens = (t.clone() for t in c1_inputs())
    assert int(lens.min()) >= 1 and int(lens.max()) <= 512
    q, k, v = q.to(dtype), k.to(dtype), v.to(dtype)
    expected = oa.paged_decode_attention(np32(q), np32(k), np32(v), table.numpy(), lens.numpy(), sm_scale=0.125)
    if kv_layout == "dim_major":
        k, v = k.permute(0, 1, 3, 2).contiguous(), v.permute(0, 1, 3, 2).contiguous()
    dev = [t.cuda() for t in (q, k, v, table, lens)]
    out = fd.decode(*dev, kv_layout=kv_layout)  # scale defaults to 1/sqrt(64)
    assert_close_to_oracle(out, expected)
    for splits in (1, 4):
        ws = (torch.empty((4, 8, 4, 64), device="cuda"), torch.empty((4, 8, 4), device="cuda"),
              torch.empty((4, 8, 4), device="cuda"))
        out2 = torch.empty_like(dev[0])
        fd.paged_decode_attention_into(*dev, out2, kv_layout=kv_layout, split_kv_workspace=ws, num_splits=splits)
        assert_close_to_oracle(out2, expected)


def test_c1_fp32_is_refused_like_the_reference():
    import flashdec_amd as fd

    q, k, v, table, lens = (t.cuda() for t in c1_inputs())
    with pytest.raises(ValueError, match="supports float16 and bfloat16"):
        fd.decode(q, k, v, table, lens)


# ------------------------------------------------------------- C4 prefix --
L, HQ, HKV, D, BS, PREFIX_BLOCKS = 2, 16, 2, 128, 32, 128


def c4_tails():
    return [int(t) for t in np.random.default_rng(1701).integers(1, 513, size=16)]


def make_prefix_engine(min_shared):
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine

    cache = PagedKVCache(L, HKV, D, BS, max_blocks=PREFIX_BLOCKS + 16 * 20, dtype=torch.bfloat16, device="cuda",
                         prefix_cache_capacity_blocks=PREFIX_BLOCKS)
    g = torch.Generator(device="cuda").manual_seed(1701)
    cache.k_cache.normal_(generator=g)
    cache.v_cache.normal_(generator=g)
    engine = DecodeEngine(cache)
    engine.cascade_min_shared_tokens = min_shared
    shape = (L, PREFIX_BLOCKS, HKV, BS, D)
    pk = torch.randn(shape, device="cuda", generator=g).to(torch.bfloat16)
    pv = torch.randn(shape, device="cuda", generator=g).to(torch.bfloat16)
    engine.register_prefix("sys", pk, pv)
    ids = [f"r{i}" for i in range(16)]
    for rid in ids:
        engine.add_request(rid)
    engine.admit(ids, prefix_id="sys")
    for rid, tail in zip(ids, c4_tails()):
        cache.seed_context([rid], tail)
    return engine, ids


def test_c4_shared_prefix_engine_cascade_matches_oracle():
    cascaded, ids = make_prefix_engine(1)
    per_row, _ = make_prefix_engine(None)
    lens0 = cascaded.cache.seq_lens_tensor(ids).cpu().numpy()
    assert np.array_equal(lens0, np.array(c4_tails()) + PREFIX_BLOCKS * BS)
    tables = cascaded.cache.block_tables(ids).cpu().numpy()
    assert (tables[:, :PREFIX_BLOCKS] == tables[0, :PREFIX_BLOCKS]).all()  # one physical prefix for all 16
    g = torch.Generator(device="cuda").manual_seed(5)
    for step in range(3):
        n = len(ids)
        q = torch.randn((L, n, HQ, D), device="cuda", generator=g).to(torch.bfloat16)
        k = torch.randn((L, n, HKV, D), device="cuda", generator=g).to(torch.bfloat16)
        v = torch.randn((L, n, HKV, D), device="cuda", generator=g).to(torch.bfloat16)
        outs = []
        for e in (cascaded, per_row):
            tx = e.begin_step(ids)
            outs.append([e.step_layer(tx, layer, q[layer], k[layer], v[layer], base=1e6).output
                         for layer in range(L)])
            torch.cuda.synchronize()
            if e is cascaded:
                for layer in range(L):
                    q_rot = orope.apply_rope(np32(q[layer]), tx.positions.cpu().numpy(), base=1e6,
                                             out_dtype="bfloat16")
                    expected = oa.paged_decode_attention(q_rot, np32(e.cache.k_cache[layer]),
                                                         np32(e.cache.v_cache[layer]), tx.block_tables.cpu().numpy(),
                                                         tx.effective_seq_lens.cpu().numpy())
                    assert_close_to_oracle(outs[0][layer], expected)
            e.commit_step(tx)
        for layer in range(L):
            assert_close_to_oracle(outs[0][layer], np32(outs[1][layer]))
    assert cascaded._cascade_decode_count == 3 * L and per_row._cascade_decode_count == 0
    assert torch.equal(cascaded.cache.k_cache, per_row.cache.k_cache)
    assert torch.equal(cascaded.cache.v_cache, per_row.cache.v_cache)
    assert cascaded.validate_invariants() and per_row.validate_invariants()


def test_c4_shared_prefix_cascade_api_matches_oracle():
    import flashdec_amd as fd
    from flashdec_amd.cascade import build_cascade_groups, paged_decode_attention_cascade

    tails = c4_tails()
    lens = [PREFIX_BLOCKS * BS + t for t in tails]
    nblk = [(n + BS - 1) // BS for n in lens]
    private = [b - PREFIX_BLOCKS for b in nblk]
    pool = int(np.ceil((PREFIX_BLOCKS + sum(private)) * 1.25)) + 1
    gen = torch.Generator().manual_seed(1701)
    perm = torch.randperm(pool, generator=gen).to(torch.int32)
    table = torch.full((16, max(nblk)), -1, dtype=torch.int32)
    cursor = PREFIX_BLOCKS
    for b, nb in enumerate(nblk):
        table[b, :PREFIX_BLOCKS] = perm[:PREFIX_BLOCKS]
        table[b, PREFIX_BLOCKS:nb] = perm[cursor:cursor + private[b]]
        cursor += private[b]
    k = torch.randn((pool, HKV, BS, D), generator=gen).to(torch.bfloat16)
    v = torch.randn((pool, HKV, BS, D), generator=gen).to(torch.bfloat16)
    q = torch.randn((16, HQ, D), generator=gen).to(torch.bfloat16)
    sl = torch.tensor(lens, dtype=torch.int32)
    expected = oa.paged_decode_attention(np32(q), np32(k), np32(v), table.numpy(), sl.numpy())
    qd, kd, vd, td, ld = (t.cuda() for t in (q, k, v, table, sl))
    groups = build_cascade_groups(td, ld, BS, HQ, HKV, device=qd.device)
    assert groups.num_groups == 1 and groups.max_prefix_len == PREFIX_BLOCKS * BS
    assert_close_to_oracle(paged_decode_attention_cascade(qd, kd, vd, td, ld, groups=groups), expected)
    assert_close_to_oracle(fd.decode(qd, kd, vd, td, ld), expected)
