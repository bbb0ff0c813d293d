"""RoPE against the reference's own torch expression on the device.

The reference rotates with fp32 torch ops (flashdec/rope.py:66-82: ``pow``,
``cos``, ``sin``, then ``x1*c - x2*s`` / ``x2*c + x1*s``), so its bits depend
on the device's fp32 ``pow``/``cos``/``sin``.  The kernels' default mode uses
the correctly rounded values instead (bit-exact against the CPU oracle, tested
elsewhere); their table mode reads cos/sin from
``rope_cos_sin_table`` -- that same torch expression evaluated on this device
-- and must then equal ``apply_rope`` on this device bit for bit: q_out, the
appended K bytes, in the RoPE + append kernel, the decode launch's fused RoPE
and a whole engine step.  The default mode's mismatch count against torch at
C3 is measured and bounded here.
"""

import math

import numpy as np
import pytest
import torch

from oracle import attention as oa
from tests.helpers import assert_close_to_oracle, np32, rope_pair_bound

pytestmark = pytest.mark.gpu


def c3_inputs(dtype=torch.bfloat16, rotary_dim=128, max_pos=8191, seed=251):
    """C3: B64, Hq16 / Hkv2, D128, theta 1e6, positions U{1..max_pos}, 32-token blocks.

    Each row appends at offset pos % 32 of its own block (distinct blocks of a
    small pool: only the slots matter here).
    """
    b, hq, hkv, d, bs, pool = 64, 16, 2, 128, 32, 128
    gen = torch.Generator().manual_seed(seed)
    pos = torch.randint(1, max_pos + 1, (b,), generator=gen)
    blk = torch.randperm(pool, generator=gen)[:b]
    off = pos % bs
    q = torch.randn((b, hq, d), generator=gen).to(dtype)
    k = torch.randn((b, hkv, d), generator=gen).to(dtype)
    v = torch.randn((b, hkv, d), generator=gen).to(dtype)
    kc = torch.zeros((pool, hkv, bs, d), dtype=dtype, device="cuda")
    dev = "cuda"
    return (q.to(dev), k.to(dev), v.to(dev), kc, kc.clone(), blk.to(dev), off.to(dev), pos.to(dev), rotary_dim)


def ulp_distance(a, b):
    """Per-element distance in units of the last place of two same-dtype tensors (16- or 32-bit floats)."""
    width = {2: (torch.int16, 0x7FFF), 4: (torch.int32, 0x7FFFFFFF)}[a.element_size()]
    ia = a.contiguous().view(width[0]).to(torch.int64)
    ib = b.contiguous().view(width[0]).to(torch.int64)
    # map sign-magnitude bit patterns onto a monotone integer line
    ia = torch.where(ia < 0, -(ia & width[1]), ia)
    ib = torch.where(ib < 0, -(ib & width[1]), ib)
    return (ia - ib).abs()


def test_default_mode_against_torch_at_c3_is_counted_and_small():
    import flashdec_amd as fd
    from flashdec_amd.rope import apply_rope

    q, k, v, kc, vc, blk, off, pos, r = c3_inputs()
    q_out = fd.fused_rope_kv_append(q, k, v, kc, vc, blk, off, pos, base=1e6)
    ref_q = apply_rope(q, pos, base=1e6)
    ref_k = apply_rope(k, pos, base=1e6)
    got_k = kc[blk, :, off]
    nq, nk = int((ulp_distance(q_out, ref_q) > 0).sum()), int((ulp_distance(got_k, ref_k) > 0).sum())
    print(f"default mode vs torch apply_rope at C3: q_out {nq}/{q_out.numel()} elements differ, "
          f"K {nk}/{got_k.numel()}")
    # torch's fp32 pow/cos/sin are within an ulp of the correctly rounded
    # values; inside the angle an ulp of inv_i is multiplied by the position,
    # so each element may differ by the per-frequency bound of the fp32
    # algorithm plus one bf16 ulp of the result (<= 2^-7 |ref|)
    p = pos.cpu().numpy()
    for x, got, ref in ((q, q_out, ref_q), (k, got_k, ref_k)):
        diff = (got.float() - ref.float()).abs().cpu().numpy()
        bound = 2.0**-7 * np.abs(np32(ref)) + rope_pair_bound(np32(x), p, 128, 1e6)
        assert (diff <= bound).all(), float((diff - bound).max())
    assert nq <= q_out.numel() // 20 and nk <= got_k.numel() // 20
    assert torch.equal(vc[blk, :, off], v)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize(("rotary_dim", "max_pos"), [(128, 8191), (64, 32767)])
def test_table_mode_equals_torch_apply_rope_bit_for_bit(dtype, rotary_dim, max_pos):
    import flashdec_amd as fd
    from flashdec_amd.rope import apply_rope, rope_cos_sin_table

    q, k, v, kc, vc, blk, off, pos, r = c3_inputs(dtype, rotary_dim, max_pos)
    tab = rope_cos_sin_table(max_pos + 1, rotary_dim, 1e6, device="cuda")
    q_out = fd.fused_rope_kv_append(q, k, v, kc, vc, blk, off, pos, rotary_dim=rotary_dim, base=1e6,
                                    cos_sin_table=tab)
    assert int(ulp_distance(q_out, apply_rope(q, pos, rotary_dim=rotary_dim, base=1e6)).max()) == 0
    assert int(ulp_distance(kc[blk, :, off], apply_rope(k, pos, rotary_dim=rotary_dim, base=1e6)).max()) == 0
    assert torch.equal(vc[blk, :, off], v)


def test_table_mode_rejects_positions_past_the_table():
    import flashdec_amd as fd
    from flashdec_amd.rope import rope_cos_sin_table

    q, k, v, kc, vc, blk, off, pos, r = c3_inputs()
    tab = rope_cos_sin_table(int(pos.max()), 128, 1e6, device="cuda")  # one row short of the largest position
    with pytest.raises(ValueError, match="cos_sin_table"):
        fd.fused_rope_kv_append(q, k, v, kc, vc, blk, off, pos, base=1e6, cos_sin_table=tab)
    with pytest.raises(ValueError, match="shape"):
        fd.fused_rope_kv_append(q, k, v, kc, vc, blk, off, pos, rotary_dim=64, base=1e6, cos_sin_table=tab)


@pytest.mark.parametrize("table", ["default", "explicit"])
@pytest.mark.parametrize("graph", [False, True])
def test_engine_step_in_table_mode_equals_torch_rope(graph, table):
    """Eager steps (RoPE + append kernel, then RoPE fused into the decode launch) and a step
    graph (RoPE fused into the decode launch) rotate with a cos/sin table: the caller's, or
    by default (no table passed) the cache's own.  Appended K equals apply_rope on the
    device bit for bit (the reference's rope.py:66-82 expression)."""
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine
    from flashdec_amd.rope import apply_rope, rope_cos_sin_table

    layers, b, hq, hkv, d, bs, ctx = 3, 8, 16, 2, 128, 32, 5000
    width = (ctx + 8 + bs - 1) // bs
    cache = PagedKVCache(layers, hkv, d, bs, max_blocks=b * width, dtype=torch.bfloat16, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(3)
    cache.k_cache.normal_(generator=g)
    cache.v_cache.normal_(generator=g)
    if graph:
        cache.enable_graph_metadata(b, width)
    engine = DecodeEngine(cache)
    ids = list(range(b))
    for rid in ids:
        engine.add_request(rid)
    engine.admit()
    cache.seed_context(ids, ctx)
    tab = rope_cos_sin_table(width * bs, d, 1e6, device="cuda") if table == "explicit" else None
    sg = engine.capture_step_graph(b, hq, base=1e6, cos_sin_table=tab) if graph else None
    if graph:
        assert sg.fused_rope and sg.cos_sin_table is (tab if table == "explicit" else cache.rope_table(d, 1e6))
        assert sg.cos_sin_table.shape[1] >= width * bs
    for step in range(3):
        q = torch.randn((layers, b, hq, d), device="cuda", generator=g).to(torch.bfloat16)
        k = torch.randn((layers, b, hkv, d), device="cuda", generator=g).to(torch.bfloat16)
        v = torch.randn((layers, b, hkv, d), device="cuda", generator=g).to(torch.bfloat16)
        tx = engine.begin_step(ids)
        if graph:
            sg.q.copy_(q)
            sg.k.copy_(k)
            sg.v.copy_(v)
            engine.step_graph(tx, sg)
            outs = [sg.out[layer] for layer in range(layers)]
        else:
            extra = {} if tab is None else {"cos_sin_table": tab}
            outs = [engine.step_layer(tx, layer, q[layer], k[layer], v[layer], base=1e6, **extra).output
                    for layer in range(layers)]
        torch.cuda.synchronize()
        blk, off = tx.physical_block_ids, tx.block_offsets
        for layer in range(layers):
            k_rot = apply_rope(k[layer], tx.positions, base=1e6)
            assert int(ulp_distance(cache.k_cache[layer][blk, :, off], k_rot).max()) == 0, (step, layer)
            assert torch.equal(cache.v_cache[layer][blk, :, off], v[layer])
            q_rot = apply_rope(q[layer], tx.positions, base=1e6)
            expected = oa.paged_decode_attention(np32(q_rot), np32(cache.k_cache[layer]), np32(cache.v_cache[layer]),
                                                 tx.block_tables.cpu().numpy(), tx.effective_seq_lens.cpu().numpy(),
                                                 sm_scale=1.0 / math.sqrt(d))
            assert_close_to_oracle(outs[layer], expected)
        engine.commit_step(tx)
    assert np.all(cache.seq_lens_tensor(ids).cpu().numpy() == ctx + 3)


def test_default_engine_steps_equal_the_torch_append_backend_bit_for_bit():
    """No table passed anywhere: the default HIP engine (RoPE + append kernel on layer 0, RoPE
    fused into the decode launch on later layers) and an engine whose append is the torch
    backend (apply_rope, then a torch scatter; the reference's rope_paged_kv_append_ref path)
    give the same attention outputs and the same cache bytes, bit for bit: q is rotated
    exactly as apply_rope rotates it, since the output is a deterministic function of the
    rotated q's bits.  The cache's fused write returns q_rot itself, checked against apply_rope."""
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine
    from flashdec_amd.rope import apply_rope

    layers, b, hq, hkv, d, bs, ctx = 3, 6, 16, 2, 128, 32, 3000
    width = (ctx + 8 + bs - 1) // bs
    engines = []
    for backend in ("fused_cuda", "torch"):
        cache = PagedKVCache(layers, hkv, d, bs, max_blocks=b * width, dtype=torch.bfloat16, device="cuda")
        g = torch.Generator(device="cuda").manual_seed(5)
        cache.k_cache.normal_(generator=g)
        cache.v_cache.normal_(generator=g)
        engine = DecodeEngine(cache, append_backend=backend)
        for rid in range(b):
            engine.add_request(rid)
        engine.admit()
        cache.seed_context(list(range(b)), ctx)
        engines.append(engine)
    g = torch.Generator(device="cuda").manual_seed(6)
    ids = list(range(b))
    for step in range(4):
        q = torch.randn((layers, b, hq, d), device="cuda", generator=g).to(torch.bfloat16)
        k = torch.randn((layers, b, hkv, d), device="cuda", generator=g).to(torch.bfloat16)
        v = torch.randn((layers, b, hkv, d), device="cuda", generator=g).to(torch.bfloat16)
        outs = []
        for engine in engines:
            tx = engine.begin_step(ids)
            outs.append([engine.step_layer(tx, layer, q[layer], k[layer], v[layer], base=1e6).output
                         for layer in range(layers)])
            engine.commit_step(tx)
        torch.cuda.synchronize()
        for layer in range(layers):
            assert torch.equal(outs[0][layer].view(torch.int16), outs[1][layer].view(torch.int16)), (step, layer)
    fused, ref = (e.cache for e in engines)
    assert torch.equal(fused.k_cache.view(torch.int16), ref.k_cache.view(torch.int16))
    assert torch.equal(fused.v_cache.view(torch.int16), ref.v_cache.view(torch.int16))
    # the cache's fused write hands back q_rot: apply_rope's bits
    tx = fused.begin_token(ids)
    pos = torch.as_tensor(fused.transaction_view(tx).positions, device="cuda")
    q_rot, _ = fused.write_token_layer_fused_cuda(tx, 0, q[0], k[0], v[0], base=1e6)
    assert torch.equal(q_rot.view(torch.int16), apply_rope(q[0], pos, base=1e6).view(torch.int16))
    fused.abort_token(tx)


def test_short_table_raises_in_eager_steps_and_aborts_the_step():
    """A caller's table without a row for every position of the step raises before any launch
    (the kernels would clamp to the last row) and aborts the token."""
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine
    from flashdec_amd.rope import rope_cos_sin_table

    cache = PagedKVCache(2, 2, 128, 32, max_blocks=64, dtype=torch.bfloat16, device="cuda")
    engine = DecodeEngine(cache)
    ids = [0, 1]
    for rid in ids:
        engine.add_request(rid)
    engine.admit()
    cache.seed_context(ids, 100)  # positions 100
    short = rope_cos_sin_table(100, 128, 1e6, device="cuda")  # rows 0..99
    q = torch.randn((2, 16, 128), device="cuda").to(torch.bfloat16)
    k = torch.randn((2, 2, 128), device="cuda").to(torch.bfloat16)
    for layer_with_short in (0, 1):
        before = (cache.seq_lens_tensor(ids).cpu(), cache.num_free_blocks, cache.state_version)
        tx = engine.begin_step(ids)
        with pytest.raises(ValueError, match="cos_sin_table"):
            for layer in range(2):
                extra = {"cos_sin_table": short} if layer == layer_with_short else {}
                engine.step_layer(tx, layer, q, k, k, base=1e6, **extra)
        assert torch.equal(cache.seq_lens_tensor(ids).cpu(), before[0]) and cache.num_free_blocks == before[1]
        assert cache.state_version == before[2] + 2
    long = rope_cos_sin_table(101, 128, 1e6, device="cuda")
    tx = engine.begin_step(ids)
    for layer in range(2):
        engine.step_layer(tx, layer, q, k, k, base=1e6, cos_sin_table=long)
    engine.commit_step(tx)
    assert engine.validate_invariants()
