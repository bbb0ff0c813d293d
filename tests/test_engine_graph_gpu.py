"""Whole-step hipGraph of the decode engine against eager per-layer steps.

Two engines start from identical caches.  One runs ``step_layer`` per layer;
the other replays a captured :class:`DecodeStepGraph`.  After every step:
- the appended K/V bytes of both caches must be identical;
- both engines' outputs must match the oracle within atol 2e-2 / rtol 1e-2
  (against fp32).
The batch's membership may change between steps as long as its size does.
The graph is checked with the split reducer kernel, with RoPE + append
fused into the decode launch, and with the in-launch merge (arrival
counters, which every replay leaves at zero).  A fused and an unfused graph
of identical engines must agree bit for bit.
"""

import pytest
import torch

from flashdec_amd.cache import PagedKVCache
from flashdec_amd.engine import DecodeEngine, DecodeStepGraph
from oracle import attention as oa
from oracle import rope as orope
from tests.helpers import assert_close_to_oracle

pytestmark = pytest.mark.gpu

L, HQ, HKV, D, BS = 3, 16, 2, 128, 16


def make_engine(arena=None):
    cache = PagedKVCache(L, HKV, D, BS, max_blocks=96, dtype=torch.bfloat16, device="cuda")
    g = torch.Generator(device="cuda").manual_seed(7)
    cache.k_cache.copy_(torch.randn(cache.k_cache.shape, device="cuda", generator=g))
    cache.v_cache.copy_(torch.randn(cache.v_cache.shape, device="cuda", generator=g))
    if arena:
        cache.enable_graph_metadata(*arena)
    return DecodeEngine(cache)


def admit(engine, ids, context):
    for rid in ids:
        engine.add_request(rid)
    engine.admit(ids)
    engine.cache.seed_context(ids, context)


def oracle_layer(cache, layer, q, tx_positions, tables, lens):
    q_rot = orope.apply_rope(q.float().cpu().numpy(), tx_positions.cpu().numpy(), base=1e6, out_dtype="bfloat16")
    return oa.paged_decode_attention(q_rot, cache.k_cache[layer].float().cpu().numpy(),
                                     cache.v_cache[layer].float().cpu().numpy(), tables.cpu().numpy(),
                                     lens.cpu().numpy())


@pytest.mark.parametrize(("merge", "fuse_rope"), [(False, False), (False, None), (True, None)])
def test_step_graph_matches_eager_steps(merge, fuse_rope):
    eager = make_engine()
    graphed = make_engine(arena=(4, 16))
    for e in (eager, graphed):
        admit(e, [0, 1, 2, 3], 40)
    sg = graphed.capture_step_graph(4, HQ, base=1e6, num_splits=3 if merge else None, merge=merge,
                                    fuse_rope=fuse_rope)
    assert isinstance(sg, DecodeStepGraph) and sg.out.shape == (L, 4, HQ, D)
    assert sg.fused_rope == (not merge and fuse_rope is None)  # by default fused wherever supported
    g = torch.Generator(device="cuda").manual_seed(11)
    for step in range(24):
        if step == 12:  # membership change at a fixed batch size
            for e in (eager, graphed):
                e.finish_request(0)
                admit(e, [9], 77)
        ids = eager.active_request_ids()
        assert ids == graphed.active_request_ids() and len(ids) == 4
        q = torch.randn((L, 4, HQ, D), device="cuda", generator=g).to(torch.bfloat16)
        k = torch.randn((L, 4, HKV, D), device="cuda", generator=g).to(torch.bfloat16)
        v = torch.randn((L, 4, HKV, D), device="cuda", generator=g).to(torch.bfloat16)
        tx_e = eager.begin_step(ids)
        eager_out = [eager.step_layer(tx_e, layer, q[layer], k[layer], v[layer], base=1e6).output
                     for layer in range(L)]
        tx_g = graphed.begin_step(ids)
        sg.q.copy_(q)
        sg.k.copy_(k)
        sg.v.copy_(v)
        graph_out = graphed.step_graph(tx_g, sg)
        torch.cuda.synchronize()
        assert torch.equal(tx_e.physical_block_ids, tx_g.physical_block_ids)
        if step % 4 == 3 or step == 12:
            for layer in range(L):
                expected = oracle_layer(graphed.cache, layer, q[layer], tx_g.positions, tx_g.block_tables,
                                        tx_g.effective_seq_lens)
                assert_close_to_oracle(graph_out[layer], expected)
                assert_close_to_oracle(eager_out[layer], expected)
        res_e = eager.commit_step(tx_e)
        res_g = graphed.commit_step(tx_g)
        assert torch.equal(res_e.seq_lens, res_g.seq_lens)
        assert res_g.output.data_ptr() == sg.out[-1].data_ptr()
    assert torch.equal(eager.cache.k_cache, graphed.cache.k_cache)
    assert torch.equal(eager.cache.v_cache, graphed.cache.v_cache)
    m = graphed.metrics()
    assert m["transaction_layer_step_count"] == 24 * L and m["cache"]["transaction_layer_write_count"] == 24 * L
    assert graphed.validate_invariants() and eager.validate_invariants()


@pytest.mark.parametrize("rotary_dim", [64, 128])
def test_fused_and_unfused_step_graphs_agree_bit_for_bit(rotary_dim):
    engines = [make_engine(arena=(4, 16)) for _ in range(2)]
    for e in engines:
        admit(e, [0, 1, 2, 3], 31)  # the first step's token opens a new block
    graphs = [e.capture_step_graph(4, HQ, rotary_dim=rotary_dim, base=5e5, fuse_rope=f)
              for e, f in zip(engines, (False, True))]
    assert not graphs[0].fused_rope and graphs[1].fused_rope
    g = torch.Generator(device="cuda").manual_seed(21)
    for step in range(6):
        q = torch.randn((L, 4, HQ, D), device="cuda", generator=g).to(torch.bfloat16)
        k = torch.randn((L, 4, HKV, D), device="cuda", generator=g).to(torch.bfloat16)
        v = torch.randn((L, 4, HKV, D), device="cuda", generator=g).to(torch.bfloat16)
        outs = []
        for e, sg in zip(engines, graphs):
            tx = e.begin_step()
            sg.q.copy_(q)
            sg.k.copy_(k)
            sg.v.copy_(v)
            outs.append(e.step_graph(tx, sg).clone())
            e.commit_step(tx)
        torch.cuda.synchronize()
        assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), step
    assert torch.equal(engines[0].cache.k_cache.view(torch.int16), engines[1].cache.k_cache.view(torch.int16))
    assert torch.equal(engines[0].cache.v_cache.view(torch.int16), engines[1].cache.v_cache.view(torch.int16))
    assert all(e.validate_invariants() for e in engines)


def test_fuse_rope_refused_where_unsupported():
    engine = make_engine(arena=(2, 8))
    admit(engine, ["a", "b"], 5)
    with pytest.raises(ValueError, match="fuse_rope needs"):
        engine.capture_step_graph(2, HQ, rotary_dim=96, fuse_rope=True)
    with pytest.raises(ValueError, match="fuse_rope needs"):
        engine.capture_step_graph(2, HQ, merge=True, num_splits=2, fuse_rope=True)
    assert not engine.capture_step_graph(2, HQ, rotary_dim=96).fused_rope


def test_step_graph_limits_abort_cleanly():
    engine = make_engine(arena=(2, 4))
    admit(engine, ["a", "b"], 64)  # 4 full blocks of 16; position 64 needs a 5th
    engine.capture_step_graph(2, HQ)
    with pytest.raises(RuntimeError, match="graph metadata arena"):
        engine.begin_step()
    assert engine.metrics()["open_step_transaction_count"] == 0
    assert engine.cache.request_state("a")["seq_len"] == 64 and engine.validate_invariants()

    small = make_engine(arena=(2, 8))
    admit(small, ["a", "b"], 5)
    one = small.capture_step_graph(1, HQ)
    tx = small.begin_step()
    with pytest.raises(ValueError, match="batch size does not match"):
        small.step_graph(tx, one)
    assert small.metrics()["transaction_abort_count"] == 1
    assert small.cache.request_state("a")["seq_len"] == 5 and small.validate_invariants()
