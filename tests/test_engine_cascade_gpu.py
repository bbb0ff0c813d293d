"""Decode engine over a registered shared prefix, with the cascade path.

Requests attached to one resident prefix (``DecodeEngine.admit(...,
prefix_id=...)``, flashdec/cache.py:192-276) lead their tables with the
prefix's blocks.  Eager steps decode them with the shared-prefix launch once
the group is large enough; every layer's output must match the oracle and an
engine that decodes row by row.  Tolerance: atol 2e-2 / rtol 1e-2.
"""

import pytest
import torch

from flashdec_amd.cache import PagedKVCache
from flashdec_amd.engine import DecodeEngine
from oracle import attention as oa
from oracle import rope as orope
from tests.helpers import assert_close_to_oracle

pytestmark = pytest.mark.gpu

L, HQ, HKV, D, BS = 2, 16, 2, 128, 16
PREFIX_BLOCKS = 6


def make_engine(min_shared):
    cache = PagedKVCache(L, HKV, D, BS, max_blocks=128, dtype=torch.bfloat16, device="cuda",
                         prefix_cache_capacity_blocks=PREFIX_BLOCKS)
    g = torch.Generator(device="cuda").manual_seed(21)
    cache.k_cache.copy_(torch.randn(cache.k_cache.shape, device="cuda", generator=g))
    cache.v_cache.copy_(torch.randn(cache.v_cache.shape, device="cuda", generator=g))
    engine = DecodeEngine(cache)
    engine.cascade_min_shared_tokens = min_shared
    shape = (L, PREFIX_BLOCKS, HKV, BS, D)
    pk = torch.randn(shape, device="cuda", generator=g).to(torch.bfloat16)
    pv = torch.randn(shape, device="cuda", generator=g).to(torch.bfloat16)
    engine.register_prefix("sys", pk, pv)
    for rid in ("a", "b", "c", "d", "solo"):
        engine.add_request(rid)
    engine.admit(["a", "b", "c", "d"], prefix_id="sys")
    engine.admit(["solo"])
    cache.seed_context(["solo"], 37)
    for rid, n in (("a", 3), ("b", 20), ("c", 1), ("d", 9)):
        cache.seed_context([rid], n)
    return engine


def test_prefix_group_decodes_with_the_cascade():
    cascaded, per_row = make_engine(1), make_engine(None)
    g = torch.Generator(device="cuda").manual_seed(5)
    for step in range(4):
        ids = cascaded.active_request_ids()
        assert ids == per_row.active_request_ids()
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
                    q_rot = orope.apply_rope(q[layer].float().cpu().numpy(), tx.positions.cpu().numpy(), base=1e6,
                                             out_dtype="bfloat16")
                    expected = oa.paged_decode_attention(q_rot, e.cache.k_cache[layer].float().cpu().numpy(),
                                                         e.cache.v_cache[layer].float().cpu().numpy(),
                                                         tx.block_tables.cpu().numpy(),
                                                         tx.effective_seq_lens.cpu().numpy())
                    assert_close_to_oracle(outs[0][layer], expected)
            e.commit_step(tx)
        for layer in range(L):
            assert_close_to_oracle(outs[0][layer], outs[1][layer].float().cpu().numpy())
    assert cascaded._cascade_decode_count == 4 * L and per_row._cascade_decode_count == 0
    assert torch.equal(cascaded.cache.k_cache, per_row.cache.k_cache)
    assert cascaded.validate_invariants() and per_row.validate_invariants()
