"""C5 at full size: the 36-layer transactional DecodeEngine step, B64 ctx 8192.

Qwen2.5-3B attention shape (Hq16 / Hkv2 / D128, bf16, 32-token blocks),
context seeded to 8192 tokens per request (seed 109), one captured step
graph (RoPE + append fused into each layer's decode launch) replayed for 100
committed steps; step 100 runs eagerly with one layer's q malformed
(``q[..., :-1]``), which must abort the whole token and roll it back
(flashdec/integrated_workload.py:49-58, 699-712: LayerFailure, whole-token
rollback); one more graph step follows.

Checked against the oracle on several steps, for three layers x four rows:
- attention output within atol 2e-2 / rtol 1e-2 (fp32 oracle over the rows'
  blocks, q rotated at the pre-append position);
- the appended K bytes equal the reference's torch RoPE of k on the device
  (apply_rope, rope.py:66-82; the graph reads the cache's cos/sin table) and
  the V bytes equal v, bit for bit, at the slots the transaction reserved;
  the rotated K stays within tolerance of the oracle's correctly rounded RoPE.
The rollback must leave block tables, lengths and free/used counts as they
were before the aborted step; the cache's state version advances by two
(begin and abort each publish one, flashdec/cache.py:438-648).
"""

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import rope as orope
from tests.helpers import assert_close_to_oracle, device_rope, np32

pytestmark = pytest.mark.gpu

LAYERS, B, HQ, HKV, D, BS, CTX = 36, 64, 16, 2, 128, 32, 8192
STEPS = 102  # 100 committed graph steps, the aborted step 100, one graph step after it
CHECK_STEPS = (0, 57, 99, 101)
CHECK_LAYERS = (0, 17, 35)
CHECK_ROWS = (0, 21, 42, 63)


def bits(t):
    return t.detach().contiguous().view(torch.int16).cpu().numpy()


def check_step(cache, sg, tx, step):
    rows = list(CHECK_ROWS)
    pos = tx.positions.cpu().numpy()[rows]
    blk = tx.physical_block_ids.cpu().numpy()[rows]
    off = tx.block_offsets.cpu().numpy()[rows]
    tables = tx.block_tables[rows]
    lens = tx.effective_seq_lens.cpu().numpy()[rows]
    assert np.array_equal(lens, pos + 1) and np.all(pos == CTX + (step if step < 100 else step - 1))
    width = tables.shape[1]
    flat = tables.clamp(min=0).flatten().long()
    compact = np.arange(len(rows) * width, dtype=np.int32).reshape(len(rows), width)
    for layer in CHECK_LAYERS:
        k_in, v_in = sg.k[layer][rows], sg.v[layer][rows]
        # the step graph rotates with the cache's cos/sin table: apply_rope's bits on this device
        k_rot = device_rope(k_in, pos, base=1e6)
        assert np.allclose(k_rot, orope.apply_rope(np32(k_in), pos, base=1e6, out_dtype="bfloat16"),
                           atol=2e-2, rtol=1e-2)
        for i in range(len(rows)):
            got_k = cache.k_cache[layer][int(blk[i]), :, int(off[i])]
            got_v = cache.v_cache[layer][int(blk[i]), :, int(off[i])]
            assert np.array_equal(bits(got_k), bits(torch.from_numpy(k_rot[i]).to(torch.bfloat16))), (step, layer, i)
            assert np.array_equal(bits(got_v), bits(v_in[i])), (step, layer, i)
        q_rot = device_rope(sg.q[layer][rows], pos, base=1e6)
        kp = np32(cache.k_cache[layer][flat])
        vp = np32(cache.v_cache[layer][flat])
        expected = oa.paged_decode_attention(q_rot, kp, vp, compact, lens)
        assert_close_to_oracle(sg.out[layer][rows], expected)


def test_c5_full_size_engine_steps_with_rollback():
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine

    dev = "cuda"
    width = (CTX + STEPS + 2 + BS - 1) // BS
    cache = PagedKVCache(LAYERS, HKV, D, BS, max_blocks=B * width, dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev).manual_seed(109)
    for layer in range(LAYERS):
        cache.k_cache[layer].normal_(generator=gen)
        cache.v_cache[layer].normal_(generator=gen)
    cache.enable_graph_metadata(B, width)
    engine = DecodeEngine(cache)
    ids = list(range(B))
    for rid in ids:
        engine.add_request(rid)
    engine.admit()
    cache.seed_context(ids, CTX)
    sg = engine.capture_step_graph(B, HQ, base=1e6)
    assert sg.fused_rope and sg.out.shape == (LAYERS, B, HQ, D)
    checked = 0
    for step in range(STEPS):
        sg.q.normal_(generator=gen)
        sg.k.normal_(generator=gen)
        sg.v.normal_(generator=gen)
        if step == 100:
            bad = 7
            before = (cache.block_tables(ids).cpu(), cache.seq_lens_tensor(ids).cpu(), cache.num_free_blocks,
                      cache.num_used_blocks, cache.state_version)
            tx = engine.begin_step(ids)
            with pytest.raises(ValueError):
                for layer in range(LAYERS):
                    q = sg.q[layer][..., :-1] if layer == bad else sg.q[layer]
                    engine.step_layer(tx, layer, q, sg.k[layer], sg.v[layer], base=1e6)
            after = (cache.block_tables(ids).cpu(), cache.seq_lens_tensor(ids).cpu(), cache.num_free_blocks,
                     cache.num_used_blocks, cache.state_version)
            assert torch.equal(before[0], after[0]) and torch.equal(before[1], after[1])
            assert before[2:4] == after[2:4]
            assert after[4] == before[4] + 2
            assert engine.validate_invariants()
            continue
        tx = engine.begin_step(ids)
        engine.step_graph(tx, sg)
        if step in CHECK_STEPS:
            torch.cuda.synchronize()
            check_step(cache, sg, tx, step)
            checked += 1
        engine.commit_step(tx)
    torch.cuda.synchronize()
    assert checked == len(CHECK_STEPS)
    assert np.all(cache.seq_lens_tensor(ids).cpu().numpy() == CTX + STEPS - 1)
    assert engine.validate_invariants()
