"""DecodeEngine and PagedKVCache transactions on the HIP path.

Each layer of each step is checked against the oracle: the rotated Q and the
appended K/V bytes bit for bit, the attention output within the
attention tolerance (atol 2e-2, rtol 1e-2 against fp32).  Forged caller views must not
steer a launch, and failures must roll the token back (the reference's
tests/test_multi_layer_engine.py:332-419, 541-570).
"""

from dataclasses import replace

import numpy as np
import pytest
import torch

from flashdec_amd.cache import PagedKVCache
from flashdec_amd.engine import DecodeEngine
from oracle import attention as oa
from oracle import rope as orope
from tests.helpers import assert_close_to_oracle, device_rope

pytestmark = pytest.mark.gpu


def as_bits(values, dtype=torch.bfloat16):
    """16-bit patterns of values that are exactly representable in ``dtype`` (numpy or tensor input)."""
    t = values if isinstance(values, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(values, np.float32))
    return t.detach().cpu().to(dtype).contiguous().view(torch.int16).numpy()


def cache_of(num_layers=2, hkv=2, d=128, bs=16, max_blocks=64, dtype=torch.bfloat16):
    return PagedKVCache(num_layers=num_layers, num_kv_heads=hkv, head_dim=d, block_size=bs, max_blocks=max_blocks,
                        dtype=dtype, device="cuda")


def rand_inputs(g, batch, hq, hkv, d, dtype):
    mk = lambda h: torch.randn(batch, h, d, generator=g).to(dtype).cuda()
    return mk(hq), mk(hkv), mk(hkv)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("hq,hkv,d,bs", [(16, 2, 128, 16), (4, 2, 64, 32), (8, 8, 128, 8)])
def test_engine_hip_layers_match_oracle(dtype, hq, hkv, d, bs):
    print(f"engine hip {dtype} hq={hq} hkv={hkv} d={d} bs={bs}", flush=True)
    num_layers = 3
    engine = DecodeEngine(cache_of(num_layers, hkv, d, bs, max_blocks=64, dtype=dtype))
    assert (engine.append_backend, engine.decode_backend) == ("fused_hip", "hip")
    ids = ["r0", "r1", "r2"]
    for rid in ids:
        engine.add_request(rid)
    engine.admit()
    g = torch.Generator().manual_seed(hq * 100 + bs)
    name = "bfloat16" if dtype == torch.bfloat16 else "float16"
    for step in range(2 * bs + 3):
        tx = engine.begin_step(ids)
        pos = tx.positions.cpu().numpy()
        for layer in range(num_layers):
            q, k, v = rand_inputs(g, 3, hq, hkv, d, dtype)
            res = engine.step_layer(tx, layer, q, k, v, base=1e6)
            if step % 5 and step != 2 * bs + 2:
                continue  # full comparison on a subset of steps keeps the test short
            torch.cuda.synchronize()
            kc = engine.cache.k_cache[layer].float().cpu().numpy()
            vc = engine.cache.v_cache[layer].float().cpu().numpy()
            # the cache's cos/sin tables: apply_rope's bits on this device
            q_rot = device_rope(q, pos, base=1e6)
            k_rot = device_rope(k, pos, base=1e6)
            # and within the per-frequency bound of the correctly rounded RoPE
            assert np.allclose(k_rot, orope.apply_rope(k.float().cpu().numpy(), pos, base=1e6, out_dtype=name),
                               atol=2e-2, rtol=1e-2)
            blk, off = tx.physical_block_ids.tolist(), tx.block_offsets.tolist()
            for row in range(3):
                assert np.array_equal(as_bits(kc[blk[row], :, off[row]], dtype), as_bits(k_rot[row], dtype))
                assert np.array_equal(as_bits(vc[blk[row], :, off[row]], dtype), as_bits(v[row], dtype))
            expected = oa.paged_decode_attention(q_rot, kc, vc, tx.block_tables.cpu().numpy(),
                                                 tx.effective_seq_lens.cpu().numpy())
            assert_close_to_oracle(res.output, expected)
        engine.commit_step(tx)
    assert engine.cache.seq_lens_tensor(ids).tolist() == [2 * bs + 3] * 3
    assert engine.validate_invariants()


def test_layers_with_different_head_counts_take_their_own_launch():
    """A later layer whose q has another head count than the step's earlier layers must not
    reuse their prepared RoPE + append or fused-decode arguments (which fix the head count):
    every layer is checked against the oracle, and the appended K / V bytes bit for bit."""
    num_layers, hkv, d, bs = 5, 2, 128, 16
    engine = DecodeEngine(cache_of(num_layers, hkv, d, bs, max_blocks=64))
    ids = ["a", "b", "c"]
    for rid in ids:
        engine.add_request(rid)
    engine.admit()
    g = torch.Generator().manual_seed(777)
    for step in range(3):
        tx = engine.begin_step(ids)
        pos = tx.positions.cpu().numpy()
        for layer, hq in enumerate((16, 8, 4, 16, 2)):
            print(f"head counts: step {step} layer {layer} hq {hq}", flush=True)
            q, k, v = rand_inputs(g, 3, hq, hkv, d, torch.bfloat16)
            res = engine.step_layer(tx, layer, q, k, v, base=1e6)
            torch.cuda.synchronize()
            assert res.output.shape == q.shape
            kc = engine.cache.k_cache[layer].float().cpu().numpy()
            vc = engine.cache.v_cache[layer].float().cpu().numpy()
            k_rot = device_rope(k, pos, base=1e6)
            blk, off = tx.physical_block_ids.tolist(), tx.block_offsets.tolist()
            for row in range(3):
                assert np.array_equal(as_bits(kc[blk[row], :, off[row]]), as_bits(k_rot[row]))
                assert np.array_equal(as_bits(vc[blk[row], :, off[row]]), as_bits(v[row]))
            expected = oa.paged_decode_attention(device_rope(q, pos, base=1e6), kc, vc,
                                                 tx.block_tables.cpu().numpy(), tx.effective_seq_lens.cpu().numpy())
            assert_close_to_oracle(res.output, expected)
        engine.commit_step(tx)
    assert engine.validate_invariants()


def test_forged_views_do_not_steer_the_fused_write():
    cache = cache_of(num_layers=2, bs=2, max_blocks=4)
    cache.add_request("r")
    tx = cache.begin_token(["r"])
    true_block = tx.physical_block_ids.item()
    forged = replace(tx, positions=torch.full_like(tx.positions, 5),
                     physical_block_ids=torch.full_like(tx.physical_block_ids, cache.max_blocks - 1),
                     block_offsets=torch.full_like(tx.block_offsets, cache.block_size - 1))
    g = torch.Generator().manual_seed(690)
    for layer in range(2):
        q, k, v = rand_inputs(g, 1, 4, 2, 128, torch.bfloat16)
        q_rot, latest = cache.write_token_layer_fused_cuda(forged, layer, q, k, v)
        torch.cuda.synchronize()
        exp_q = orope.apply_rope(q.float().cpu().numpy(), [0], out_dtype="bfloat16")
        exp_k = orope.apply_rope(k.float().cpu().numpy(), [0], out_dtype="bfloat16")
        assert np.array_equal(as_bits(q_rot), as_bits(exp_q))
        assert np.array_equal(as_bits(cache.k_cache[layer, true_block, :, 0]), as_bits(exp_k[0]))
        assert torch.equal(cache.v_cache[layer, true_block, :, 0], v[0])
        assert latest.next_layer_idx == layer + 1
    assert not cache.k_cache[:, cache.max_blocks - 1].any()
    cache.commit_token(forged)
    assert cache.request_block_ids("r") == (true_block,)
    assert cache.validate_invariants()


def test_fused_write_failure_rolls_back_reserved_block():
    engine = DecodeEngine(cache_of(num_layers=2, bs=1, max_blocks=2))
    engine.add_request("r")
    engine.admit()
    tx = engine.begin_step(["r"])
    assert engine.cache.num_used_blocks == 1
    g = torch.Generator().manual_seed(1)
    q, k, v = rand_inputs(g, 1, 4, 2, 128, torch.bfloat16)
    q_strided = torch.empty(1, 4, 256, device="cuda", dtype=torch.bfloat16)[..., ::2]
    q_strided.copy_(q)
    with pytest.raises(ValueError, match="contiguous"):
        engine.step_layer(tx, 0, q_strided, k, v)
    assert engine.cache.num_used_blocks == 0 and engine.cache.request_block_ids("r") == ()
    assert engine.metrics()["transaction_abort_count"] == 1
    assert engine.validate_invariants()


def test_engine_abort_mid_token_then_continue():
    engine = DecodeEngine(cache_of(num_layers=3, bs=16, max_blocks=8))
    for rid in (1, 2):
        engine.add_request(rid)
    engine.admit()
    g = torch.Generator().manual_seed(4)
    for step in range(20):
        tx = engine.begin_step()
        layers = 3 if step % 7 != 6 else 1
        for layer in range(layers):
            engine.step_layer(tx, layer, *rand_inputs(g, 2, 16, 2, 128, torch.bfloat16))
        if layers == 3:
            engine.commit_step(tx)
        else:
            engine.abort_step(tx)
    torch.cuda.synchronize()
    committed = 20 - len([s for s in range(20) if s % 7 == 6])
    assert engine.cache.seq_lens_tensor([1, 2]).tolist() == [committed, committed]
    assert engine.metrics()["transaction_abort_count"] == 2
    assert engine.validate_invariants()


@pytest.mark.parametrize("table", [False, True])
@pytest.mark.parametrize("rotary_dim", [None, 64])
@pytest.mark.parametrize("hq,bs", [(16, 16), (8, 32), (2, 8)])
def test_eager_layers_with_rope_in_the_decode_launch_match_two_launches(hq, bs, rotary_dim, table):
    """Eager steps: layers after the first run RoPE + K/V write inside the decode launch; outputs and cache
    bytes equal the two-launch path's bit for bit, over steps that cross block boundaries."""
    from flashdec_amd.rope import rope_cos_sin_table

    print(f"eager fused hq={hq} bs={bs} rotary_dim={rotary_dim} table={table}", flush=True)
    num_layers, hkv, d = 4, 2, 128
    engines = []
    for fuse in (False, True):
        e = DecodeEngine(cache_of(num_layers, hkv, d, bs, max_blocks=96))
        e.eager_fuse_rope = fuse
        for rid in ("a", "b", "c"):
            e.add_request(rid)
        e.admit()
        engines.append(e)
    tab = rope_cos_sin_table(256, rotary_dim or d, base=1e6) if table else None
    g = torch.Generator().manual_seed(hq + bs)
    fused_layers = 0
    for step in range(bs + 3):
        txs = [e.begin_step(["a", "b", "c"]) for e in engines]
        for layer in range(num_layers):
            q, k, v = rand_inputs(g, 3, hq, hkv, d, torch.bfloat16)
            outs = [e.step_layer(tx, layer, q, k, v, rotary_dim=rotary_dim, base=1e6, cos_sin_table=tab).output
                    for e, tx in zip(engines, txs)]
            fused_layers += engines[1]._open.fused_launch is not None and layer > 0
            assert engines[0]._open.fused_launch is None
            assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), (step, layer)
        for e, tx in zip(engines, txs):
            e.commit_step(tx)
    assert fused_layers == (bs + 3) * (num_layers - 1)
    torch.cuda.synchronize()
    for a, b in ((engines[0].cache.k_cache, engines[1].cache.k_cache),
                 (engines[0].cache.v_cache, engines[1].cache.v_cache)):
        assert torch.equal(a.view(torch.int16), b.view(torch.int16))
    assert engines[1].validate_invariants()
    assert engines[0].metrics() == engines[1].metrics()


def test_eager_fused_layers_follow_a_rope_setting_that_changes_within_the_step():
    """Layers 0-1 rotate all 128 dims, layers 2-3 the first 64, layer 4 a different base: the layers that
    run RoPE inside the decode launch use each layer's own setting (bits equal to the two-launch path)."""
    settings = [(None, 1e6), (None, 1e6), (64, 1e6), (64, 1e6), (64, 1e4)]
    engines = []
    for fuse in (False, True):
        e = DecodeEngine(cache_of(len(settings), 2, 128, 16, max_blocks=32))
        e.eager_fuse_rope = fuse
        e.add_request("a")
        e.add_request("b")
        e.admit()
        engines.append(e)
    g = torch.Generator().manual_seed(5)
    for step in range(3):
        txs = [e.begin_step(["a", "b"]) for e in engines]
        for layer, (rdim, base) in enumerate(settings):
            q, k, v = rand_inputs(g, 2, 16, 2, 128, torch.bfloat16)
            outs = [e.step_layer(tx, layer, q, k, v, rotary_dim=rdim, base=base).output for e, tx in zip(engines, txs)]
            assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16)), (step, layer)
        for e, tx in zip(engines, txs):
            e.commit_step(tx)
    torch.cuda.synchronize()
    assert torch.equal(engines[0].cache.k_cache.view(torch.int16), engines[1].cache.k_cache.view(torch.int16))
