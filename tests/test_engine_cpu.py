"""DecodeEngine on a CPU cache (torch append + reference decode backends).

Layer outputs are checked against the numpy oracle (RoPE of the pre-append
position, then paged attention over the cache including the new token).
Lifecycle scenarios follow the reference's tests/test_multi_layer_engine.py
and tests/test_decode_engine.py.
"""

from dataclasses import replace

import numpy as np
import pytest
import torch

from flashdec_amd.cache import PagedKVCache
from flashdec_amd.engine import DecodeEngine, DecodeLayerResult, DecodeStepResult, DecodeStepTransaction
from flashdec_amd.rope import apply_rope
from oracle import attention as oracle_attn
from oracle import rope as oracle_rope


def make_cache(num_layers=2, block_size=2, max_blocks=4, head_dim=4, num_kv_heads=1):
    return PagedKVCache(num_layers=num_layers, num_kv_heads=num_kv_heads, head_dim=head_dim, block_size=block_size,
                        max_blocks=max_blocks, dtype=torch.float32, device="cpu")


def inputs(batch, seed, hq=2, hkv=1, d=4):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(batch, hq, d, generator=g), torch.randn(batch, hkv, d, generator=g),
            torch.randn(batch, hkv, d, generator=g))


def oracle_layer(cache, layer, q, positions, block_tables, eff_lens):
    qr = oracle_rope.apply_rope(q.numpy(), positions.numpy())
    return oracle_attn.paged_decode_attention(qr, cache.k_cache[layer].numpy(), cache.v_cache[layer].numpy(),
                                              block_tables.numpy(), eff_lens.numpy())


@pytest.mark.parametrize("num_layers", [2, 4])
def test_multi_layer_outputs_match_oracle_and_commit_once(num_layers):
    engine = DecodeEngine(make_cache(num_layers=num_layers, max_blocks=8))
    assert (engine.append_backend, engine.decode_backend) == ("torch", "reference")
    engine.add_request(20)
    engine.add_request(10)
    engine.admit()
    for step in range(3):
        tx = engine.begin_step([20, 10])
        assert isinstance(tx, DecodeStepTransaction)
        assert tx.positions.tolist() == [step, step]
        assert tx.effective_seq_lens.tolist() == [step + 1, step + 1]
        for layer in range(num_layers):
            q, k, v = inputs(2, 100 * step + layer)
            res = engine.step_layer(tx, layer, q, k, v)
            assert isinstance(res, DecodeLayerResult) and res.layer_idx == layer
            expected = oracle_layer(engine.cache, layer, q, tx.positions, tx.block_tables, tx.effective_seq_lens)
            np.testing.assert_allclose(res.output.numpy(), expected, atol=1e-5, rtol=1e-5)
            # the new K was rotated at its position before landing in the cache
            blk, off = tx.physical_block_ids.tolist(), tx.block_offsets.tolist()
            k_expected = oracle_rope.apply_rope(k.numpy(), tx.positions.numpy())
            for row in range(2):
                np.testing.assert_allclose(engine.cache.k_cache[layer, blk[row], :, off[row]].numpy(),
                                           k_expected[row], atol=1e-6)
                assert torch.equal(engine.cache.v_cache[layer, blk[row], :, off[row]], v[row])
            assert engine.cache.seq_lens_tensor([20, 10]).tolist() == [step, step]
        result = engine.commit_step(tx)
        assert isinstance(result, DecodeStepResult) and result.status == DecodeEngine.STEP_OK
        assert result.seq_lens.tolist() == [step + 1, step + 1]
    m = engine.metrics()
    assert m["completed_step_count"] == 3 and m["appended_token_count"] == 6
    assert m["transaction_layer_step_count"] == 3 * num_layers
    assert m["cache"]["transaction_commit_count"] == 3
    assert engine.validate_invariants()


def test_layer_failure_aborts_whole_token():
    engine = DecodeEngine(make_cache(num_layers=2, block_size=1, max_blocks=1))
    engine.add_request("r")
    engine.admit()
    tx = engine.begin_step(["r"])
    q, k, v = inputs(1, 611)
    engine.step_layer(tx, 0, q, k, v)
    with pytest.raises(ValueError, match="q shape"):
        engine.step_layer(tx, 1, torch.ones(1, 2, 3), k, v)
    assert engine.cache.request_state("r")["seq_len"] == 0
    assert engine.cache.request_block_ids("r") == () and engine.cache.num_used_blocks == 0
    m = engine.metrics()
    assert (m["transaction_abort_count"], m["open_step_transaction_count"]) == (1, 0)
    with pytest.raises(RuntimeError, match="no open"):
        engine.abort_step(tx)
    assert engine.validate_invariants()


def test_early_commit_stays_open_until_abort():
    engine = DecodeEngine(make_cache(num_layers=2))
    engine.add_request(1)
    engine.admit()
    tx = engine.begin_step([1])
    engine.step_layer(tx, 0, *inputs(1, 613))
    with pytest.raises(RuntimeError, match="before all layers"):
        engine.commit_step(tx)
    assert engine.metrics()["open_step_transaction_count"] == 1
    assert engine.abort_step(tx).state == "aborted"
    assert engine.cache.request_state(1)["seq_len"] == 0
    assert engine.validate_invariants()


def test_stale_handle_rejected_without_aborting_owner():
    engine = DecodeEngine(make_cache(num_layers=2))
    engine.add_request(1)
    engine.admit()
    tx = engine.begin_step([1])
    with pytest.raises(RuntimeError, match="stale or invalid"):
        engine.step_layer(replace(tx, engine_version=tx.engine_version + 1), 0, *inputs(1, 615))
    assert engine.metrics()["open_step_transaction_count"] == 1
    with pytest.raises(RuntimeError, match="requires layer 0"):
        engine.step_layer(tx, 1, *inputs(1, 616))
    # an out-of-order layer is a layer error: the token is aborted
    assert engine.metrics()["open_step_transaction_count"] == 0
    assert engine.validate_invariants()


def test_open_step_blocks_lifecycle_calls():
    engine = DecodeEngine(make_cache(num_layers=2))
    engine.add_request("active")
    engine.add_request("waiting")
    engine.admit(["active"])
    tx = engine.begin_step(["active"])
    q, k, v = inputs(1, 617)
    for action in (lambda: engine.add_request("new"), lambda: engine.admit(["waiting"]),
                   lambda: engine.finish_request("active"), lambda: engine.cancel_request("active"),
                   lambda: engine.step(q, k, v, ["active"]), lambda: engine.begin_step(["active"])):
        with pytest.raises(RuntimeError, match="open decode step transaction"):
            action()
    engine.abort_step(tx)
    assert engine.admit(["waiting"])[0].status == DecodeEngine.ACTIVE
    assert engine.validate_invariants()


def test_fused_backend_on_cpu_cache_aborts_transaction():
    engine = DecodeEngine(make_cache(num_layers=2), append_backend="fused_cuda")
    engine.add_request(1)
    engine.admit()
    tx = engine.begin_step([1])
    with pytest.raises(ValueError, match="CUDA-resident"):
        engine.step_layer(tx, 0, *inputs(1, 621))
    assert engine.cache.num_used_blocks == 0
    m = engine.metrics()
    assert (m["transaction_abort_count"], m["open_step_transaction_count"]) == (1, 0)
    assert engine.validate_invariants()


def test_fused_transaction_routes_through_cache_api(monkeypatch):
    engine = DecodeEngine(make_cache(num_layers=2), append_backend="fused_cuda", decode_backend="reference")
    engine.add_request(1)
    engine.admit()
    seen = []

    def fused_stand_in(transaction, layer_idx, q, k, v, *, rotary_dim=None, base=10_000.0, q_out=None):
        seen.append(layer_idx)
        view = engine.cache.transaction_view(transaction)
        latest = engine.cache.write_token_layer(transaction, layer_idx,
                                                apply_rope(k, view.positions, rotary_dim=rotary_dim, base=base), v)
        return apply_rope(q, view.positions, rotary_dim=rotary_dim, base=base), latest

    monkeypatch.setattr(engine.cache, "write_token_layer_fused_cuda", fused_stand_in)
    tx = engine.begin_step([1])
    for layer in range(2):
        engine.step_layer(tx, layer, *inputs(1, 625 + layer))
    result = engine.commit_step(tx)
    assert seen == [0, 1] and result.status == DecodeEngine.STEP_OK and result.seq_lens.tolist() == [1]
    assert engine.validate_invariants()


def test_unfused_hip_backend_rejected_for_transactions():
    engine = DecodeEngine(make_cache(num_layers=2), append_backend="cuda")
    engine.add_request(1)
    engine.admit()
    with pytest.raises(RuntimeError, match="append_backend='torch' or 'fused_cuda'"):
        engine.begin_step([1])
    assert engine.cache.num_used_blocks == 0
    assert engine.validate_invariants()


def test_single_layer_step_wrapper_and_backpressure():
    engine = DecodeEngine(make_cache(num_layers=1, block_size=1, max_blocks=1))
    engine.add_request(1)
    engine.add_request(2)
    engine.admit()
    q, k, v = inputs(1, 619)
    result = engine.step(q, k, v, [1])
    assert result.status == DecodeEngine.STEP_OK and result.seq_lens.tolist() == [1]
    assert engine.cache.metrics()["transaction_commit_count"] == 1
    version = engine.cache.state_version
    blocked = engine.step(q, k, v, [2])
    assert blocked.status == DecodeEngine.STEP_BACKPRESSURE
    assert blocked.reason == "insufficient_physical_blocks"
    assert (blocked.needed_new_blocks, blocked.free_blocks) == (1, 0) and blocked.output is None
    assert engine.cache.state_version == version
    m = engine.metrics()
    assert (m["completed_step_count"], m["backpressure_count"]) == (1, 1)
    engine.finish_request(1)
    assert engine.step(q, k, v, [2]).status == DecodeEngine.STEP_OK
    assert engine.validate_invariants()


def test_single_layer_step_matches_oracle_over_many_tokens():
    engine = DecodeEngine(make_cache(num_layers=1, block_size=4, max_blocks=16, head_dim=8, num_kv_heads=2))
    for rid in ("a", "b", "c"):
        engine.add_request(rid)
    engine.admit()
    for step in range(9):
        q, k, v = inputs(3, 700 + step, hq=4, hkv=2, d=8)
        res = engine.step(q, k, v)
        expected = oracle_layer(engine.cache, 0, q, res.positions, res.block_tables, res.seq_lens)
        np.testing.assert_allclose(res.output.numpy(), expected, atol=1e-5, rtol=1e-5)
    assert engine.cache.seq_lens_tensor(["a", "b", "c"]).tolist() == [9, 9, 9]
    engine.cancel_request("b")
    assert engine.active_request_ids() == ("a", "c")
    assert engine.validate_invariants()


def test_request_lifecycle_errors():
    engine = DecodeEngine(make_cache(num_layers=1))
    assert engine.add_request("x").status == DecodeEngine.WAITING
    with pytest.raises(RuntimeError, match="already exists"):
        engine.add_request("x")
    with pytest.raises(RuntimeError, match="expected active"):
        engine.finish_request("x")
    with pytest.raises(KeyError, match="unknown request_id"):
        engine.request_state("nope")
    with pytest.raises(ValueError, match="at least one active request"):
        engine.step(*inputs(1, 1))
    assert engine.request_state("x") == {"request_id": "x", "status": "waiting"}
    engine.admit()
    assert engine.request_state("x")["cache"]["status"] == "active"
    with pytest.raises(ValueError, match="append_backend"):
        DecodeEngine(make_cache(), append_backend="bogus")
    with pytest.raises(ValueError, match="decode_backend"):
        DecodeEngine(make_cache(), decode_backend="bogus")
    with pytest.raises(TypeError, match="PagedKVCache"):
        DecodeEngine(object())


def test_shared_prefix_through_engine():
    cache = PagedKVCache(num_layers=2, num_kv_heads=1, head_dim=4, block_size=2, max_blocks=6, dtype=torch.float32,
                         device="cpu", prefix_cache_capacity_blocks=2)
    engine = DecodeEngine(cache)
    g = torch.Generator().manual_seed(5)
    pk = torch.randn(2, 2, 1, 2, 4, generator=g)
    prefix_ids = engine.register_prefix("sys", pk, pk + 1)["block_ids"]
    for rid in ("a", "b"):
        engine.add_request(rid)
    engine.admit(prefix_id="sys")
    assert cache.metrics()["active_prefix_references"] == 2
    tx = engine.begin_step()
    assert tx.positions.tolist() == [4, 4]
    for layer in range(2):
        q, k, v = inputs(2, 900 + layer)
        res = engine.step_layer(tx, layer, q, k, v)
        expected = oracle_layer(cache, layer, q, tx.positions, tx.block_tables, tx.effective_seq_lens)
        np.testing.assert_allclose(res.output.numpy(), expected, atol=1e-5, rtol=1e-5)
    engine.commit_step(tx)
    assert cache.metrics()["shared_prefix_blocks"] == 2 and cache.metrics()["saved_prefix_blocks"] == 2
    engine.finish_request("a")
    engine.finish_request("b")
    assert engine.evict_prefix("sys") == prefix_ids
    assert cache.num_free_blocks == cache.max_blocks
    assert engine.validate_invariants()
