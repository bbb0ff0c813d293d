"""PagedKVCache on the CPU: allocator, multi-layer transactions, shared prefixes.

Expected values are the literal known answers of the reference's own tests
(tests/golden/reference_kats.json cites each source line); the scenarios are
restated here, not copied.
"""

import json
import pathlib
from dataclasses import replace

import pytest
import torch

import flashdec_amd
from flashdec_amd.cache import KVTokenTransactionView, PagedKVCache

KATS = json.loads((pathlib.Path(__file__).parent / "golden" / "reference_kats.json").read_text())


def make_cache(num_layers=1, block_size=2, max_blocks=4, head_dim=2, prefix_capacity=0):
    return PagedKVCache(num_layers=num_layers, num_kv_heads=1, head_dim=head_dim, block_size=block_size,
                        max_blocks=max_blocks, dtype=torch.float32, device="cpu",
                        prefix_cache_capacity_blocks=prefix_capacity)


def tok(n, value, head_dim=2):
    return torch.full((n, 1, head_dim), float(value))


def write_all_layers(cache, tx, base=0.0):
    for layer in range(cache.num_layers):
        cache.write_token_layer(tx, layer, tok(len(tx.request_ids), base + layer, cache.head_dim),
                                tok(len(tx.request_ids), base + 100 + layer, cache.head_dim))


# ---------------------------------------------------------------- allocator
def test_noncontiguous_block_ownership_kat():
    kat = KATS["cache_noncontiguous_blocks"]
    cache = make_cache(block_size=kat["block_size"], max_blocks=kat["max_blocks"], head_dim=kat["head_dim"])
    for rid, value in kat["appends"]:
        cache.append(0, [rid], torch.tensor([[value]]), torch.tensor([[value]]) * 10)
    for rid, ids in kat["block_ids"].items():
        assert cache.request_block_ids(int(rid)) == tuple(ids)
    tables = cache.block_tables([10, 20])
    assert tables.dtype == torch.int32
    assert tables.tolist() == kat["block_tables"]
    assert cache.seq_lens_tensor([10, 20]).tolist() == kat["seq_lens"]
    assert cache.num_used_blocks == kat["used_blocks"] and cache.num_free_blocks == kat["free_blocks"]
    # token 2 of request 10 sits in physical block 2 offset 0; token 1 in block 0 offset 1
    assert cache.k_cache[0, 2, 0, 0].tolist() == [7.0, 8.0]
    assert cache.k_cache[0, 0, 0, 1].tolist() == [5.0, 6.0]
    k_dense, v_dense, lens = cache.to_dense(0, [10, 20])
    assert k_dense[0, :3, 0].tolist() == [[1.0, 2.0], [5.0, 6.0], [7.0, 8.0]]
    assert torch.equal(v_dense, k_dense * 10)
    assert lens.tolist() == [3, 1]
    assert cache.validate_invariants()


def test_finish_releases_blocks_for_reuse_kat():
    kat = KATS["cache_finish_reuse"]
    cache = make_cache(block_size=2, max_blocks=4)
    cache.append(0, [1, 2], tok(2, 1), tok(2, 1))
    released = cache.finish_request(1)
    assert released == (0,)
    # released blocks return to the front of the free list and are reused first
    cache.append(0, [3], tok(1, 2), tok(1, 2))
    assert cache.request_block_ids(3) == (0,)
    cache.cancel_request(2)
    m = cache.metrics()
    for key in ("allocation_count", "fresh_allocation_count", "free_count", "reuse_count"):
        assert m[key] == kat[key], key
    assert cache.request_state(1)["status"] == "finished"
    assert cache.request_state(2)["status"] == "cancelled"
    with pytest.raises(RuntimeError, match="finished and cannot accept append"):
        cache.append(0, [1], tok(1, 0), tok(1, 0))
    with pytest.raises(RuntimeError, match="cannot be reactivated"):
        cache.add_request(1)
    assert cache.validate_invariants()


def test_metrics_exact_kat():
    kat = KATS["cache_metrics_exact"]["metrics"]
    cache = make_cache(block_size=4, max_blocks=4)
    cache.append(0, [1, 2], tok(2, 1), tok(2, 1))
    cache.append(0, [1], tok(1, 2), tok(1, 2))
    assert cache.metrics() == kat
    assert len(kat) == 45


def test_capacity_failure_does_not_mutate():
    cache = make_cache(block_size=1, max_blocks=2)
    cache.append(0, [1, 2], tok(2, 1), tok(2, 1))
    version = cache.state_version
    with pytest.raises(RuntimeError, match="out of physical blocks"):
        cache.append(0, [3], tok(1, 1), tok(1, 1))
    assert cache.state_version == version
    assert cache.metrics()["capacity_failure_count"] == 1
    with pytest.raises(KeyError):
        cache.request_state(3)
    assert cache.validate_invariants()


def test_churn_reuses_single_block_kat():
    kat = KATS["cache_churn"]
    cache = make_cache(block_size=4, max_blocks=1)
    for i in range(20):
        cache.append(0, [i], tok(1, i), tok(1, i))
        if i % 2:
            cache.cancel_request(i)
        else:
            cache.finish_request(i)
    m = cache.metrics()
    for key, expected in kat.items():
        if key != "source":
            assert m[key] == expected, key
    assert cache.validate_invariants()


def test_input_validation_messages():
    cache = make_cache()
    with pytest.raises(ValueError, match="request_ids must be non-empty"):
        cache.append(0, [], tok(0, 0), tok(0, 0))
    with pytest.raises(ValueError, match="unique"):
        cache.append(0, [1, 1], tok(2, 0), tok(2, 0))
    with pytest.raises(ValueError, match="shapes must match"):
        cache.append(0, [1], torch.zeros(1, 1, 3), torch.zeros(1, 1, 3))
    with pytest.raises(ValueError, match="cache dtype"):
        cache.append(0, [1], tok(1, 0).half(), tok(1, 0).half())
    with pytest.raises(ValueError, match="layer_idx"):
        cache.append(1, [1], tok(1, 0), tok(1, 0))
    with pytest.raises(ValueError, match="hashable"):
        cache.add_request([1])
    with pytest.raises(ValueError, match="max_blocks must be positive"):
        PagedKVCache(1, 1, 2, 2, 0, dtype=torch.float32, device="cpu")
    with pytest.raises(ValueError, match="floating point"):
        PagedKVCache(1, 1, 2, 2, 2, dtype=torch.int32, device="cpu")
    assert cache.metrics()["used_blocks"] == 0


def test_hip_append_paths_refuse_cpu_cache():
    cache = make_cache()
    with pytest.raises(ValueError, match="CUDA-resident"):
        cache.append_cuda(0, [1], tok(1, 0), tok(1, 0))
    with pytest.raises(ValueError, match="CUDA-resident"):
        cache.append_fused_cuda(0, [1], torch.zeros(1, 2, 2), tok(1, 0), tok(1, 0), torch.zeros(1, dtype=torch.long))
    assert cache.metrics()["used_blocks"] == 0


# ------------------------------------------------------ token transactions
@pytest.mark.parametrize("num_layers", [2, 4])
def test_transaction_commits_once_and_reuses_locations(num_layers):
    cache = make_cache(num_layers=num_layers)
    cache.add_request(10).add_request(20)
    tx = cache.begin_token([10, 20])
    assert isinstance(tx, KVTokenTransactionView)
    assert flashdec_amd.KVTokenTransactionView is KVTokenTransactionView
    assert tx.state == "open" and tx.next_layer_idx == 0
    assert tx.positions.tolist() == [0, 0] and tx.block_offsets.tolist() == [0, 0]
    assert tx.effective_seq_lens.tolist() == [1, 1]
    assert tx.positions.dtype == tx.physical_block_ids.dtype == tx.block_offsets.dtype == torch.int64
    assert tx.effective_seq_lens.dtype == tx.block_tables.dtype == torch.int32
    ids = tx.physical_block_ids.tolist()
    for layer in range(num_layers):
        latest = cache.write_token_layer(tx, layer, tok(2, layer + 1), tok(2, layer + 101))
        assert latest.next_layer_idx == layer + 1
        assert latest.physical_block_ids.tolist() == ids
        for row, blk in enumerate(ids):
            assert cache.k_cache[layer, blk, 0, 0].tolist() == [layer + 1.0] * 2
            assert cache.v_cache[layer, blk, 0, 0].tolist() == [layer + 101.0] * 2
        assert cache.seq_lens_tensor([10, 20]).tolist() == [0, 0]  # invisible until commit
    committed = cache.commit_token(tx)
    assert committed.state == "committed"
    assert cache.seq_lens_tensor([10, 20]).tolist() == [1, 1]
    m = cache.metrics()
    assert (m["transaction_commit_count"], m["transaction_layer_write_count"], m["open_transaction_count"]) == (
        1, num_layers, 0)
    for layer in range(num_layers):
        k_dense, v_dense, lens = cache.to_dense(layer, [10, 20])
        assert torch.equal(k_dense[:, 0], tok(2, layer + 1))
        assert torch.equal(v_dense[:, 0], tok(2, layer + 101))
    assert cache.validate_invariants()


def test_transaction_views_are_detached_from_allocator_metadata():
    cache = make_cache(num_layers=2)
    cache.add_request(1)
    tx = cache.begin_token([1])
    tx.physical_block_ids.fill_(3)
    tx.block_tables.fill_(3)
    meta = cache.transaction_device_metadata(tx)
    assert meta.block_ids.tolist() == [0] and meta.block_tables.tolist() == [[0]]
    write_all_layers(cache, tx)
    cache.commit_token(tx)
    assert cache.request_block_ids(1) == (0,)
    assert cache.validate_invariants()


def test_transaction_mixed_tail_and_boundary_reserves_only_needed_block():
    cache = make_cache(num_layers=2, max_blocks=3)
    cache.add_request("tail")
    first = cache.begin_token(["tail"])
    write_all_layers(cache, first)
    cache.commit_token(first)
    tail_block = cache.request_block_ids("tail")[0]
    cache.add_request("boundary")
    tx = cache.begin_token(["tail", "boundary"])
    assert tx.positions.tolist() == [1, 0] and tx.block_offsets.tolist() == [1, 0]
    assert tx.physical_block_ids[0].item() == tail_block
    assert tx.block_tables.tolist() == [[tail_block], [1]]
    m = cache.metrics()
    assert m["reserved_transaction_blocks"] == 1 and m["pending_request_count"] == 2
    assert cache.validate_invariants()
    cache.abort_token(tx)
    assert cache.request_state("tail")["seq_len"] == 1 and cache.request_state("boundary")["seq_len"] == 0
    assert cache.request_block_ids("tail") == (tail_block,) and cache.request_block_ids("boundary") == ()
    assert cache.validate_invariants()


def test_transaction_capacity_failure_has_no_mutation():
    cache = make_cache(num_layers=2, block_size=1, max_blocks=1)
    cache.add_request(1).add_request(2)
    version, s1, s2 = cache.state_version, cache.request_state(1), cache.request_state(2)
    with pytest.raises(RuntimeError, match="out of physical blocks"):
        cache.begin_token([1, 2])
    assert cache.state_version == version
    assert (cache.request_state(1), cache.request_state(2)) == (s1, s2)
    assert cache.num_used_blocks == 0
    assert cache.metrics()["open_transaction_count"] == 0
    assert cache.metrics()["transaction_failure_count"] == 1
    assert cache.validate_invariants()


def test_location_proof_failure_rolls_back_reservation(monkeypatch):
    cache = make_cache(num_layers=2, block_size=1, max_blocks=2)
    cache.add_request("r")
    version = cache.state_version
    original = cache._validate_reserved_transaction_locations

    def broken(*_a, **_k):
        raise RuntimeError("planted location proof failure")

    monkeypatch.setattr(cache, "_validate_reserved_transaction_locations", broken)
    with pytest.raises(RuntimeError, match="planted location proof"):
        cache.begin_token(["r"])
    assert cache.state_version == version
    assert cache.request_block_ids("r") == () and cache.num_free_blocks == 2
    m = cache.metrics()
    assert (m["open_transaction_count"], m["transaction_begin_count"], m["transaction_failure_count"]) == (0, 0, 1)
    assert cache.validate_invariants()
    monkeypatch.setattr(cache, "_validate_reserved_transaction_locations", original)
    tx = cache.begin_token(["r"])
    assert tx.physical_block_ids.tolist() == [0]
    cache.abort_token(tx)
    assert cache.validate_invariants()


def test_location_proof_rejects_inconsistent_rows():
    cache = make_cache(num_layers=1, block_size=2, max_blocks=2)
    cache.add_request(1)
    state = cache._seqs[1]
    state.pages.append(0)
    with pytest.raises(RuntimeError, match="offset does not match"):
        cache._validate_reserved_transaction_locations([1], [state], [0], [(0, 1)])
    with pytest.raises(RuntimeError, match="out of range"):
        cache._validate_reserved_transaction_locations([1], [state], [0], [(5, 0)])
    with pytest.raises(RuntimeError, match="does not match request"):
        cache._validate_reserved_transaction_locations([1], [state], [0], [(1, 0)])
    with pytest.raises(RuntimeError, match="not allocated"):
        cache._validate_reserved_transaction_locations([1], [state], [2], [(0, 0)])


def test_abort_hides_partial_layer_and_rolls_back_boundary_block():
    cache = make_cache(num_layers=2, block_size=1, max_blocks=1)
    cache.add_request("r")
    tx = cache.begin_token(["r"])
    reserved = tx.physical_block_ids.item()
    cache.write_token_layer(tx, 0, tok(1, 7), tok(1, 107))
    aborted = cache.abort_token(tx)
    assert aborted.state == "aborted"
    assert cache.request_state("r")["seq_len"] == 0 and cache.request_block_ids("r") == ()
    assert cache.num_used_blocks == 0
    k_dense, v_dense, lens = cache.to_dense(0, ["r"])
    assert lens.tolist() == [0] and not k_dense.any() and not v_dense.any()
    assert cache.metrics()["transaction_rollback_block_count"] == 1
    again = cache.begin_token(["r"])
    assert again.physical_block_ids.item() == reserved
    write_all_layers(cache, again, base=8)
    cache.commit_token(again)
    assert cache.request_state("r")["seq_len"] == 1
    assert cache.metrics()["reuse_count"] == 1
    assert cache.validate_invariants()


def test_transaction_state_machine_rejections():
    cache = make_cache(num_layers=2)
    cache.add_request(1)
    tx = cache.begin_token([1])
    t = tok(1, 1)
    with pytest.raises(RuntimeError, match="requires layer 0"):
        cache.write_token_layer(tx, 1, t, t)
    with pytest.raises(RuntimeError, match="before all layers"):
        cache.commit_token(tx)
    for call in (lambda: cache.begin_token([1]), lambda: cache.finish_request(1), lambda: cache.cancel_request(1),
                 lambda: cache.add_request(2)):
        with pytest.raises(RuntimeError, match="open token transaction"):
            call()
    cache.write_token_layer(tx, 0, t, t)
    with pytest.raises(RuntimeError, match="requires layer 1"):
        cache.write_token_layer(tx, 0, t, t)
    cache.write_token_layer(tx, 1, t, t)
    committed = cache.commit_token(tx)
    for call in (cache.commit_token, cache.abort_token, cache.transaction_view):
        with pytest.raises(RuntimeError, match="already committed"):
            call(committed)
    with pytest.raises(TypeError, match="KVTokenTransactionView"):
        cache.commit_token(object())
    assert cache.validate_invariants()


def test_terminal_history_is_bounded_and_tensor_free():
    kat = KATS["terminal_history"]
    cache = make_cache(num_layers=1, block_size=16, max_blocks=1)
    cache._journal.limit = kat["limit"]
    cache.add_request("r")
    handles = []
    for i in range(kat["transactions"]):
        tx = cache.begin_token(["r"])
        handles.append(tx)
        if i % 3 == 2:
            cache.abort_token(tx)
        else:
            write_all_layers(cache, tx)
            cache.commit_token(tx)
        m = cache.metrics()
        assert m["retained_transaction_state_count"] == 0
        assert m["terminal_transaction_history_count"] <= kat["limit"]
        assert cache.validate_invariants()
    assert list(cache._journal.history) == kat["retained_ids"]
    assert not any(isinstance(getattr(t, f), torch.Tensor) for t in cache._journal.history.values() for f in t.__slots__)
    with pytest.raises(RuntimeError, match="unknown token transaction"):
        cache.abort_token(handles[0])
    with pytest.raises(RuntimeError, match="already aborted"):
        cache.abort_token(handles[-1])
    with pytest.raises(RuntimeError, match="already committed"):
        cache.commit_token(handles[-2])
    with pytest.raises(RuntimeError, match="stale or invalid"):
        cache.commit_token(replace(handles[-2], request_ids=("forged",)))


@pytest.mark.parametrize("op", ["commit", "abort"])
def test_terminal_view_failure_leaves_transaction_open(monkeypatch, op):
    cache = make_cache(num_layers=1, block_size=1, max_blocks=1)
    cache.add_request("r")
    tx = cache.begin_token(["r"])
    if op == "commit":
        write_all_layers(cache, tx)
    original = cache._snapshot

    def broken(_state):
        raise RuntimeError("planted view failure")

    monkeypatch.setattr(cache, "_snapshot", broken)
    call = getattr(cache, f"{op}_token")
    with pytest.raises(RuntimeError, match="planted view failure"):
        call(tx)
    assert cache.has_open_transaction
    assert cache.request_state("r")["seq_len"] == 0 and cache.request_block_ids("r") == (0,)
    m = cache.metrics()
    assert (m["retained_transaction_state_count"], m["terminal_transaction_history_count"]) == (1, 0)
    assert cache.validate_invariants()
    monkeypatch.setattr(cache, "_snapshot", original)
    assert call(tx).state == {"commit": "committed", "abort": "aborted"}[op]
    m = cache.metrics()
    assert (m["retained_transaction_state_count"], m["terminal_transaction_history_count"]) == (0, 1)
    assert cache.validate_invariants()


def test_invalid_layer_values_rejected_before_write():
    cache = make_cache(num_layers=2)
    cache.add_request(1)
    tx = cache.begin_token([1])
    bad = torch.ones(1, 1, 3)
    with pytest.raises(ValueError, match="shapes must match"):
        cache.write_token_layer(tx, 0, bad, bad)
    assert cache.transaction_view(tx).next_layer_idx == 0
    assert cache.metrics()["transaction_failure_count"] == 1
    cache.abort_token(tx)
    assert cache.validate_invariants()


def test_legacy_append_rejected_during_transaction_and_for_multi_layer():
    cache = make_cache(num_layers=1)
    cache.add_request(1)
    tx = cache.begin_token([1])
    with pytest.raises(RuntimeError, match="open token transaction"):
        cache.append(0, [1], tok(1, 1), tok(1, 1))
    cache.abort_token(tx)
    multi = make_cache(num_layers=2)
    with pytest.raises(RuntimeError, match="token transaction API"):
        multi.append(0, [1], tok(1, 1), tok(1, 1))


def test_invariant_checker_detects_planted_corruption():
    cache = make_cache(block_size=2, max_blocks=4)
    cache.append(0, [1, 2], tok(2, 1), tok(2, 1))
    assert cache.validate_invariants()
    cache._pool.free.append(cache.request_block_ids(1)[0])
    with pytest.raises(RuntimeError):
        cache.validate_invariants()
    cache._pool.free.pop()
    cache._seqs[2].length = 5
    with pytest.raises(RuntimeError, match="block count does not match"):
        cache.validate_invariants()


# ------------------------------------------------------------ shared prefix
def prefix_blocks(cache, n, start=0):
    shape = (cache.num_layers, n, cache.num_kv_heads, cache.block_size, cache.head_dim)
    k = torch.arange(start, start + torch.Size(shape).numel(), dtype=cache.dtype).reshape(shape)
    return k, k + 1000


def dense_of(blocks, layer):
    return blocks[layer].permute(0, 2, 1, 3).reshape(-1, blocks.shape[2], blocks.shape[4])


def test_shared_prefix_reuse_and_private_tail():
    kat = KATS["shared_prefix_metrics"]
    cache = make_cache(num_layers=2, block_size=2, max_blocks=5, head_dim=3, prefix_capacity=4)
    pk, pv = prefix_blocks(cache, 2)
    ids = cache.register_prefix("system", pk, pv)["block_ids"]
    cache.add_request("a").add_request("b")
    assert cache.attach_prefix("a", "system") == ids and cache.attach_prefix("b", "system") == ids
    assert cache.prefix_state("system")["active_refcount"] == 2
    for layer in range(2):
        k_dense, v_dense, lens = cache.to_dense(layer, ["a", "b"])
        assert torch.equal(k_dense[0, :4], dense_of(pk, layer)) and torch.equal(k_dense[1, :4], dense_of(pk, layer))
        assert torch.equal(v_dense[1, :4], dense_of(pv, layer))
        assert lens.tolist() == [4, 4]
    stored = cache.k_cache[:, list(ids)].clone()
    tx = cache.begin_token(["a"])
    assert tx.block_tables.tolist() == [list(ids) + [2]]
    write_all_layers(cache, tx, base=100)
    cache.commit_token(tx)
    assert torch.equal(cache.k_cache[:, list(ids)], stored)  # shared blocks are immutable
    a_blocks = cache.request_block_ids("a")
    assert a_blocks[:2] == ids and len(a_blocks) == 3 and cache.request_state("a")["seq_len"] == 5
    m = cache.metrics()
    for key in ("used_blocks", "active_tokens", "physical_data_tokens", "shared_prefix_blocks",
                "saved_prefix_blocks", "active_prefix_references"):
        assert m[key] == kat[key], key
    assert cache.finish_request("a") == (a_blocks[-1],)
    assert cache.prefix_state("system")["active_refcount"] == 1
    assert cache.finish_request("b") == ()
    assert cache.num_used_blocks == 2
    assert cache.evict_prefix("system") == ids
    assert cache.num_free_blocks == cache.max_blocks
    assert cache.validate_invariants()


def test_shared_prefix_lru_evicts_only_inactive():
    cache = make_cache(num_layers=1, block_size=2, max_blocks=3, head_dim=3, prefix_capacity=2)
    cache.register_prefix("old", *prefix_blocks(cache, 1, 0))
    cache.register_prefix("protected", *prefix_blocks(cache, 1, 100))
    cache.add_request("owner")
    protected = cache.attach_prefix("owner", "protected")
    cache.register_prefix("new", *prefix_blocks(cache, 1, 200))
    with pytest.raises(KeyError, match="unknown prefix_id"):
        cache.prefix_state("old")
    assert cache.prefix_state("protected")["block_ids"] == protected
    assert cache.metrics()["prefix_eviction_count"] == 1
    cache.add_request("lookup")
    with pytest.raises(KeyError, match="unknown prefix_id"):
        cache.attach_prefix("lookup", "old")
    cache.attach_prefix("lookup", "new")
    with pytest.raises(RuntimeError, match="active request references"):
        cache.evict_prefix("protected")
    m = cache.metrics()
    assert (m["prefix_hit_count"], m["prefix_miss_count"]) == (2, 1)
    assert m["prefix_hit_ratio"] == pytest.approx(2 / 3)
    assert cache.validate_invariants()


def test_shared_prefix_capacity_failure_is_atomic():
    cache = make_cache(num_layers=1, block_size=2, max_blocks=2, head_dim=3, prefix_capacity=2)
    cache.register_prefix("active", *prefix_blocks(cache, 2))
    cache.add_request("owner")
    cache.attach_prefix("owner", "active")
    before = (cache.request_state("owner"), cache.prefix_state("active"), cache.state_version)
    with pytest.raises(RuntimeError, match="insufficient evictable prefix capacity"):
        cache.register_prefix("blocked", *prefix_blocks(cache, 1, 100))
    assert (cache.request_state("owner"), cache.prefix_state("active"), cache.state_version) == before
    assert cache.num_free_blocks == 0
    m = cache.metrics()
    assert (m["capacity_failure_count"], m["prefix_capacity_failure_count"]) == (1, 1)
    assert cache.validate_invariants()


def test_shared_prefix_abort_returns_only_private_boundary_block():
    cache = make_cache(num_layers=2, block_size=2, max_blocks=3, head_dim=3, prefix_capacity=1)
    ids = cache.register_prefix("p", *prefix_blocks(cache, 1))["block_ids"]
    cache.add_request("r")
    cache.attach_prefix("r", "p")
    tx = cache.begin_token(["r"])
    cache.write_token_layer(tx, 0, torch.ones(1, 1, 3), torch.ones(1, 1, 3))
    cache.abort_token(tx)
    assert cache.request_block_ids("r") == ids
    assert cache.request_state("r")["seq_len"] == cache.block_size
    assert cache.prefix_state("p")["active_refcount"] == 1 and cache.num_used_blocks == 1
    assert cache.validate_invariants()


def test_shared_prefix_attach_rejections():
    cache = make_cache(num_layers=1, block_size=2, max_blocks=4, head_dim=3, prefix_capacity=2)
    cache.register_prefix("p", *prefix_blocks(cache, 1))
    cache.append(0, ["busy"], torch.ones(1, 1, 3), torch.ones(1, 1, 3))
    with pytest.raises(RuntimeError, match="empty active request"):
        cache.attach_prefix("busy", "p")
    with pytest.raises(ValueError, match="must not be None"):
        cache.attach_prefix("busy", None)
    with pytest.raises(RuntimeError, match="already registered"):
        cache.register_prefix("p", *prefix_blocks(cache, 1))
    with pytest.raises(ValueError, match="shape does not match"):
        cache.register_prefix("q", torch.zeros(1, 1, 1, 3, 3), torch.zeros(1, 1, 1, 3, 3))
    assert cache.validate_invariants()


# -------------------------------------------------------- bulk seeding, arena
def test_seed_context_equals_token_by_token_commits():
    a = make_cache(num_layers=2, block_size=4, max_blocks=32)
    b = make_cache(num_layers=2, block_size=4, max_blocks=32)
    for c in (a, b):
        for rid in ("x", "y", "z"):
            c.add_request(rid)
    g = torch.Generator().manual_seed(3)
    # y starts mid-block so the two paths interleave allocations the same way
    tx = a.begin_token(["y"])
    write_all_layers(a, tx)
    a.commit_token(tx)
    tx = b.begin_token(["y"])
    write_all_layers(b, tx)
    b.commit_token(tx)
    k = torch.randn(2, 3, 9, 1, 2, generator=g)
    v = torch.randn(2, 3, 9, 1, 2, generator=g)
    for t in range(9):
        tx = a.begin_token(["x", "y", "z"])
        for layer in range(2):
            a.write_token_layer(tx, layer, k[layer, :, t], v[layer, :, t])
        a.commit_token(tx)
    lens = b.seed_context(["x", "y", "z"], 9, k, v)
    assert lens.tolist() == [9, 10, 9]
    for rid in ("x", "y", "z"):
        assert a.request_block_ids(rid) == b.request_block_ids(rid)
    assert list(a._pool.free) == list(b._pool.free)
    assert torch.equal(a.k_cache, b.k_cache) and torch.equal(a.v_cache, b.v_cache)
    for key in ("used_blocks", "allocation_count", "fresh_allocation_count", "active_tokens"):
        assert a.metrics()[key] == b.metrics()[key]
    assert b.validate_invariants()


def test_seed_context_capacity_failure_is_atomic():
    cache = make_cache(block_size=4, max_blocks=2)
    cache.add_request(1).add_request(2)
    with pytest.raises(RuntimeError, match="out of physical blocks"):
        cache.seed_context([1, 2], 5)
    assert cache.num_used_blocks == 0 and cache.seq_lens_tensor([1, 2]).tolist() == [0, 0]
    with pytest.raises(ValueError, match="together"):
        cache.seed_context([1], 1, k=torch.zeros(1, 1, 1, 1, 2))


def test_graph_metadata_arena_layout_and_limits():
    cache = make_cache(num_layers=1, block_size=2, max_blocks=16)
    arena = cache.enable_graph_metadata(max_batch=4, max_blocks_per_seq=3)
    for rid in ("a", "b"):
        cache.add_request(rid)
    cache.seed_context(["a"], 3)
    tx = cache.begin_token(["a", "b"])
    meta = cache.transaction_device_metadata(tx)
    view2 = cache.graph_metadata(2)
    assert meta.buf.data_ptr() == arena.buf.data_ptr()
    assert meta.block_ids.data_ptr() == view2.block_ids.data_ptr() == arena.block_ids.data_ptr()
    assert meta.block_tables.data_ptr() == arena.block_tables.data_ptr()
    assert meta.positions.tolist() == [3, 0] and meta.offsets.tolist() == [1, 0]
    assert meta.eff_lens.tolist() == [4, 1]
    assert meta.block_tables.tolist() == [[0, 1, -1], [2, -1, -1]]
    assert tx.block_tables.tolist() == [[0, 1, -1], [2, -1, -1]]
    write_all_layers(cache, tx)
    cache.commit_token(tx)
    cache.seed_context(["a"], 2)  # a now needs 3 blocks; its next token needs a 4th
    version = cache.state_version
    with pytest.raises(RuntimeError, match="graph metadata arena"):
        cache.begin_token(["a", "b"])
    assert cache.state_version == version and not cache.has_open_transaction
    assert cache.request_block_ids("a") == (0, 1, 3) and cache.validate_invariants()
