"""Seeded random engine lifecycles checked against a host shadow of every request's K/V history.

The other engine tests compare each layer's output with the oracle run over
the cache's own tables, so a table that pointed at the wrong block (a block
freed by one request and reused by another, a prefix block released while
still attached) would agree with itself.  Here the host keeps, per request
and layer, the K/V rows it has committed -- the registered prefix's tokens,
seeded context, and every appended token (K after the oracle's RoPE, V as
given) -- and the expected attention comes from those histories alone.

Each lifecycle mixes, at random (seeded): admissions with and without a
shared prefix (the reference's attach at admission, flashdec/engine.py:
352-371), seeded context, finish and cancel (engine.py:373-401), steps that
fail on a malformed layer input and roll the whole token back (the
reference's LayerFailure, flashdec/integrated_workload.py:49-58), steps the
caller aborts after every layer ran, backpressure when the pool runs dry
(engine.py:604-612), and the shared-prefix launch for attached rows.  After
each committed step the cache's dense K/V of every active request must equal
the shadow bit for bit; at the end every block is back in the free list.

The graph lifecycle keeps a batch of four rows and replaces finished ones, so
one captured step graph is replayed over changing requests, lengths and
tables.
"""

import numpy as np
import pytest
import torch

from flashdec_amd.cache import PagedKVCache
from flashdec_amd.engine import DecodeEngine
from oracle import attention as oa
from tests.helpers import assert_close_to_oracle

L, HQ, HKV, D, BS = 3, 16, 2, 128, 8
BASE = 1e4


def _bits(x):
    t = x if isinstance(x, torch.Tensor) else torch.from_numpy(np.ascontiguousarray(x, np.float32))
    return t.detach().cpu().to(torch.bfloat16).contiguous().view(torch.int16).numpy()


class Shadow:
    """Per request and layer: the committed K rows and V rows ([Hkv, D] float32, bf16-exact)."""

    def __init__(self):
        self.k, self.v = {}, {}

    def start(self, rid, k_rows=None, v_rows=None):
        self.k[rid] = [list(k_rows[layer]) if k_rows is not None else [] for layer in range(L)]
        self.v[rid] = [list(v_rows[layer]) if v_rows is not None else [] for layer in range(L)]

    def drop(self, rid):
        del self.k[rid], self.v[rid]

    def length(self, rid):
        return len(self.k[rid][0])

    def expected(self, ids, layer, q_rot, k_new, v_new):
        """Oracle attention of rows ``ids`` over history + the step's new token (compact paged copy)."""
        blocks_k, blocks_v, table_rows, lens = [], [], [], []
        for row, rid in enumerate(ids):
            ks = np.stack(self.k[rid][layer] + [k_new[row]])
            vs = np.stack(self.v[rid][layer] + [v_new[row]])
            n = ks.shape[0]
            nb = -(-n // BS)
            pad = nb * BS - n
            ks = np.concatenate([ks, np.zeros((pad, HKV, D), np.float32)]).reshape(nb, BS, HKV, D)
            vs = np.concatenate([vs, np.zeros((pad, HKV, D), np.float32)]).reshape(nb, BS, HKV, D)
            table_rows.append(list(range(len(blocks_k), len(blocks_k) + nb)))
            blocks_k.extend(ks.transpose(0, 2, 1, 3))
            blocks_v.extend(vs.transpose(0, 2, 1, 3))
            lens.append(n)
        width = max(len(r) for r in table_rows)
        table = np.full((len(ids), width), -1, dtype=np.int32)
        for row, r in enumerate(table_rows):
            table[row, :len(r)] = r
        return oa.paged_decode_attention(q_rot, np.stack(blocks_k), np.stack(blocks_v), table, np.asarray(lens))

    def commit(self, ids, new_rows):
        for layer, (k_new, v_new) in new_rows.items():
            for row, rid in enumerate(ids):
                self.k[rid][layer].append(k_new[row])
                self.v[rid][layer].append(v_new[row])

    def check_cache(self, cache, ids):
        for layer in range(L):
            kd, vd, lens = cache.to_dense(layer, list(ids))
            assert lens.tolist() == [self.length(rid) for rid in ids]
            for row, rid in enumerate(ids):
                n = self.length(rid)
                if n == 0:
                    continue
                assert np.array_equal(_bits(kd[row, :n]), _bits(np.stack(self.k[rid][layer]))), (rid, layer)
                assert np.array_equal(_bits(vd[row, :n]), _bits(np.stack(self.v[rid][layer]))), (rid, layer)


def _rand(g, *shape):
    return torch.randn(*shape, generator=g).to(torch.bfloat16)


def _prefix_tokens(kb):
    """[L, n, Hkv, bs, D] prefix blocks -> per layer, the token rows [Hkv, D] in order."""
    a = kb.float().numpy()
    return [[a[layer, j, :, t] for j in range(a.shape[1]) for t in range(BS)] for layer in range(L)]


def _admit(engine, shadow, rng, g, ids, prefixes, device):
    choice = int(rng.integers(0, len(prefixes) + 1))
    pid = None if choice == len(prefixes) else sorted(prefixes)[choice]
    for rid in ids:
        engine.add_request(rid)
    engine.admit(ids, prefix_id=pid)
    for rid in ids:
        if pid is None:
            shadow.start(rid)
        else:
            shadow.start(rid, *prefixes[pid])
    seed = int(rng.integers(0, 3)) * int(rng.integers(1, 40))
    if seed and engine.cache.num_free_blocks >= len(ids) * (-(-seed // BS) + 1):
        k = _rand(g, L, len(ids), seed, HKV, D)
        v = _rand(g, L, len(ids), seed, HKV, D)
        engine.cache.seed_context(ids, seed, k.to(device), v.to(device))
        for row, rid in enumerate(ids):
            for layer in range(L):
                shadow.k[rid][layer].extend(k[layer, row].float().numpy())
                shadow.v[rid][layer].extend(v[layer, row].float().numpy())


def _register_prefixes(engine, g, device):
    prefixes = {}
    for pid, n in (("pa", 3), ("pb", 6)):
        kb, vb = _rand(g, L, n, HKV, BS, D), _rand(g, L, n, HKV, BS, D)
        engine.register_prefix(pid, kb.to(device), vb.to(device))
        prefixes[pid] = (_prefix_tokens(kb), _prefix_tokens(vb))
    return prefixes


def _step_inputs(g, batch, device):
    return _rand(g, batch, HQ, D).to(device), _rand(g, batch, HKV, D).to(device), _rand(g, batch, HKV, D).to(device)


def _rotated(x, pos):
    """The appended K / rotated q the engine must produce: the reference's own formula
    (flashdec/rope.py:66-82, torch's fp32 functions) on x's device -- the CPU (torch) backend
    evaluates it directly, the HIP kernels read the cache's cos/sin tables built with it --
    which may sit an ulp off the correctly rounded values of the oracle's RoPE."""
    from flashdec_amd.rope import apply_rope

    return apply_rope(x, torch.as_tensor(pos).to(x.device), base=BASE).float().cpu().numpy()


def run_eager_lifecycle(device, seed, iters, max_blocks=56):
    rng = np.random.default_rng(seed)
    g = torch.Generator().manual_seed(seed)
    cache = PagedKVCache(L, HKV, D, BS, max_blocks=max_blocks, dtype=torch.bfloat16, device=device,
                         prefix_cache_capacity_blocks=9)
    engine = DecodeEngine(cache)
    engine.cascade_min_shared_tokens = 16  # attached rows take the shared-prefix launch
    prefixes = _register_prefixes(engine, g, device)
    shadow = Shadow()
    counts = {"committed": 0, "failed": 0, "aborted": 0, "backpressure": 0, "resolved": 0, "checked": 0}
    next_id = 0
    for it in range(iters):
        active = engine.active_request_ids()
        if len(active) < 7 and (not active or rng.random() < 0.35):
            n = int(rng.integers(1, 4))
            ids = [f"r{next_id + i}" for i in range(n)]
            next_id += n
            _admit(engine, shadow, rng, g, ids, prefixes, device)
        active = engine.active_request_ids()
        if len(active) > 1 and rng.random() < 0.2:
            rid = active[int(rng.integers(0, len(active)))]
            (engine.finish_request if rng.random() < 0.5 else engine.cancel_request)(rid)
            shadow.drop(rid)
            counts["resolved"] += 1
        ids = list(engine.active_request_ids())
        if not ids:
            continue
        before = (cache.num_free_blocks, cache.seq_lens_tensor(ids).tolist())
        try:
            tx = engine.begin_step(ids)
        except RuntimeError as e:
            assert "insufficient physical blocks" in str(e)
            assert (cache.num_free_blocks, cache.seq_lens_tensor(ids).tolist()) == before
            rid = max(ids, key=shadow.length)  # free the longest row and go on
            engine.finish_request(rid)
            shadow.drop(rid)
            counts["backpressure"] += 1
            continue
        pos = tx.positions.cpu().numpy()
        assert pos.tolist() == [shadow.length(rid) for rid in ids]
        fail_at = int(rng.integers(0, L)) if rng.random() < 0.12 else None
        abort_after = rng.random() < 0.08
        check = rng.random() < 0.5
        new_rows = {}
        failed = False
        for layer in range(L):
            q, k, v = _step_inputs(g, len(ids), device)
            if layer == fail_at:
                with pytest.raises(ValueError):
                    engine.step_layer(tx, layer, q[..., :-1], k, v, base=BASE)
                failed = True
                break
            res = engine.step_layer(tx, layer, q, k, v, base=BASE)
            k_rot = _rotated(k, pos)
            new_rows[layer] = (list(k_rot), list(v.float().cpu().numpy()))
            if check:
                expected = shadow.expected(ids, layer, _rotated(q, pos), *new_rows[layer])
                assert_close_to_oracle(res.output, expected)
        if failed or abort_after:
            if abort_after and not failed:
                engine.abort_step(tx)
            counts["failed" if failed else "aborted"] += 1
            assert (cache.num_free_blocks, cache.seq_lens_tensor(ids).tolist()) == before
            continue
        engine.commit_step(tx)
        shadow.commit(ids, new_rows)
        counts["committed"] += 1
        if check:
            shadow.check_cache(cache, ids)
            counts["checked"] += 1
    for rid in engine.active_request_ids():
        engine.finish_request(rid)
    for pid in ("pa", "pb"):
        engine.evict_prefix(pid)
    assert cache.num_free_blocks == max_blocks
    assert engine.validate_invariants() and cache.validate_invariants()
    return counts, engine


@pytest.mark.parametrize("seed", [3, 11])
def test_random_eager_lifecycle_on_the_torch_backends(seed):
    """The same lifecycles through the reference's CPU backends (torch append, torch decode): the
    allocator, transactions and prefixes against the shadow, no GPU."""
    counts, engine = run_eager_lifecycle("cpu", seed, iters=60)
    assert (engine.append_backend, engine.decode_backend) == ("torch", "reference")
    assert counts["committed"] > 20 and counts["checked"] > 5 and counts["resolved"] > 3, counts
    assert counts["failed"] + counts["aborted"] > 0, counts


@pytest.mark.gpu
@pytest.mark.parametrize("seed", [3, 11, 29])
def test_random_eager_lifecycle_matches_the_shadow(seed):
    print(f"eager lifecycle seed={seed}", flush=True)
    counts, engine = run_eager_lifecycle("cuda", seed, iters=60)
    assert counts["committed"] > 20 and counts["checked"] > 5, counts
    assert counts["failed"] + counts["aborted"] > 0, counts
    assert engine._cascade_decode_count > 0  # attached rows went through the shared-prefix launch


@pytest.mark.gpu
@pytest.mark.parametrize("fuse_rope", [True, False])
def test_step_graph_over_changing_requests_matches_the_shadow(fuse_rope):
    print(f"graph lifecycle fuse_rope={fuse_rope}", flush=True)
    rng = np.random.default_rng(41)
    g = torch.Generator().manual_seed(41)
    cache = PagedKVCache(L, HKV, D, BS, max_blocks=120, dtype=torch.bfloat16, device="cuda")
    cache.enable_graph_metadata(4, 40)
    engine = DecodeEngine(cache)
    shadow = Shadow()
    prefixes = {}
    ids = [f"r{i}" for i in range(4)]
    _admit(engine, shadow, rng, g, ids, prefixes, "cuda")
    sg = engine.capture_step_graph(4, HQ, base=BASE, fuse_rope=fuse_rope, cascade=False)
    next_id = 4
    replays = aborted = 0
    for it in range(45):
        ids = list(engine.active_request_ids())
        tx = engine.begin_step(ids)
        pos = tx.positions.cpu().numpy()
        assert pos.tolist() == [shadow.length(rid) for rid in ids]
        inputs = [_step_inputs(g, 4, "cuda") for _ in range(L)]
        for layer, (q, k, v) in enumerate(inputs):
            sg.q[layer].copy_(q)
            sg.k[layer].copy_(k)
            sg.v[layer].copy_(v)
        out = engine.step_graph(tx, sg)
        replays += 1
        new_rows = {layer: (list(_rotated(k, pos)), list(v.float().cpu().numpy()))
                    for layer, (q, k, v) in enumerate(inputs)}
        for layer in (0, L - 1):
            expected = shadow.expected(ids, layer, _rotated(inputs[layer][0], pos), *new_rows[layer])
            assert_close_to_oracle(out[layer], expected)
        if rng.random() < 0.1:
            engine.abort_step(tx)
            aborted += 1
            continue
        engine.commit_step(tx)
        shadow.commit(ids, new_rows)
        shadow.check_cache(cache, ids)
        # replace a row now and then: the graph's batch keeps four rows
        if rng.random() < 0.25 or max(shadow.length(r) for r in ids) > 36 * BS:
            rid = max(ids, key=shadow.length) if rng.random() < 0.5 else ids[int(rng.integers(0, 4))]
            (engine.finish_request if rng.random() < 0.5 else engine.cancel_request)(rid)
            shadow.drop(rid)
            new = f"r{next_id}"
            next_id += 1
            _admit(engine, shadow, rng, g, [new], prefixes, "cuda")
    assert replays == 45 and aborted > 0 and next_id > 6
    for rid in engine.active_request_ids():
        engine.finish_request(rid)
    assert cache.num_free_blocks == 120
    assert engine.validate_invariants()
