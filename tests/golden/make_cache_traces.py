"""Write ``cache_traces.json``: seeded random PagedKVCache traces recorded on the reference.

The reference allocator (cysong2025/flashdec flashdec/cache.py:74-1409) is
imported from the checkout given on the command line and driven through its
public API with the operations of ``cache_trace_ops``.  Each operation's
result (or exception type and message) and every observable afterwards
(state version, free/used counts, the metrics dict, each request's and
prefix's state, the invariant check, K/V checksums) is recorded.  Only these
inputs and outputs are committed; the reference itself is not.

    python tests/golden/make_cache_traces.py /root/reference
"""

from __future__ import annotations

import json
import os
import random
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from cache_trace_ops import apply, delta, observe, outcome  # noqa: E402

# name, cache shape, operation count, seed
CONFIGS = [
    {"name": "two_layers", "num_layers": 2, "num_kv_heads": 1, "head_dim": 4, "block_size": 4, "max_blocks": 20,
     "prefix_cache_capacity_blocks": 6, "ops": 150, "seed": 11},
    {"name": "one_layer_legacy_append", "num_layers": 1, "num_kv_heads": 2, "head_dim": 2, "block_size": 2,
     "max_blocks": 12, "prefix_cache_capacity_blocks": 4, "ops": 120, "seed": 12},
    {"name": "tight_pool", "num_layers": 3, "num_kv_heads": 1, "head_dim": 2, "block_size": 2, "max_blocks": 9,
     "prefix_cache_capacity_blocks": 4, "ops": 150, "seed": 13},
    {"name": "prefix_churn", "num_layers": 2, "num_kv_heads": 1, "head_dim": 2, "block_size": 2, "max_blocks": 14,
     "prefix_cache_capacity_blocks": 6, "ops": 160, "seed": 14, "prefix_bias": True},
]


def _pick_op(rng, cache, ctx, names, prefixes, cfg):
    """A plausible next operation, with invalid ones mixed in (their errors are recorded too)."""
    states = {}
    for rid in names:
        r = outcome(lambda: cache.request_state(rid))
        if "ok" in r:
            states[rid] = r["ok"]
    active = [rid for rid, st in states.items() if st["status"] == "active"]
    tx = ctx.get("tx")
    r = rng.random()
    if tx is not None:
        if tx.next_layer_idx == cfg["num_layers"] and r < 0.6:
            return {"op": "commit_token"}
        if r < 0.05:
            return {"op": "begin_token", "rids": active[:1] or ["r0"]}
        if r < 0.10:
            return {"op": "transaction_view"}
        if r < 0.15:
            return {"op": "commit_token", "stale": True}
        if r < 0.20:
            return {"op": "write_token_layer", "layer": rng.randrange(cfg["num_layers"] + 1), "base": rng.randrange(50)}
        if r < 0.24:
            return {"op": "write_token_layer", "layer": 0, "base": 3, "rows": len(tx.request_ids) + 1}
        if r < 0.30:
            return {"op": "abort_token"}
        if r < 0.34 and active:
            return {"op": "finish_request", "rid": rng.choice(active)}
        if r < 0.38:
            return {"op": "commit_token"}
        return {"op": "write_token_layer", "layer": tx.next_layer_idx % cfg["num_layers"], "base": rng.randrange(50)}
    if cfg.get("prefix_bias") and r < 0.3:
        # new requests that take a resident prefix at once, and registry churn
        r2 = rng.random()
        if r2 < 0.4:
            return {"op": "add_request", "rid": f"r{len(names)}"}
        empty = [rid for rid in active if states[rid]["seq_len"] == 0]
        if r2 < 0.75 and empty and prefixes:
            return {"op": "attach_prefix", "rid": rng.choice(empty), "pid": rng.choice(prefixes)}
        if r2 < 0.9:
            pid = f"p{rng.randrange(5)}"
            return {"op": "register_prefix", "pid": pid, "blocks": rng.randint(1, 3), "base": rng.randrange(50)}
        return {"op": "evict_prefix", "pid": rng.choice(prefixes) if prefixes else "p0"}
    if r < 0.16 or not active:
        if rng.random() < 0.08 and names:
            return {"op": "add_request", "rid": rng.choice(names)}  # duplicate id
        return {"op": "add_request", "rid": f"r{len(names)}"}
    if r < 0.50:
        k = rng.randint(1, min(4, len(active)))
        rids = rng.sample(active, k)
        if rng.random() < 0.05:
            rids = rids + rids[:1]  # duplicate ids
        if cfg["num_layers"] == 1 and rng.random() < 0.6:
            return {"op": "append", "layer": 0, "rids": rids, "base": rng.randrange(50)}
        return {"op": "begin_token", "rids": rids}
    if r < 0.58:
        return {"op": "finish_request", "rid": rng.choice(active)}
    if r < 0.64:
        return {"op": "cancel_request", "rid": rng.choice(active + ["missing"])}
    if r < 0.72:
        pid = f"p{rng.randrange(4)}"
        return {"op": "register_prefix", "pid": pid, "blocks": rng.randint(1, 3), "base": rng.randrange(50)}
    if r < 0.80:
        empty = [rid for rid in active if states[rid]["seq_len"] == 0]
        rid = rng.choice(empty) if empty and rng.random() < 0.8 else rng.choice(active)
        pid = rng.choice(prefixes) if prefixes and rng.random() < 0.85 else f"p{rng.randrange(4)}"
        return {"op": "attach_prefix", "rid": rid, "pid": pid}
    if r < 0.85:
        pid = rng.choice(prefixes) if prefixes and rng.random() < 0.7 else f"p{rng.randrange(4)}"
        return {"op": "evict_prefix", "pid": pid}
    if r < 0.90:
        return {"op": "next_positions", "rids": rng.sample(active, rng.randint(1, len(active)))}
    if r < 0.95:
        return {"op": "block_tables", "rids": rng.sample(active, rng.randint(1, len(active))),
                "width": rng.choice([None, 8])}
    return {"op": "seq_lens_tensor", "rids": active}


def record(PagedKVCache, cfg):
    import torch

    rng = random.Random(cfg["seed"])
    cache = PagedKVCache(cfg["num_layers"], cfg["num_kv_heads"], cfg["head_dim"], cfg["block_size"],
                         cfg["max_blocks"], dtype=torch.float32, device="cpu",
                         prefix_cache_capacity_blocks=cfg["prefix_cache_capacity_blocks"])
    ctx = {}
    names, prefixes, steps = [], [], []
    prev = None
    for _ in range(cfg["ops"]):
        op = _pick_op(rng, cache, ctx, names, prefixes, cfg)
        res = outcome(lambda: apply(cache, op, ctx))
        if op["op"] == "add_request" and "ok" in res and op["rid"] not in names:
            names.append(op["rid"])
        if op["op"] == "register_prefix" and "ok" in res and op["pid"] not in prefixes:
            prefixes.append(op["pid"])
        obs = observe(cache, names, prefixes)
        steps.append({"op": op, "result": res, "changed": delta(prev, obs)})
        prev = obs
    return {"config": cfg, "steps": steps}


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, root)
    from flashdec.cache import PagedKVCache

    traces = [record(PagedKVCache, cfg) for cfg in CONFIGS]
    out = os.path.join(HERE, "cache_traces.json")
    with open(out, "w") as f:
        json.dump({"source": "cysong2025/flashdec flashdec/cache.py (PagedKVCache), imported from the checkout",
                   "generator": "tests/golden/make_cache_traces.py", "traces": traces}, f,
                  separators=(",", ":"))
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
