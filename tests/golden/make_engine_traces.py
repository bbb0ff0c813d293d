"""Write ``engine_traces.json``: seeded random DecodeEngine traces recorded on the reference.

The reference engine (cysong2025/flashdec flashdec/engine.py:21-1183) and
allocator are imported from the checkout given on the command line and run
on the CPU with their own backends (``append_backend="torch"``,
``decode_backend="reference"``).  Each operation's result (or exception type
and message) and every engine and cache observable afterwards are recorded;
only these inputs and outputs are committed.

    python tests/golden/make_engine_traces.py /root/reference
"""

from __future__ import annotations

import json
import os
import random
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, HERE)

from cache_trace_ops import delta, outcome  # noqa: E402
from engine_trace_ops import apply, observe  # noqa: E402

CONFIGS = [
    {"name": "two_layers", "num_layers": 2, "num_kv_heads": 1, "head_dim": 4, "block_size": 2, "max_blocks": 16,
     "prefix_cache_capacity_blocks": 4, "ops": 120, "seed": 21},
    {"name": "one_layer_step", "num_layers": 1, "num_kv_heads": 1, "head_dim": 4, "block_size": 2, "max_blocks": 10,
     "prefix_cache_capacity_blocks": 2, "ops": 110, "seed": 22},
    {"name": "tight_pool_rope", "num_layers": 3, "num_kv_heads": 2, "head_dim": 4, "block_size": 2, "max_blocks": 8,
     "prefix_cache_capacity_blocks": 2, "ops": 120, "seed": 23, "rope": True},
]

# prefixes are registered before the first request (the reference engine
# refuses later registrations), then the random operations follow
PRELUDE = [{"op": "register_prefix", "pid": "p0", "blocks": 1, "base": 5},
           {"op": "register_prefix", "pid": "p1", "blocks": 1, "base": 9}]


def _pick_op(rng, engine, ctx, names, prefixes, cfg):
    active = list(engine.active_request_ids())
    waiting = []
    for rid in names:
        st = outcome(lambda: engine.request_state(rid))
        if "ok" in st and st["ok"]["status"] == "waiting":
            waiting.append(rid)
    tx = ctx.get("tx")
    rope = {"rotary_dim": rng.choice([None, 2, 4]), "rope_base": 10_000.0} if cfg.get("rope") else {}
    r = rng.random()
    if tx is not None:
        nxt = ctx.get("next_layer", 0)
        if nxt == cfg["num_layers"] and r < 0.6:
            return {"op": "commit_step"}
        if r < 0.04:
            return {"op": "begin_step"}
        if r < 0.08:
            return {"op": "commit_step", "stale": True}
        if r < 0.12:
            return {"op": "step_layer", "layer": (nxt + 1) % cfg["num_layers"], "base": rng.randrange(40)}
        if r < 0.15:
            return {"op": "step_layer", "layer": nxt, "base": 1, "rows": len(tx.request_ids) + 1}
        if r < 0.21:
            return {"op": "abort_step"}
        if r < 0.24 and active:
            return {"op": "finish_request", "rid": rng.choice(active)}
        if r < 0.28:
            return {"op": "commit_step"}
        return {"op": "step_layer", "layer": nxt % cfg["num_layers"], "base": rng.randrange(40), **rope}
    if r < 0.14 or not names:
        if rng.random() < 0.06 and names:
            return {"op": "add_request", "rid": rng.choice(names)}
        return {"op": "add_request", "rid": f"r{len(names)}"}
    if r < 0.24:
        if waiting and rng.random() < 0.7:
            return {"op": "admit", "rids": rng.sample(waiting, rng.randint(1, len(waiting)))}
        return {"op": "admit"}
    if r < 0.56 and active:
        rids = None if rng.random() < 0.3 else rng.sample(active, rng.randint(1, min(3, len(active))))
        if cfg["num_layers"] == 1 and rng.random() < 0.6:
            return {"op": "step", "rids": rids, "base": rng.randrange(40)}
        return {"op": "begin_step", "rids": rids}
    if r < 0.64 and active:
        return {"op": "finish_request", "rid": rng.choice(active)}
    if r < 0.70:
        return {"op": "cancel_request", "rid": rng.choice(active + names + ["missing"])}
    if r < 0.80:
        return {"op": "register_prefix", "pid": f"p{rng.randrange(3)}", "blocks": rng.randint(1, 2),
                "base": rng.randrange(40)}
    if r < 0.86:
        pid = rng.choice(prefixes) if prefixes and rng.random() < 0.7 else f"p{rng.randrange(3)}"
        return {"op": "evict_prefix", "pid": pid}
    if r < 0.90 and active and prefixes:
        return {"op": "cache_attach_prefix", "rid": rng.choice(active), "pid": rng.choice(prefixes)}
    return {"op": "admit", "rids": ["missing"]}


def record(PagedKVCache, DecodeEngine, cfg):
    import torch

    rng = random.Random(cfg["seed"])
    cache = PagedKVCache(cfg["num_layers"], cfg["num_kv_heads"], cfg["head_dim"], cfg["block_size"],
                         cfg["max_blocks"], dtype=torch.float32, device="cpu",
                         prefix_cache_capacity_blocks=cfg["prefix_cache_capacity_blocks"])
    engine = DecodeEngine(cache, append_backend="torch", decode_backend="reference")
    ctx = {}
    names, prefixes, steps = [], [], []
    prev = None
    for i in range(cfg["ops"]):
        op = PRELUDE[i] if i < len(PRELUDE) else _pick_op(rng, engine, ctx, names, prefixes, cfg)
        res = outcome(lambda: apply(engine, op, ctx))
        if op["op"] == "add_request" and "ok" in res and op["rid"] not in names:
            names.append(op["rid"])
        if op["op"] == "register_prefix" and "ok" in res and op["pid"] not in prefixes:
            prefixes.append(op["pid"])
        if op["op"] == "begin_step" and "ok" in res:
            ctx["next_layer"] = 0
        if op["op"] == "step_layer":
            ctx["next_layer"] = ctx.get("next_layer", 0) + 1 if "ok" in res else 0
            if "error" in res:
                ctx["tx"] = None  # a failed layer aborts the whole step
        obs = observe(engine, names, prefixes)
        steps.append({"op": op, "result": res, "changed": delta(prev, obs)})
        prev = obs
    return {"config": cfg, "steps": steps}


def main():
    root = sys.argv[1] if len(sys.argv) > 1 else "/root/reference"
    sys.path.insert(0, root)
    from flashdec.cache import PagedKVCache
    from flashdec.engine import DecodeEngine

    traces = [record(PagedKVCache, DecodeEngine, cfg) for cfg in CONFIGS]
    out = os.path.join(HERE, "engine_traces.json")
    with open(out, "w") as f:
        json.dump({"source": "cysong2025/flashdec flashdec/engine.py (DecodeEngine) and flashdec/cache.py, "
                             "imported from the checkout", "generator": "tests/golden/make_engine_traces.py",
                   "traces": traces}, f, separators=(",", ":"))
    print(out, os.path.getsize(out), "bytes")


if __name__ == "__main__":
    main()
