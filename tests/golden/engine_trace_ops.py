"""Operations and observations of the recorded DecodeEngine traces.

Like ``cache_trace_ops`` for the allocator: one module drives the generator
(``make_engine_traces.py``, on the reference engine of cysong2025/flashdec
flashdec/engine.py:21-1183 with its CPU backends ``append_backend="torch"``,
``decode_backend="reference"``) and the replay
(``tests/test_engine_traces_cpu.py``, on ``flashdec_amd.engine.DecodeEngine``
with the same backends).  q/K/V are rebuilt from integer bases (``ramp``).
"""

from __future__ import annotations

from cache_trace_ops import normalize, observe as observe_cache, outcome, ramp


def observe(engine, request_ids, prefix_ids):
    """Engine observables plus the cache's (see ``cache_trace_ops.observe``).

    The engine's request states carry the cache's, and its metrics the
    cache's metrics dict, which is kept as a key of its own so that an
    observation's delta stays per counter.
    """
    metrics = normalize(engine.metrics())
    cache_metrics = metrics.pop("cache")
    obs = {
        "engine_version": engine.state_version,
        "engine_metrics": metrics,
        "active": normalize(engine.active_request_ids()),
        "engine_requests": {},
        "engine_invariants": outcome(engine.validate_invariants),
        "cache_metrics": cache_metrics,
    }
    for rid in request_ids:
        obs["engine_requests"][rid] = outcome(lambda: engine.request_state(rid))
    cache_obs = observe_cache(engine.cache, [], prefix_ids)
    obs.update({f"cache_{k}": v for k, v in cache_obs.items() if k not in ("metrics", "requests")})
    return obs


def apply(engine, op, ctx):
    """Run one operation; ctx carries the open step handle and the last closed one."""
    cache = engine.cache
    kind = op["op"]
    hq, hkv, d = op.get("hq", 2), cache.num_kv_heads, cache.head_dim
    if kind == "add_request":
        return engine.add_request(op["rid"])
    if kind == "admit":
        return engine.admit(op.get("rids"))
    if kind == "finish_request":
        return engine.finish_request(op["rid"])
    if kind == "cancel_request":
        return engine.cancel_request(op["rid"])
    if kind == "register_prefix":
        shape = (cache.num_layers, op["blocks"], hkv, cache.block_size, d)
        return engine.register_prefix(op["pid"], ramp(op["base"], shape), ramp(op["base"] + 3, shape))
    if kind == "evict_prefix":
        return engine.evict_prefix(op["pid"])
    if kind == "cache_attach_prefix":
        # the cache mutated behind the engine's back
        return cache.attach_prefix(op["rid"], op["pid"])
    if kind == "begin_step":
        handle = engine.begin_step(op.get("rids"))
        ctx["tx"] = handle
        return handle
    if kind == "step_layer":
        tx = ctx.get("tx")
        n = op.get("rows", len(tx.request_ids) if tx is not None else 1)
        q = ramp(op["base"], (n, hq, d))
        k = ramp(op["base"] + 4, (n, hkv, d))
        v = ramp(op["base"] + 9, (n, hkv, d))
        return engine.step_layer(tx, op["layer"], q, k, v, rotary_dim=op.get("rotary_dim"),
                                 base=op.get("rope_base", 10_000.0))
    if kind in ("commit_step", "abort_step"):
        tx = ctx.get("old_tx") if op.get("stale") else ctx.get("tx")
        result = getattr(engine, kind)(tx)
        if not op.get("stale"):
            ctx["old_tx"], ctx["tx"] = ctx.get("tx"), None
        return result
    if kind == "step":
        n = len(op["rids"]) if op.get("rids") else len(engine.active_request_ids())
        q = ramp(op["base"], (n, hq, d))
        k = ramp(op["base"] + 4, (n, hkv, d))
        v = ramp(op["base"] + 9, (n, hkv, d))
        return engine.step(q, k, v, request_ids=op.get("rids"), rotary_dim=op.get("rotary_dim"))
    raise ValueError(f"unknown trace operation {kind!r}")
