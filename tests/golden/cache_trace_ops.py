"""Operations and observations of the recorded PagedKVCache traces.

One module drives both sides of ``cache_traces.json``: the generator
(``make_cache_traces.py``) applies each operation to the reference allocator
(cysong2025/flashdec flashdec/cache.py:74-1409) and stores what it observes;
``tests/test_cache_traces_cpu.py`` applies the same operations to
``flashdec_amd.cache.PagedKVCache`` and compares every observation.  Because
the same code runs on both, a difference can only come from the allocators.

An operation is a dict ``{"op": name, ...}``.  Tensor arguments are not
stored: they are rebuilt from a small integer ``base`` (``ramp``), so K/V
values are small integers and the cache checksums below are exact.
"""

from __future__ import annotations

import dataclasses

import torch


def ramp(base, shape):
    """Deterministic small-integer float32 tensor: ((i + base) % 13) - 6 over the flat index i."""
    n = 1
    for s in shape:
        n *= s
    return ((torch.arange(n, dtype=torch.int64) + int(base)) % 13 - 6).to(torch.float32).reshape(shape)


def normalize(x):
    """Plain JSON-able form of a result: tensors and tuples become lists, dataclasses dicts."""
    if isinstance(x, torch.Tensor):
        return normalize(x.detach().cpu().tolist())
    if dataclasses.is_dataclass(x) and not isinstance(x, type):
        return {f.name: normalize(getattr(x, f.name)) for f in dataclasses.fields(x)}
    if isinstance(x, dict):
        return {str(k): normalize(v) for k, v in x.items()}
    if isinstance(x, (list, tuple)):
        return [normalize(v) for v in x]
    if x is None or isinstance(x, (bool, int, float, str)):
        return x
    return {"object": type(x).__name__}  # e.g. a method returning the cache itself


def _checksum(t):
    w = (torch.arange(t.numel(), dtype=torch.float64) % 97 + 1).reshape(t.shape)
    return float((t.double() * w).sum())


def observe(cache, request_ids, prefix_ids):
    """Every public observable after an operation."""
    obs = {
        "version": cache.state_version,
        "free": cache.num_free_blocks,
        "used": cache.num_used_blocks,
        "open": cache.has_open_transaction,
        "metrics": normalize(cache.metrics()),
        "requests": {},
        "prefixes": {},
        "k": _checksum(cache.k_cache),
        "v": _checksum(cache.v_cache),
    }
    for rid in request_ids:
        obs["requests"][rid] = outcome(lambda: cache.request_state(rid))
    for pid in prefix_ids:
        obs["prefixes"][pid] = outcome(lambda: cache.prefix_state(pid))
    obs["invariants"] = outcome(cache.validate_invariants)
    return obs


def outcome(fn):
    """{"ok": normalized result} or {"error": [exception type, message]}."""
    try:
        return {"ok": normalize(fn())}
    except Exception as exc:  # the trace records error paths too
        return {"error": [type(exc).__name__, str(exc)]}


def apply(cache, op, ctx):
    """Run one operation; ctx carries the open transaction handle and the last finished one."""
    kind = op["op"]
    if kind == "add_request":
        return cache.add_request(op["rid"])
    if kind == "finish_request":
        return cache.finish_request(op["rid"])
    if kind == "cancel_request":
        return cache.cancel_request(op["rid"])
    if kind == "begin_token":
        view = cache.begin_token(op["rids"])
        ctx["tx"] = view
        return view
    if kind == "write_token_layer":
        tx = ctx.get("tx")
        n = op.get("rows", len(tx.request_ids) if tx is not None else 1)
        shape = (n, cache.num_kv_heads, cache.head_dim)
        view = cache.write_token_layer(tx, op["layer"], ramp(op["base"], shape), ramp(op["base"] + 5, shape))
        ctx["tx"] = view  # the latest snapshot (next_layer_idx advanced)
        return view
    if kind in ("commit_token", "abort_token"):
        tx = ctx.get("old_tx") if op.get("stale") else ctx.get("tx")
        result = getattr(cache, kind)(tx)
        if not op.get("stale"):
            ctx["old_tx"], ctx["tx"] = ctx.get("tx"), None
        return result
    if kind == "transaction_view":
        return cache.transaction_view(ctx.get("tx"))
    if kind == "register_prefix":
        shape = (cache.num_layers, op["blocks"], cache.num_kv_heads, cache.block_size, cache.head_dim)
        return cache.register_prefix(op["pid"], ramp(op["base"], shape), ramp(op["base"] + 3, shape))
    if kind == "attach_prefix":
        return cache.attach_prefix(op["rid"], op["pid"])
    if kind == "evict_prefix":
        return cache.evict_prefix(op["pid"])
    if kind == "append":
        n = len(op["rids"])
        shape = (n, cache.num_kv_heads, cache.head_dim)
        return cache.append(op["layer"], op["rids"], ramp(op["base"], shape), ramp(op["base"] + 7, shape))
    if kind == "next_positions":
        return cache.next_positions(op["rids"])
    if kind == "block_tables":
        return cache.block_tables(op["rids"], max_blocks_per_seq=op.get("width"))
    if kind == "seq_lens_tensor":
        return cache.seq_lens_tensor(op["rids"])
    raise ValueError(f"unknown trace operation {kind!r}")


def delta(prev, obs):
    """What changed from ``prev`` to ``obs``: top-level values, and per key inside nested dicts.

    Keys never disappear between observations (the known request and prefix
    ids only grow, the metrics keys are fixed), so a delta is only updates.
    """
    out = {}
    for key, value in obs.items():
        old = prev.get(key) if prev else None
        if isinstance(value, dict) and isinstance(old, dict):
            sub = {k: v for k, v in value.items() if old.get(k, _MISSING) != v}
            if sub:
                out[key] = sub
        elif old != value or prev is None or key not in prev:
            out[key] = value
    return out


def apply_delta(prev, d):
    """Inverse of ``delta``: the full observation after ``d``."""
    obs = {k: (dict(v) if isinstance(v, dict) else v) for k, v in (prev or {}).items()}
    for key, value in d.items():
        if isinstance(value, dict) and isinstance(obs.get(key), dict):
            obs[key].update(value)
        else:
            obs[key] = value
    return obs


_MISSING = object()
