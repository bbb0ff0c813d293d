"""DecodeEngine against randomized traces recorded on the reference engine.

``tests/golden/engine_traces.json`` holds seeded operation sequences -- requests
added, admitted, finished and cancelled, multi-layer decode steps begun,
run layer by layer (with and without RoPE), committed, aborted and misused,
single-layer ``step`` calls, prefix registration and eviction, and a cache
mutated behind the engine -- with what the reference engine (cysong2025/
flashdec flashdec/engine.py:21-1183, CPU backends ``torch`` / ``reference``)
returned or raised and every engine and cache observable afterwards.
``tests/golden/make_engine_traces.py`` recorded them; operations and
observations are the shared code in ``tests/golden/engine_trace_ops.py``.

Exact: exception types and messages, ids, positions, block ids and tables,
lengths, counters, versions.  Attention outputs and K/V checksums are floats
computed by two implementations of the same math (the reference's fp32 torch
oracle and this package's): equal within 1e-5 relative / absolute.
"""

import json
import math
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

from cache_trace_ops import apply_delta, outcome  # noqa: E402
from engine_trace_ops import apply, observe  # noqa: E402

with open(os.path.join(HERE, "golden", "engine_traces.json")) as f:
    TRACES = json.load(f)["traces"]

TOL = 1e-5


def _same(a, b):
    """Structural equality; floats within TOL (ints, strings, bools and None exactly)."""
    if isinstance(a, float) or isinstance(b, float):
        if isinstance(a, bool) or isinstance(b, bool) or not isinstance(a, (int, float)) \
                or not isinstance(b, (int, float)):
            return False
        if math.isnan(a) or math.isnan(b):
            return math.isnan(a) and math.isnan(b)
        return math.isclose(a, b, rel_tol=TOL, abs_tol=TOL)
    if isinstance(a, dict) and isinstance(b, dict):
        return a.keys() == b.keys() and all(_same(a[k], b[k]) for k in a)
    if isinstance(a, list) and isinstance(b, list):
        return len(a) == len(b) and all(_same(x, y) for x, y in zip(a, b))
    return a == b


def _round_trip(x):
    return json.loads(json.dumps(x))


@pytest.mark.parametrize("trace", TRACES, ids=[t["config"]["name"] for t in TRACES])
def test_trace_matches_reference(trace):
    import torch

    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine

    cfg = trace["config"]
    cache = PagedKVCache(cfg["num_layers"], cfg["num_kv_heads"], cfg["head_dim"], cfg["block_size"],
                         cfg["max_blocks"], dtype=torch.float32, device="cpu",
                         prefix_cache_capacity_blocks=cfg["prefix_cache_capacity_blocks"])
    engine = DecodeEngine(cache, append_backend="torch", decode_backend="reference")
    ctx = {}
    names, prefixes = [], []
    expected = None
    for i, step in enumerate(trace["steps"]):
        op = step["op"]
        res = _round_trip(outcome(lambda: apply(engine, op, ctx)))
        assert _same(res, step["result"]), f"step {i} {op}: result {res} != reference {step['result']}"
        if op["op"] == "add_request" and "ok" in res and op["rid"] not in names:
            names.append(op["rid"])
        if op["op"] == "register_prefix" and "ok" in res and op["pid"] not in prefixes:
            prefixes.append(op["pid"])
        if op["op"] == "step_layer" and "error" in res:
            ctx["tx"] = None  # a failed layer aborts the whole step (the generator tracks the same)
        expected = apply_delta(expected, step["changed"])
        got = _round_trip(observe(engine, names, prefixes))
        assert set(got) == set(expected), f"step {i} {op}: keys {sorted(got)} != {sorted(expected)}"
        for key in expected:
            assert _same(got[key], expected[key]), f"step {i} {op}: {key} {got[key]} != reference {expected[key]}"
