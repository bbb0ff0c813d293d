"""PagedKVCache against randomized traces recorded on the reference allocator.

``tests/golden/cache_traces.json`` holds seeded operation sequences --
requests added, finished and cancelled, token transactions begun, written
layer by layer, committed, aborted and misused, legacy single-layer appends,
prefixes registered, attached and evicted, table and position queries --
together with what the reference (cysong2025/flashdec flashdec/cache.py:
74-1409) returned or raised for each operation and every public observable
afterwards.  ``tests/golden/make_cache_traces.py`` recorded them; the
operations and observations are the shared code in
``tests/golden/cache_trace_ops.py``.  Bit-exact: results, exception types and
messages, block ids and tables, counters, the metrics dict and K/V checksums.
"""

import json
import os
import sys

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "golden"))

from cache_trace_ops import apply, apply_delta, observe, outcome  # noqa: E402

with open(os.path.join(HERE, "golden", "cache_traces.json")) as f:
    TRACES = json.load(f)["traces"]


def _round_trip(x):
    # the fixture went through JSON: compare in that form
    return json.loads(json.dumps(x))


@pytest.mark.parametrize("trace", TRACES, ids=[t["config"]["name"] for t in TRACES])
def test_trace_matches_reference(trace):
    import torch

    from flashdec_amd.cache import PagedKVCache

    cfg = trace["config"]
    cache = PagedKVCache(cfg["num_layers"], cfg["num_kv_heads"], cfg["head_dim"], cfg["block_size"],
                         cfg["max_blocks"], dtype=torch.float32, device="cpu",
                         prefix_cache_capacity_blocks=cfg["prefix_cache_capacity_blocks"])
    ctx = {}
    names, prefixes = [], []
    expected = None
    for i, step in enumerate(trace["steps"]):
        op = step["op"]
        res = _round_trip(outcome(lambda: apply(cache, op, ctx)))
        assert res == step["result"], f"step {i} {op}: result {res} != reference {step['result']}"
        if op["op"] == "add_request" and "ok" in res and op["rid"] not in names:
            names.append(op["rid"])
        if op["op"] == "register_prefix" and "ok" in res and op["pid"] not in prefixes:
            prefixes.append(op["pid"])
        expected = apply_delta(expected, step["changed"])
        got = _round_trip(observe(cache, names, prefixes))
        for key in expected:
            assert got[key] == expected[key], f"step {i} {op}: {key} {got[key]} != reference {expected[key]}"
        assert set(got) == set(expected)
