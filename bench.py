"""Paged-decode benchmark on one MI355X (ctx 2048).

A step is one ``paged_decode_attention_into`` call (the hot path) over one
synthetic batch: B=8 requests, Hq=16 / Hkv=2 (Qwen2.5-3B attention shape),
head_dim 128, bf16, 32-token blocks, every seq_len = 2048, block tables drawn
from a shuffled pool of 1.25x the needed blocks.  Inputs are resident in HBM
before timing starts.  Steps rotate over ``--pools`` independent KV pools
(default 48 x 21 MB ~ 1 GB) so the 256 MB Infinity Cache cannot serve them.

Timing:
* ``ms_per_step``/``value``: K steps captured in one hipGraph, replayed once
  between two synchronisations (the serving-loop view, launch gaps included).
* ``roofline.achieved``: algorithmic bytes per call / mean duration of the
  dominant kernel (the attention kernel), measured live: every call of a
  separate eager loop passes HIP events through the library's
  ``timing_events`` hook, which records them around exactly that dispatch
  (and around the split reducer, reported beside it).
* ``roofline.traffic``: HBM bytes per attention-kernel dispatch from the
  committed PMC summary ``profiles/decode_mfma_b8_ctx2048_traffic.json``
  (FETCH_SIZE + WRITE_SIZE scaled by a copy kernel of known size), or null.
* ``cpu_baseline``: the repo's numpy oracle (one thread) on a bounded sample
  of the same workload, on this host.

``--profile-kernels N`` instead runs N eager calls and a 64 MiB device copy
(the counter-scaling reference) and prints one line: the form profiled by
``rocprofv3 --kernel-trace --stats`` and ``rocprofv3 --pmc``.

Prints one JSON line.  ``--gpus N`` with N > 1 exits: this build runs on one GPU.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "paged-decode µs/call + achieved HBM GB/s (% of peak), B8 ctx2048 Qwen2.5-3B shape"
HBM_PEAK_GBS = 8000.0
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "decode_mfma_b8_ctx2048_traffic.json")
COPY_PROBE_MIB = 64


def log(msg):
    print(msg, file=sys.stderr, flush=True)


def parse_args():
    p = argparse.ArgumentParser(description=__doc__)
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=480)
    p.add_argument("--warmup", type=int, default=96)
    p.add_argument("--ctx", type=int, default=2048)
    p.add_argument("--batch", type=int, default=8)
    p.add_argument("--pools", type=int, default=48)
    p.add_argument("--cpu-seconds", type=float, default=10.0, help="budget for the CPU baseline sample")
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    p.add_argument("--profile-kernels", type=int, default=0, metavar="N",
                   help="run N eager calls plus a 64 MiB copy (for rocprofv3) and exit")
    return p.parse_args()


def build_pools(torch, n_pools, batch, ctx, hq, hkv, d, bs, dev):
    """n_pools independent (q, k_cache, v_cache, table, seq_lens, out) sets."""
    nblk = (ctx + bs - 1) // bs
    pool_blocks = int(math.ceil(batch * nblk * 1.25))
    pools = []
    gen = torch.Generator(device=dev)
    for i in range(n_pools):
        gen.manual_seed(20260830 + batch + ctx + i)
        k = torch.randn((pool_blocks, hkv, bs, d), device=dev, generator=gen, dtype=torch.float32).to(torch.bfloat16)
        v = torch.randn((pool_blocks, hkv, bs, d), device=dev, generator=gen, dtype=torch.float32).to(torch.bfloat16)
        q = torch.randn((batch, hq, d), device=dev, generator=gen, dtype=torch.float32).to(torch.bfloat16)
        perm = torch.randperm(pool_blocks, device=dev, generator=gen)[: batch * nblk]
        table = perm.view(batch, nblk).to(torch.int32).contiguous()
        lens = torch.full((batch,), ctx, device=dev, dtype=torch.int32)
        out = torch.empty_like(q)
        pools.append((q, k, v, table, lens, out))
    return pools


def algorithmic_bytes(batch, ctx, hq, hkv, d, bs, elt=2):
    nblk = (ctx + bs - 1) // bs
    return batch * ctx * hkv * d * 2 * elt + 2 * batch * hq * d * elt + 4 * batch * nblk + 4 * batch


def prepared_args(pool, sm_scale, block_size, num_kv_heads):
    """The ctypes argument block ``paged_decode_attention_into`` builds for this pool (auto splits)."""
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    q, k, v, table, lens, out = pool
    stream = _lib.current_stream_handle(q.device)
    max_seq_len = table.shape[1] * block_size
    splits = _lib.paged_decode_plan(q.shape[0], q.shape[1], num_kv_heads, q.shape[2], max_seq_len)
    args = _lib.PagedDecodeArgs()
    pd._fill_common(args, q, k, v, pd._cache_strides(k, 2, 3), pd._cache_strides(v, 2, 3), table, lens, out,
                    num_kv_heads, block_size, sm_scale)
    args.num_blocks = k.shape[0]
    args.max_seq_len = max_seq_len
    acc = mx = sm = None
    if splits > 1:
        acc, mx, sm, _ = pd._auto_workspace(q, num_kv_heads, splits, stream)
    pd._fill_workspace(args, acc, mx, sm, splits)
    return args, stream


def load_traffic():
    """HBM bytes per attention-kernel dispatch from the committed PMC summary, or None."""
    try:
        with open(TRAFFIC_SUMMARY) as f:
            t = json.load(f)
        return float(t["fetch_bytes_per_dispatch"]) + float(t["write_bytes_per_dispatch"]), t
    except (OSError, KeyError, ValueError):
        return None, None


def cpu_baseline(pools, budget_s, sm_scale):
    """Median seconds per call of the numpy oracle on pool 0 (one BLAS thread)."""
    import numpy as np
    from threadpoolctl import threadpool_limits

    from oracle.attention import paged_decode_attention as oracle_decode

    q, k, v, table, lens, _ = pools[0]
    qn = q.float().cpu().numpy()
    kn = k.float().cpu().numpy()
    vn = v.float().cpu().numpy()
    tn = table.cpu().numpy()
    ln = lens.cpu().numpy()
    times = []
    with threadpool_limits(limits=1):
        t_end = time.perf_counter() + budget_s
        while len(times) < 3 or (time.perf_counter() < t_end and len(times) < 1000):
            t0 = time.perf_counter()
            oracle_decode(qn, kn, vn, tn, ln, sm_scale=sm_scale, out_dtype="bfloat16")
            times.append(time.perf_counter() - t0)
    del np
    return statistics.median(times), len(times)


def back_to_back(torch, lib, prepared, n, events=None):
    """n library calls submitted while the GPU is held busy, so they run back to back.

    A sleep kernel occupies the stream while the host enqueues every call;
    ``events[i]`` (four HIP events) go through the library's timing hook.
    """
    torch.cuda.synchronize()
    torch.cuda._sleep(200_000_000)
    for i in range(n):
        a, st = prepared[i % len(prepared)]
        if events is not None:
            a.timing_events[:] = [e.cuda_event for e in events[i]]
        lib.paged_decode(a, st)
        if events is not None:
            a.timing_events[:] = [None] * 4
    torch.cuda.synchronize()


def profile_kernels(torch, dev, lib, prepared, n):
    """Back-to-back calls and a plain copy of known size, for rocprofv3 runs."""
    back_to_back(torch, lib, prepared, n)
    numel = COPY_PROBE_MIB * 2**20 // 2
    src = torch.ones(numel, device=dev, dtype=torch.bfloat16)
    dst = torch.empty_like(src)
    for _ in range(4):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"profile_kernels": n, "copy_probe_mib": COPY_PROBE_MIB, "copies": 4}), flush=True)


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on exactly one GPU; --gpus {args.gpus} is not supported "
            "(the decode path shards per request / KV head with no exchange).",
            file=sys.stderr,
        )
        sys.exit(2)

    import torch

    import flashdec_amd as fd
    from flashdec_amd import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    _lib.load_library()
    batch, ctx, hq, hkv, d, bs = args.batch, args.ctx, 16, 2, 128, 32
    sm_scale = 1.0 / math.sqrt(d)
    log(f"[bench] building {args.pools} KV pools: B{batch} ctx{ctx} Hq{hq}/Hkv{hkv} D{d} bs{bs} bf16")
    pools = build_pools(torch, args.pools, batch, ctx, hq, hkv, d, bs, dev)
    pool_bytes = sum(p[1].numel() * 2 * 2 for p in pools)
    nbytes = algorithmic_bytes(batch, ctx, hq, hkv, d, bs)
    splits = _lib.paged_decode_plan(batch, hq, hkv, d, pools[0][3].shape[1] * bs)
    log(f"[bench] KV pool bytes {pool_bytes / 2**20:.0f} MiB, algorithmic bytes/call {nbytes}, splits {splits}")

    def call(i):
        q, k, v, table, lens, out = pools[i % len(pools)]
        fd.paged_decode_attention_into(q, k, v, table, lens, out, sm_scale=sm_scale)

    stream = torch.cuda.current_stream(dev)
    call(0)  # one call through the public API builds the stream's split workspace
    prepared = [prepared_args(pool, sm_scale, bs, hkv) for pool in pools]
    if args.profile_kernels:
        profile_kernels(torch, dev, _lib, prepared, args.profile_kernels)
        return
    back_to_back(torch, _lib, prepared, args.warmup)
    log("[bench] warmup done")

    # K steps in one graph, replayed once inside the timed region
    graph = torch.cuda.CUDAGraph()
    cap = torch.cuda.Stream(dev)
    cap.wait_stream(stream)
    with torch.cuda.stream(cap):
        call(0)  # the capture stream's split workspace exists before capture
        cap.synchronize()
        with torch.cuda.graph(graph, stream=cap):
            for i in range(args.steps):
                call(i)
    stream.wait_stream(cap)
    torch.cuda.synchronize()
    graph.replay()  # untimed replay (first-replay setup)
    torch.cuda.synchronize()
    t_start = torch.cuda.Event(enable_timing=True)
    t_stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    graph.replay()
    t_stop.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_stop)
    ms_per_step = total_ms / args.steps
    log(f"[bench] graph: {args.steps} calls in {total_ms:.3f} ms -> {ms_per_step * 1e3:.2f} us/call")

    # live per-kernel durations: the library records events around each dispatch
    n_calls = min(4 * len(pools), 192)
    events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n_calls)]
    for evs in events:  # create the HIP events before their handles are passed down
        for e in evs:
            e.record(stream)
    back_to_back(torch, _lib, prepared, n_calls, events)
    attn_ms = [evs[0].elapsed_time(evs[1]) for evs in events]
    red_ms = [evs[2].elapsed_time(evs[3]) for evs in events] if splits > 1 else [0.0]
    kernel_ms = statistics.mean(attn_ms)
    log(f"[bench] attention kernel: mean {kernel_ms * 1e3:.2f} us, median {statistics.median(attn_ms) * 1e3:.2f} us"
        f"; reducer: mean {statistics.mean(red_ms) * 1e3:.2f} us ({n_calls} calls)")

    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    traffic, traffic_meta = load_traffic()
    traffic_src = None if traffic_meta is None else os.path.relpath(TRAFFIC_SUMMARY, ROOT)
    if traffic is not None:
        traffic = int(round(traffic))
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    cpu = None
    if not args.no_cpu:
        cpu_s, reps = cpu_baseline(pools, args.cpu_seconds, sm_scale)
        cpu = {
            "value": round(nbytes / cpu_s / 1e9, 4),
            "unit": "GB/s",
            "cores": 1,
            "kind": "port",
            "sample": f"numpy oracle (oracle/attention.py), full B{batch} ctx{ctx} call on pool 0, "
                      f"median of {reps} calls, {cpu_s * 1e6:.0f} us/call, one BLAS thread",
        }
        log(f"[bench] cpu oracle: {cpu_s * 1e3:.1f} ms/call over {reps} calls")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "us_per_call": round(ms_per_step * 1e3, 3),
        "hbm_frac": round(value / HBM_PEAK_GBS, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": f"paged-decode-b{batch}-ctx{ctx}-hq{hq}-hkv{hkv}-d{d}-bs{bs}",
            "batch": batch,
            "seq_len": ctx,
            "num_q_heads": hq,
            "num_kv_heads": hkv,
            "head_dim": d,
            "block_size": bs,
            "kv_pools": len(pools),
            "kv_pool_mib": round(pool_bytes / 2**20, 1),
            "num_splits": splits,
            "timing": "hipGraph of K calls replayed once; hipEvents",
            "merge": "reducer kernel" if splits > 1 else "none",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
            "kernel": "decode_mfma_kernel<bf16, bs32>",
            "kernel_us_mean": round(kernel_ms * 1e3, 3),
            "reducer_us_mean": round(statistics.mean(red_ms) * 1e3, 3),
            "algorithmic_bytes_per_call": nbytes,
            "traffic_source": traffic_src,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
