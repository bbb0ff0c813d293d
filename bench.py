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
* ``roofline.achieved``: algorithmic bytes per call / mean per-call device
  time, bracketed by HIP events on the launch stream around every call, with
  the queue pre-filled so host submission gaps are excluded.
* ``cpu_baseline``: the repo's numpy oracle (one thread) on a bounded sample
  of the same workload, on this host.

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
    p.add_argument("--merge", choices=("reducer", "in-launch"), default="reducer",
                   help="split merge: a second reducer kernel (default, the library's own choice) "
                        "or inside the decode launch (arrival counters)")
    p.add_argument("--copy-probe-mib", type=int, default=0,
                   help="also run a plain device copy of this size (PMC scaling reference)")
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


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on exactly one GPU; --gpus {args.gpus} is not supported "
            "(the decode path shards per request/KV head with no exchange; see DESIGN.md).",
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

    if args.merge == "reducer":
        def call(i):
            q, k, v, table, lens, out = pools[i % len(pools)]
            fd.paged_decode_attention_into(q, k, v, table, lens, out, sm_scale=sm_scale)
    else:
        # the in-launch merge through the unchecked launcher's counter extension
        from flashdec_amd.paged_decode import _vllm_paged_decode_attention_into as launch

        ws = (torch.empty((batch, hq, splits, d), device=dev), torch.empty((batch, hq, splits), device=dev),
              torch.empty((batch, hq, splits), device=dev))
        counters = torch.zeros(batch * hkv * _lib.SPLIT_COUNTER_STRIDE, device=dev, dtype=torch.int32)

        def call(i):
            q, k, v, table, lens, out = pools[i % len(pools)]
            _in_launch(q, k, v, table, lens, out, ws, counters)

    def _in_launch(q, k, v, table, lens, out, ws, counters):
        from flashdec_amd import paged_decode as pd

        args_ = _lib.PagedDecodeArgs()
        pd._fill_common(args_, q, k, v, pd._cache_strides(k, 2, 3), pd._cache_strides(v, 2, 3), table, lens, out,
                        hkv, bs, sm_scale)
        args_.num_blocks = k.shape[0]
        args_.max_seq_len = ctx
        pd._fill_workspace(args_, ws[0], ws[1], ws[2], splits, counters)
        _lib.paged_decode(args_, _lib.current_stream_handle(dev))

    stream = torch.cuda.current_stream(dev)
    # warmup (eager)
    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
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

    # per-call device time: events around each launch, queue pre-filled
    n_ev = min(2 * len(pools), 192)
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    stops = [torch.cuda.Event(enable_timing=True) for _ in range(n_ev)]
    torch.cuda.synchronize()
    torch.cuda._sleep(200_000_000)
    for i in range(n_ev):
        starts[i].record(stream)
        call(i)
        stops[i].record(stream)
    torch.cuda.synchronize()
    per_call_ms = [s.elapsed_time(e) for s, e in zip(starts, stops)]
    kernel_ms = statistics.mean(per_call_ms)
    kernel_med = statistics.median(per_call_ms)
    log(f"[bench] per-call events: mean {kernel_ms * 1e3:.2f} us, median {kernel_med * 1e3:.2f} us, "
        f"min {min(per_call_ms) * 1e3:.2f} us")

    if args.copy_probe_mib:
        n = args.copy_probe_mib * 2**20 // 2
        src = torch.ones(n, device=dev, dtype=torch.bfloat16)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"[bench] copy probe: {args.copy_probe_mib} MiB read + {args.copy_probe_mib} MiB written x3")

    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
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
            "merge": args.merge,
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": None,
            "per_call_us_mean": round(kernel_ms * 1e3, 3),
            "algorithmic_bytes_per_call": nbytes,
        },
        "cpu_baseline": cpu,
    }
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
