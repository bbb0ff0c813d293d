"""Paged-decode benchmark on one MI355X (the headline B8 ctx2048 decode shape).

A step is one ``paged_decode_attention_into`` call (the hot path) over one
synthetic batch: B=8 requests, Hq=16 / Hkv=2 (Qwen2.5-3B attention shape),
head_dim 128, bf16, 32-token blocks, every seq_len = 2048, block tables drawn
from a shuffled pool of 1.25x the needed blocks.  Inputs are resident in HBM
before timing starts.  Steps rotate over ``--pools`` independent KV pools
(default 48 x 21 MB ~ 1 GB) so the 256 MB Infinity Cache cannot serve them.

Timing:
* warm-up: at least ``--warmup`` calls and at least 100 ms of calls.
* ``ms_per_step``/``value``: p50 of the per-call time over 240 samples, each
  one replay of a hipGraph holding one call per pool (one rotation), replayed
  back to back with hipEvents between the replays.
* ``single_replay_ms_per_step``: K steps captured in one hipGraph, replayed
  once between two synchronisations (the serving-loop view, launch gaps
  included).
* ``roofline.achieved``: algorithmic bytes per call / mean duration of the
  dominant kernel (the attention kernel), measured live: every call of a
  separate eager loop passes HIP events through the library's
  ``timing_events`` hook, which records them around exactly that dispatch
  (and around the split reducer, reported beside it).  Events cannot bracket
  one kernel inside a captured graph; the rocprofv3 kernel trace of the
  graph replays is the cross-check.
* ``roofline.traffic``: HBM bytes per attention-kernel dispatch from the
  committed PMC summary ``profiles/decode_mfma_b8_ctx2048_traffic.json``
  (FETCH_SIZE + WRITE_SIZE scaled by a copy kernel of known size), or null
  (also for any other shape than the headline one those counters were
  taken on).
* ``ctx1024``: the same call at ctx1024 (the C2 config names both
  contexts), timed the same way on 48 pools of its own.
* ``cpu_baseline``: the reference's CPU path as fp32 torch-CPU ops in its
  per-(sequence, query-head) loop (oracle/torch_loop.py) under
  ``torch.set_num_threads`` (os.cpu_count(), capped at the box's 16-thread
  share; ``torch.get_num_threads()`` recorded), one synchronous call at a
  time; beside it the numpy oracle over worker processes, each call one
  synchronised unit between two barriers.  C1 and the C2 call at ctx1024
  and ctx2048: p50 of >= 20 calls after 3 warm-ups, with the CPU model.  It
  runs first, before this process touches the GPU.

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
    p.add_argument("--workload", choices=("decode", "c2-floor", "c2-timeline", "c4-timeline", "rope", "ragged", "prefix",
                                          "prefix-large",
                                          "prefix-sweep", "engine", "engine-prefix", "formats", "vllm",
                                          "ref-shapes"),
                   default="decode",
                   help="decode: the headline C2 call (default); c2-floor: the C2 call beside a bare read of "
                        "its bytes and a dependent empty launch (the floor of a call of that size); c2-timeline / "
                        "c4-timeline: per-wave phase stamps of the C2 attention kernel / the C4 shared-prefix "
                        "cascade kernel (measurement build); rope: C3 fused RoPE + KV append; ragged / "
                        "prefix: C4 ragged long-context and shared-prefix decode; prefix-large: 64 requests "
                        "sharing a 16384-token prefix; prefix-sweep: cascade chunk rows x prefix splits at four "
                        "shared-prefix sizes; engine: C5 36-layer step; engine-prefix: 36-layer steps "
                        "of 64 rows sharing a 16384-token prefix; formats: head_dim 64, large groups, MHA, "
                        "dim-major caches and 8-token blocks; vllm: the vLLM hook's launch at B8 ctx1024/2048, "
                        "block size 16, fused append; ref-shapes: the reference's own published benchmark "
                        "rows (Hq32/Hkv8 grouped decode, small vLLM shapes, the RoPE + append call)")
    p.add_argument("--engine-steps", type=int, default=200, help="timed steps of the engine workload")
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


def prepared_args(pool, sm_scale, block_size, num_kv_heads, ragged=False, kv_reuse=False):
    """The ctypes argument block ``paged_decode_attention_into`` builds for this pool (auto splits)."""
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    q, k, v, table, lens, out = pool
    stream = _lib.current_stream_handle(q.device)
    max_seq_len = table.shape[1] * block_size
    balance = _lib.paged_decode_balance_target(q.shape[0], num_kv_heads) if ragged else 0
    if balance:
        splits = max(2, min(balance, -(-max_seq_len // 32)))
    else:
        splits = _lib.paged_decode_plan(q.shape[0], q.shape[1], num_kv_heads, q.shape[2], max_seq_len)
    args = _lib.PagedDecodeArgs()
    pd._fill_common(args, q, k, v, pd._cache_strides(k, 2, 3), pd._cache_strides(v, 2, 3), table, lens, out,
                    num_kv_heads, block_size, sm_scale)
    args.num_blocks = k.shape[0]
    args.max_seq_len = max_seq_len
    args.balance_target = balance
    args.kv_reuse = 1 if kv_reuse else 0
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


def cpu_model():
    """The host CPU's model name (first ``model name`` of /proc/cpuinfo), or None."""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return None


def cpu_inputs(name):
    """Seeded numpy inputs of a CPU-baseline config (fp32 arrays, sm_scale, out_dtype, algorithmic bytes).

    C1 (the first benchmark config): B4 Hq8 Hkv2 D64 fp32, bs32, L ~ U{1..512} over a 128-block pool whose
    table rows are consecutive slices of a permutation, seed 61.  C2: B8 Hq16 Hkv2 D128, bs32, every
    length 2048, a 640-block pool (1.25x) with permuted tables, bf16 values (N(0,1) rounded to bf16)
    held in fp32 as the reference upcasts them, seed 20260830 + 8 + 2048.  C2-ctx1024: the same at
    length 1024 (a 320-block pool, seed 20260830 + 8 + 1024).
    """
    import numpy as np

    from oracle.rope import round_to

    if name == "C1":
        rng = np.random.default_rng(61)
        b, hq, hkv, d, bs, pool = 4, 8, 2, 64, 32, 128
        lens = rng.integers(1, 513, size=b).astype(np.int32)
        dtype = "float32"
    else:
        ctx = 1024 if name == "C2-ctx1024" else 2048
        rng = np.random.default_rng(20260830 + 8 + ctx)
        b, hq, hkv, d, bs, pool = 8, 16, 2, 128, 32, 640 * ctx // 2048
        lens = np.full(b, ctx, dtype=np.int32)
        dtype = "bfloat16"
    nblk = [(int(n) + bs - 1) // bs for n in lens]
    perm = rng.permutation(pool)
    table = np.full((b, max(nblk)), -1, dtype=np.int32)
    cursor = 0
    for row, n in enumerate(nblk):
        table[row, :n] = perm[cursor:cursor + n]
        cursor += n
    k = round_to(rng.standard_normal((pool, hkv, bs, d), dtype=np.float32), dtype)
    v = round_to(rng.standard_normal((pool, hkv, bs, d), dtype=np.float32), dtype)
    q = round_to(rng.standard_normal((b, hq, d), dtype=np.float32), dtype)
    elt = 4 if dtype == "float32" else 2
    nbytes = int(int(lens.sum()) * hkv * d * 2 * elt + 2 * q.size * elt + 4 * table.size + 4 * b)
    return (q, k, v, table, lens), 1.0 / math.sqrt(d), dtype, nbytes


_CPU_WORKER = {}
# CPU-baseline configs: (rows, KV heads) per call; a work item is one (row, KV head)
CPU_CONFIGS = {"C1": (4, 2), "C2-ctx1024": (8, 2), "C2": (8, 2)}
# host threads of the GPU box's share (its OMP_NUM_THREADS), whatever os.cpu_count() shows
CPU_THREAD_CAP = 16


def cpu_threads():
    """Threads for the CPU baseline: os.cpu_count(), capped at the box's CPU share."""
    return max(1, min(os.cpu_count() or 1, CPU_THREAD_CAP))


def cpu_baseline_torch(budget_s):
    """The reference's CPU path as fp32 torch-CPU ops (oracle/torch_loop.py, restating
    paged_reference.py:92-125: the per-(sequence, query-head) loop) under
    ``torch.set_num_threads(cpu_threads())``.  Each config's inputs are the seeded
    ``cpu_inputs`` arrays as torch tensors (bf16 for C2, as the reference's callers hold
    them); a call is one synchronous ``paged_decode_attention_loop``.  p50 of >= 20 calls
    after 3 warm-ups (more while within the budget, at most 200)."""
    import torch

    from oracle.torch_loop import paged_decode_attention_loop

    threads = cpu_threads()
    torch.set_num_threads(threads)
    results = {}
    for name in CPU_CONFIGS:
        (q, k, v, table, lens), scale, dtype, nbytes = cpu_inputs(name)
        tdt = torch.float32 if dtype == "float32" else torch.bfloat16
        args = [torch.from_numpy(x).to(tdt) for x in (q, k, v)] + [torch.from_numpy(table), torch.from_numpy(lens)]

        def call():
            paged_decode_attention_loop(*args, scale)

        for _ in range(3):
            call()
        t0 = time.perf_counter()
        call()
        probe = time.perf_counter() - t0
        reps = int(min(200, max(20, budget_s / len(CPU_CONFIGS) / max(probe, 1e-6))))
        times = []
        for _ in range(reps):
            t0 = time.perf_counter()
            call()
            times.append(time.perf_counter() - t0)
        sec = statistics.median(times)
        results[name] = {"us_per_call": round(sec * 1e6, 1), "gb_per_s": round(nbytes / sec / 1e9, 4),
                         "threads": torch.get_num_threads(), "calls": reps, "algorithmic_bytes": nbytes}
    return results, threads


def _cpu_worker_init():
    """Worker initializer: one BLAS thread, and each config's inputs built locally."""
    from threadpoolctl import threadpool_limits

    _CPU_WORKER["blas"] = threadpool_limits(limits=1)
    for name in CPU_CONFIGS:
        _CPU_WORKER[name] = cpu_inputs(name)


def _cpu_item(name, item):
    """The oracle on one (row, KV head) of a config: the row's query heads of that KV head (runs in a worker)."""
    from oracle.attention import paged_decode_attention as oracle_decode

    (q, k, v, table, lens), scale, out_dtype, _ = _CPU_WORKER[name]
    hkv = k.shape[1]
    b, h = divmod(item, hkv)
    group = q.shape[1] // hkv
    return oracle_decode(q[b:b + 1, h * group:(h + 1) * group], k[:, h:h + 1], v[:, h:h + 1], table[b:b + 1],
                         lens[b:b + 1], sm_scale=scale, out_dtype=out_dtype)


def _cpu_worker_loop(rank, workers, start, done, jobs):
    """A baseline worker: for every job (config, calls), run its share of each call between two
    barriers that every worker and the parent pass together (runs in a worker process)."""
    _cpu_worker_init()
    while True:
        job = jobs.get()
        if job is None:
            return
        name, calls = job
        n = CPU_CONFIGS[name][0] * CPU_CONFIGS[name][1]
        share = list(range(rank, n, workers))
        for _ in range(calls):
            start.wait()
            for item in share:
                _cpu_item(name, item)
            done.wait()


def cpu_baseline_numpy(budget_s):
    """The numpy oracle (oracle/attention.py) on this host's cores, one call at a time.

    A call's (row, KV head) pairs are independent: each of
    min(cpu_threads(), pairs) worker processes (one BLAS thread each) takes a
    fixed share.  Every call is one synchronised unit: the parent and all
    workers pass a start barrier, the workers run their shares, and all pass
    an end barrier; a call's time is the parent's time between the two
    barriers (barrier overhead included).  p50 of >= 20 calls after 3
    warm-ups per config.  Started before this process touches the GPU.
    """
    import multiprocessing as mp

    ctx = mp.get_context("spawn")
    workers = min(cpu_threads(), max(r * h for r, h in CPU_CONFIGS.values()))
    start, done = ctx.Barrier(workers + 1), ctx.Barrier(workers + 1)
    queues = [ctx.Queue() for _ in range(workers)]
    procs = [ctx.Process(target=_cpu_worker_loop, args=(r, workers, start, done, queues[r]), daemon=True)
             for r in range(workers)]
    for p in procs:
        p.start()
    results = {}
    try:
        for name in CPU_CONFIGS:
            nbytes = cpu_inputs(name)[3]
            # 3 warm-ups and one probe call size the sample to the budget
            for qu in queues:
                qu.put((name, 4))
            for i in range(4):
                start.wait()
                t0 = time.perf_counter()
                done.wait()
                probe = time.perf_counter() - t0
            reps = int(min(200, max(20, budget_s / len(CPU_CONFIGS) / max(probe, 1e-6))))
            for qu in queues:
                qu.put((name, reps))
            times = []
            for _ in range(reps):
                start.wait()
                t0 = time.perf_counter()
                done.wait()
                times.append(time.perf_counter() - t0)
            sec = statistics.median(times)
            used = min(workers, CPU_CONFIGS[name][0] * CPU_CONFIGS[name][1])
            results[name] = {"us_per_call": round(sec * 1e6, 1), "gb_per_s": round(nbytes / sec / 1e9, 4),
                             "processes": workers, "busy_processes": used, "calls": reps,
                             "algorithmic_bytes": nbytes}
    finally:
        for qu in queues:
            qu.put(None)
        for p in procs:
            p.join(timeout=10)
    return results


def cpu_baseline(budget_s):
    """Both CPU baselines (reported, not targets): the torch-CPU loop form of the reference's
    path (the primary figure) and the numpy oracle spread over worker processes."""
    numpy_res = cpu_baseline_numpy(budget_s / 2)
    torch_res, threads = cpu_baseline_torch(budget_s / 2)
    return torch_res, numpy_res, threads


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


def graph_ms_per_call(torch, dev, fn, n_calls, warmup=8):
    """Mean ms per call of ``fn(i)`` for ``n_calls`` calls captured in one hipGraph, replayed once."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fn(0)  # per-stream workspaces exist before capture
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for i in range(n_calls):
                fn(i)
    torch.cuda.current_stream(dev).wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    graph.replay()
    stop.record()
    torch.cuda.synchronize()
    return start.elapsed_time(stop) / n_calls


def graph_p50_us(torch, dev, fn, n_calls, samples=240, warmup=96):
    """p50 us per call of ``fn(i)``: one hipGraph holding ``n_calls`` calls (one per pool),
    replayed ``samples`` times back to back with hipEvents between the replays."""
    for i in range(warmup):
        fn(i)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        fn(0)  # per-stream workspaces exist before capture
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for i in range(n_calls):
                fn(i)
    torch.cuda.current_stream(dev).wait_stream(side)
    graph.replay()
    torch.cuda.synchronize()
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(samples + 1)]
    marks[0].record()
    for i in range(samples):
        graph.replay()
        marks[i + 1].record()
    torch.cuda.synchronize()
    per = sorted(marks[i].elapsed_time(marks[i + 1]) / n_calls * 1e3 for i in range(samples))
    return statistics.median(per)


def attention_kernel_us(torch, prepared, n_calls):
    """Mean attention-kernel and reducer durations (us) through the library's timing hook."""
    from flashdec_amd import _lib

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n_calls)]
    for evs in events:
        for e in evs:
            e.record()
    back_to_back(torch, _lib, prepared, n_calls, events)
    attn = statistics.mean(e[0].elapsed_time(e[1]) for e in events) * 1e3
    has_reducer = prepared[0][0].num_splits > 1
    red = statistics.mean(e[2].elapsed_time(e[3]) for e in events) * 1e3 if has_reducer else 0.0
    return attn, red


def common_fields(args, metric, value, unit, ms_per_step, higher_is_better, config, dtype="bf16"):
    return {"metric": metric, "value": value, "unit": unit, "n_gpus": 1, "steps": args.steps,
            "warmup": args.warmup, "ms_per_step": round(ms_per_step, 6), "higher_is_better": higher_is_better,
            "scaling": "weak", "vs_baseline": None, "dtype": dtype, "data": "synthetic", "config": config}


def run_rope(torch, dev, args):
    """C3: fused RoPE + paged K/V append, B64 Hq16 Hkv2 D128 bf16, theta 1e6, pos ~ U{1..8191}."""
    from flashdec_amd._fused_rope_kv_append import _fused_rope_kv_append_trusted

    batch, hq, hkv, d, bs = 64, 16, 2, 128, 32
    gen = torch.Generator(device=dev)
    gen.manual_seed(251)
    blocks = batch * 256
    kc = torch.zeros((blocks, hkv, bs, d), device=dev, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    table = torch.randperm(blocks, device=dev, generator=gen).view(batch, 256)
    pos = torch.randint(1, 8192, (batch,), device=dev, generator=gen)
    blk = table.gather(1, (pos // bs).unsqueeze(1)).squeeze(1).contiguous()
    off = (pos % bs).contiguous()
    calls = []
    for i in range(4):
        q = torch.randn((batch, hq, d), device=dev, generator=gen).to(torch.bfloat16)
        k = torch.randn((batch, hkv, d), device=dev, generator=gen).to(torch.bfloat16)
        v = torch.randn((batch, hkv, d), device=dev, generator=gen).to(torch.bfloat16)
        calls.append((q, k, v, torch.empty_like(q)))

    def fn(i):
        q, k, v, qo = calls[i % len(calls)]
        _fused_rope_kv_append_trusted(q, k, v, kc, vc, blk, off, pos, base=1e6, q_out=qo)

    ms = graph_ms_per_call(torch, dev, fn, args.steps)
    # the same launch reading cos/sin from a table (what the cache and the
    # engine pass by default: apply_rope's bits), 8192 rows
    from flashdec_amd.rope import rope_cos_sin_table

    tab = rope_cos_sin_table(8192, d, 1e6, device=dev)

    def fn_table(i):
        q, k, v, qo = calls[i % len(calls)]
        _fused_rope_kv_append_trusted(q, k, v, kc, vc, blk, off, pos, base=1e6, q_out=qo, cos_sin_table=tab)

    ms_t = graph_ms_per_call(torch, dev, fn_table, args.steps)
    nbytes = batch * (2 * hq + 3 * hkv) * d * 2 + 24 * batch
    log(f"[bench] rope+append: {ms * 1e3:.2f} us/call (cos/sin evaluated), {ms_t * 1e3:.2f} us/call (cos/sin table), "
        f"{nbytes} B/call")
    out = common_fields(args, "fused RoPE + KV append us/call, B64 Hq16 Hkv2 D128 bf16 (C3)", round(ms * 1e3, 3),
                        "us", ms, False, {"workload": "rope-kv-append-b64-hq16-hkv2-d128-bs32", "batch": batch,
                                          "rope_theta": 1e6, "positions": "U{1..8191} seed 251"})
    out["roofline"] = {"bound": "launch", "algorithmic_bytes_per_call": nbytes,
                       "achieved": round(nbytes / (ms * 1e-3) / 1e9, 2), "unit": "GB/s", "peak": HBM_PEAK_GBS}
    out["cos_sin_table"] = {"us_per_call": round(ms_t * 1e3, 3), "rows": 8192,
                            "note": "the default of PagedKVCache / DecodeEngine launches (bit-exact to apply_rope)"}
    return out


def ragged_lengths(n, seed):
    import numpy as np

    rng = np.random.default_rng(seed)
    return [int(round(math.exp(x))) for x in rng.uniform(math.log(128), math.log(32768), size=n)]


def decode_pools(torch, dev, lens, hq, hkv, d, bs, n_pools, seed, prefix_blocks=0, dtype=None):
    """Independent (q, k, v, table, lens, out) sets; the first ``prefix_blocks`` of every row are shared.
    bf16 unless ``dtype`` names another cache dtype."""
    dtype = torch.bfloat16 if dtype is None else dtype
    nblk = [(n + bs - 1) // bs for n in lens]
    private = [max(0, b - prefix_blocks) for b in nblk]
    pool_blocks = int(math.ceil((prefix_blocks + sum(private)) * 1.25)) + 1
    width = max(nblk)
    pools = []
    gen = torch.Generator(device=dev)
    for i in range(n_pools):
        gen.manual_seed(seed + i)
        k = torch.empty((pool_blocks, hkv, bs, d), device=dev, dtype=dtype).normal_(generator=gen)
        v = torch.empty_like(k).normal_(generator=gen)
        q = torch.randn((len(lens), hq, d), device=dev, generator=gen).to(dtype)
        perm = torch.randperm(pool_blocks, device=dev, generator=gen).to(torch.int32)
        table = torch.full((len(lens), width), -1, device=dev, dtype=torch.int32)
        shared = perm[:prefix_blocks]
        cursor = prefix_blocks
        for b, nb in enumerate(nblk):
            table[b, :prefix_blocks] = shared
            table[b, prefix_blocks:nb] = perm[cursor:cursor + private[b]]
            cursor += private[b]
        pools.append((q, k, v, table, torch.tensor(lens, device=dev, dtype=torch.int32), torch.empty_like(q)))
    return pools


def cascade_prepared(torch, pool, groups, sm_scale, block_size, num_kv_heads):
    """The ctypes argument blocks ``paged_decode_attention_cascade_into`` builds for this pool."""
    from flashdec_amd import _lib, cascade
    from flashdec_amd import paged_decode as pd

    q, k, v, table, lens, out = pool
    stream = _lib.current_stream_handle(q.device)
    chunk_rows = cascade.plan_chunk_rows(groups, q.shape[1], num_kv_heads)
    chunks = cascade.prefix_chunks(groups, q.shape[1], num_kv_heads, chunk_rows)
    psplits, splits = cascade.plan_cascade_splits(q.shape[0], q.shape[1], num_kv_heads, q.shape[2], groups, chunks,
                                                  cascade._num_cus(q.device))
    acc, mx, sm, _ = pd._auto_workspace(q, num_kv_heads, splits + psplits, stream)
    args = _lib.PagedDecodeArgs()
    pd._fill_common(args, q, k, v, pd._cache_strides(k, 2, 3), pd._cache_strides(v, 2, 3), table, lens, out,
                    num_kv_heads, block_size, sm_scale)
    args.num_blocks = k.shape[0]
    args.max_seq_len = groups.max_prefix_len + groups.max_tail_len
    args.kv_reuse = 1  # the cascade's default: plain loads
    pd._fill_workspace(args, acc, mx, sm, splits)
    args.split_acc, args.split_max, args.split_sum = acc.data_ptr(), mx.data_ptr(), sm.data_ptr()
    args.split_acc_stride[:] = acc.stride()
    args.split_stats_stride[:] = mx.stride()
    cas = _lib.CascadeArgs()
    cas.num_groups, cas.max_members, cas.prefix_splits = groups.num_groups, groups.max_members, psplits
    cas.group_members = groups.members.data_ptr()
    cas.group_prefix_len = groups.prefix_len.data_ptr()
    cas.row_prefix_len = groups.row_prefix_len.data_ptr()
    cas.max_prefix_len = groups.max_prefix_len
    cas.chunk_rows = chunk_rows
    return args, cas, stream


def cascade_kernel_us(torch, prepared, n_calls):
    """Mean (prefix + tail pass) and reducer durations (us) of cascade calls, through the timing hook."""
    from flashdec_amd import _lib

    events = [[torch.cuda.Event(enable_timing=True) for _ in range(4)] for _ in range(n_calls)]
    for evs in events:
        for e in evs:
            e.record()
    torch.cuda.synchronize()
    torch.cuda._sleep(200_000_000)
    for i in range(n_calls):
        a, cas, st = prepared[i % len(prepared)]
        a.timing_events[:] = [e.cuda_event for e in events[i]]
        _lib.paged_decode_cascade(a, cas, st)
        a.timing_events[:] = [None] * 4
    torch.cuda.synchronize()
    attn = statistics.mean(e[0].elapsed_time(e[1]) for e in events) * 1e3
    red = statistics.mean(e[2].elapsed_time(e[3]) for e in events) * 1e3
    return attn, red


def run_decode_variant(torch, dev, args, name, lens, n_pools, seed, prefix_blocks=0, ragged=False):
    import flashdec_amd as fd

    hq, hkv, d, bs = 16, 2, 128, 32
    sm_scale = 1.0 / math.sqrt(d)
    pools = decode_pools(torch, dev, lens, hq, hkv, d, bs, n_pools, seed, prefix_blocks)
    # rows sharing a prefix: the per-row path reads K/V with plain, cached
    # loads (kv_reuse), as a caller that knows its tables share blocks would
    reuse = prefix_blocks > 0

    def fn(i):
        q, k, v, table, sl, out = pools[i % len(pools)]
        fd.paged_decode_attention_into(q, k, v, table, sl, out, sm_scale=sm_scale, kv_reuse=reuse)

    ms = graph_ms_per_call(torch, dev, fn, args.steps)
    prepared = [prepared_args(p, sm_scale, bs, hkv, kv_reuse=reuse) for p in pools]
    attn_us, red_us = attention_kernel_us(torch, prepared, min(4 * len(pools), 96))
    nblk = max((n + bs - 1) // bs for n in lens)
    table_q = 4 * len(lens) * nblk + 4 * len(lens) + 2 * len(lens) * hq * d * 2
    logical = sum(lens) * hkv * d * 2 * 2 + table_q
    unique_tokens = prefix_blocks * bs + sum(max(0, n - prefix_blocks * bs) for n in lens)
    unique = unique_tokens * hkv * d * 2 * 2 + table_q
    splits = prepared[0][0].num_splits
    log(f"[bench] {name}: {ms * 1e3:.2f} us/call (graph); attention kernel {attn_us:.2f} us, reducer {red_us:.2f} us;"
        f" splits {splits}; logical {logical} B, unique {unique} B")
    out = common_fields(args, f"paged-decode us/call + achieved HBM GB/s, {name}", round(unique / (ms * 1e-3) / 1e9, 2),
                        "GB/s", ms, True,
                        {"workload": name, "batch": len(lens), "num_q_heads": hq, "num_kv_heads": hkv, "head_dim": d,
                         "block_size": bs, "seq_lens_sum": sum(lens), "seq_len_max": max(lens),
                         "prefix_blocks": prefix_blocks, "kv_pools": n_pools, "num_splits": splits,
                         "kv_loads": "plain (kv_reuse)" if reuse else "non-temporal"})
    out["us_per_call"] = round(ms * 1e3, 3)
    out["roofline"] = {"bound": "hbm", "achieved": round(unique / (attn_us * 1e-6) / 1e9, 2), "peak": HBM_PEAK_GBS,
                       "unit": "GB/s", "frac": round(unique / (attn_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
                       "traffic": None, "kernel_us_mean": round(attn_us, 3), "reducer_us_mean": round(red_us, 3),
                       "algorithmic_bytes_per_call": unique, "logical_bytes_per_call": logical}
    if ragged:
        # the same pools with per-row split counts (ragged=True); the line's
        # value is the faster of the two
        def fn_ragged(i):
            q, k, v, table, sl, o = pools[i % len(pools)]
            fd.paged_decode_attention_into(q, k, v, table, sl, o, sm_scale=sm_scale, ragged=True)

        ms_r = graph_ms_per_call(torch, dev, fn_ragged, args.steps)
        prepared_r = [prepared_args(p, sm_scale, bs, hkv, ragged=True) for p in pools]
        attn_r, red_r = attention_kernel_us(torch, prepared_r, min(4 * len(pools), 96))
        log(f"[bench] {name} ragged=True: {ms_r * 1e3:.2f} us/call (graph); attention kernel {attn_r:.2f} us, "
            f"reducer {red_r:.2f} us; balance target {prepared_r[0][0].balance_target}, "
            f"splits <= {prepared_r[0][0].num_splits}")
        balanced = {"us_per_call": round(ms_r * 1e3, 3), "value": round(unique / (ms_r * 1e-3) / 1e9, 2),
                    "balance_target": prepared_r[0][0].balance_target, "num_splits": prepared_r[0][0].num_splits,
                    "roofline": {"bound": "hbm", "achieved": round(unique / (attn_r * 1e-6) / 1e9, 2),
                                 "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": round(unique / (attn_r * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                                 "kernel_us_mean": round(attn_r, 3), "reducer_us_mean": round(red_r, 3),
                                 "algorithmic_bytes_per_call": unique, "logical_bytes_per_call": logical}}
        if ms_r < ms:
            uniform = {k: out[k] for k in ("us_per_call", "value", "roofline")}
            uniform["num_splits"] = out["config"]["num_splits"]
            out.update({k: balanced[k] for k in ("us_per_call", "value", "roofline")})
            out["ms_per_step"] = round(ms_r, 6)
            out["config"].update(splits="per-row (ragged=True)", balance_target=balanced["balance_target"],
                                 num_splits=balanced["num_splits"])
            out["uniform_splits_path"] = uniform
        else:
            out["config"]["splits"] = "uniform"
            out["per_row_splits_path"] = balanced
    if prefix_blocks == 0:
        return out
    # the same pools through the cascade (prefix read once per group): the
    # line reports it, with the per-row path beside it
    from flashdec_amd import cascade

    groups = [cascade.build_cascade_groups(p[3], p[4], bs, hq, hkv) for p in pools]
    assert all(g.num_groups == 1 and g.max_prefix_len == prefix_blocks * bs for g in groups)

    def fn_cascade(i):
        q, k, v, table, sl, o = pools[i % len(pools)]
        cascade.paged_decode_attention_cascade_into(q, k, v, table, sl, o, groups[i % len(pools)], sm_scale=sm_scale)

    ms_c = graph_ms_per_call(torch, dev, fn_cascade, args.steps)
    prepared_c = [cascade_prepared(torch, p, g, sm_scale, bs, hkv) for p, g in zip(pools, groups)]
    attn_c, red_c = cascade_kernel_us(torch, prepared_c, min(4 * len(pools), 96))
    log(f"[bench] {name} cascade: {ms_c * 1e3:.2f} us/call (graph); prefix + tail passes {attn_c:.2f} us, reducer "
        f"{red_c:.2f} us; tail splits {prepared_c[0][0].num_splits}, prefix splits {prepared_c[0][1].prefix_splits}, "
        f"chunk rows {prepared_c[0][1].chunk_rows}")
    cascade_line = {"us_per_call": round(ms_c * 1e3, 3), "value": round(unique / (ms_c * 1e-3) / 1e9, 2),
                    "num_splits": prepared_c[0][0].num_splits, "prefix_splits": prepared_c[0][1].prefix_splits,
                    "chunk_rows": prepared_c[0][1].chunk_rows,
                    "roofline": {"bound": "hbm", "achieved": round(unique / (attn_c * 1e-6) / 1e9, 2),
                                 "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                 "frac": round(unique / (attn_c * 1e-6) / 1e9 / HBM_PEAK_GBS, 4), "traffic": None,
                                 "kernel_us_mean": round(attn_c, 3), "reducer_us_mean": round(red_c, 3),
                                 "algorithmic_bytes_per_call": unique, "logical_bytes_per_call": logical}}
    # the line's value is the faster of the two paths; the other rides along
    if ms_c < ms:
        per_row = {k: out[k] for k in ("us_per_call", "value", "roofline")}
        per_row["num_splits"] = out["config"]["num_splits"]
        out.update({k: cascade_line[k] for k in ("us_per_call", "value", "roofline")})
        out["ms_per_step"] = round(ms_c, 6)
        out["config"].update(path="cascade", num_splits=cascade_line["num_splits"],
                             prefix_splits=cascade_line["prefix_splits"], chunk_rows=cascade_line["chunk_rows"])
        out["per_row_path"] = per_row
    else:
        out["config"]["path"] = "per-row"
        out["cascade_path"] = cascade_line
    return out


def load_probes():
    """``libflashdec_probe.so`` (csrc/floor_probe.hip): the floor workload's probe kernels."""
    import ctypes

    from flashdec_amd import _build

    path = _build.PROBE_LIB_PATH
    if not path.exists():
        raise RuntimeError(f"{path} is not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(str(path))
    vp, u64 = ctypes.c_void_p, ctypes.c_uint64
    lib.fdp_stream_read.argtypes = [vp, u64, vp, vp, vp, vp]
    lib.fdp_empty.argtypes = [ctypes.c_uint, ctypes.c_uint, vp]
    lib.fdp_xcc_map.argtypes = [vp, ctypes.c_uint, vp]
    i32, i64 = ctypes.c_int, ctypes.c_int64
    lib.fdp_paged_read.argtypes = [vp, i32, i32, i32, i32, vp, vp, i64, i64, vp, vp, vp, vp, vp, vp]
    lib.fdp_reduce_read.argtypes = [vp, vp, vp, i32, i32, vp, vp]
    for f in (lib.fdp_stream_read, lib.fdp_empty, lib.fdp_xcc_map, lib.fdp_paged_read, lib.fdp_reduce_read):
        f.restype = ctypes.c_int
    return lib


def run_c2_floor(torch, dev, args):
    """What a C2 call costs against what a call of its bytes costs with no attention work.

    For ctx 2048 and 1024 (B8 Hq16 Hkv2 D128 bs32 bf16, the headline pools),
    every term is a p50 over 240 replays of a hipGraph of one call per pool
    (48 pools or 48 buffers of the call's algorithmic bytes, so the Infinity
    Cache serves none of them):
      read        -- one non-temporal read of the call's bytes (fdp_stream_read);
      read+empty  -- that read, then a dependent empty kernel of the reducer's
                     grid (B*Hq workgroups of 64 threads): two dependent
                     launches with no work beyond the read;
      paged_read  -- the attention kernel's memory pattern without its
                     arithmetic (fdp_paged_read): its grid, each wave's
                     block-table entry then its K/V unit, the waves combined
                     through LDS, one partial per (query head, split) stored;
      paged_read+reduce_read
                  -- then the reducer's memory pattern (fdp_reduce_read):
                     every split's partials and statistics loaded up front, a
                     weighted sum, the output row stored.  The floor of a
                     two-launch split-KV paged call of this shape;
      shipped     -- paged_decode_attention_into: attention + reducer kernel;
      merge       -- the opt-in single-dispatch path (split_counters: the last
                     workgroup of each (request, KV head) merges);
    plus eager kernel durations (HIP events around each dispatch) of the bare
    read, the paged read, the attention kernel and the reducer, and the
    workgroup -> XCD map of a 256-workgroup grid (the in-launch merge reads
    same-XCD partials from L2).
    """
    import flashdec_amd as fd
    from flashdec_amd import _lib
    from flashdec_amd import paged_decode as pd

    probes = load_probes()
    batch, hq, hkv, d, bs = 8, 16, 2, 128, 32
    sm_scale = 1.0 / math.sqrt(d)
    res = {}
    xmap = torch.zeros(256, dtype=torch.int32, device=dev)
    stream0 = torch.cuda.current_stream(dev).cuda_stream
    assert probes.fdp_xcc_map(xmap.data_ptr(), 256, stream0) == 0
    torch.cuda.synchronize()
    xcc = xmap.cpu().tolist()
    for ctx in (2048, 1024):
        pools = build_pools(torch, args.pools, batch, ctx, hq, hkv, d, bs, dev)
        nbytes = algorithmic_bytes(batch, ctx, hq, hkv, d, bs)
        n16 = (nbytes + 15) // 16 * 16
        bufs = [torch.randint(0, 255, (n16,), dtype=torch.uint8, device=dev) for _ in range(args.pools)]
        sink = torch.zeros(256, dtype=torch.int32, device=dev)

        def rd(i, events=(None, None)):
            st = torch.cuda.current_stream(dev).cuda_stream
            assert probes.fdp_stream_read(bufs[i % len(bufs)].data_ptr(), n16, sink.data_ptr(), st, *events) == 0

        def rd_empty(i):
            rd(i)
            assert probes.fdp_empty(batch * hq, 64, torch.cuda.current_stream(dev).cuda_stream) == 0

        def shipped(i):
            q, k, v, table, lens, out = pools[i % len(pools)]
            fd.paged_decode_attention_into(q, k, v, table, lens, out, sm_scale=sm_scale)

        splits = _lib.paged_decode_plan(batch, hq, hkv, d, pools[0][3].shape[1] * bs)
        probe_ws = (torch.empty((batch * hq, splits, d), device=dev), torch.empty((batch * hq, splits), device=dev),
                    torch.empty((batch * hq, splits), device=dev))

        def paged_read(i, events=(None, None)):
            q, k, v, table, lens, out = pools[i % len(pools)]
            st = torch.cuda.current_stream(dev).cuda_stream
            assert probes.fdp_paged_read(table.data_ptr(), table.shape[1], batch, hkv, splits, k.data_ptr(),
                                         v.data_ptr(), k.stride(0) * 2, k.stride(1) * 2,
                                         *(t.data_ptr() for t in probe_ws), st, *events) == 0

        def paged_reduce(i):
            paged_read(i)
            out = pools[i % len(pools)][5]
            assert probes.fdp_reduce_read(*(t.data_ptr() for t in probe_ws), batch * hq, splits, out.data_ptr(),
                                          torch.cuda.current_stream(dev).cuda_stream) == 0
        ws = (torch.empty((batch, hq, splits, d), device=dev), torch.empty((batch, hq, splits), device=dev),
              torch.empty((batch, hq, splits), device=dev))
        counters = torch.zeros(batch * hkv * _lib.SPLIT_COUNTER_STRIDE, device=dev, dtype=torch.int32)

        def merge(i):
            q, k, v, table, lens, out = pools[i % len(pools)]
            pd._decode_with_workspace(q, k, v, table, lens, out, sm_scale, bs, splits, ws, k.shape[0],
                                      counters=counters)

        n = len(pools)
        terms = {name: round(graph_p50_us(torch, dev, fn, n), 3)
                 for name, fn in (("read", rd), ("read+empty", rd_empty), ("paged_read", paged_read),
                                  ("paged_read+reduce_read", paged_reduce), ("shipped", shipped), ("merge", merge))}
        # eager durations: HIP events recorded around exactly each bare-read
        # dispatch (hipExtLaunchKernel), the reads back to back behind a sleep
        evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(2 * n)]
        for a, b in evs:  # create the HIP events before their handles are passed down
            a.record()
            b.record()
        torch.cuda.synchronize()
        torch.cuda._sleep(100_000_000)
        for i, (a, b) in enumerate(evs):
            rd(i, (a.cuda_event, b.cuda_event))
        torch.cuda.synchronize()
        read_kernel = statistics.mean(a.elapsed_time(b) for a, b in evs) * 1e3
        torch.cuda._sleep(100_000_000)
        for i, (a, b) in enumerate(evs):
            paged_read(i, (a.cuda_event, b.cuda_event))
        torch.cuda.synchronize()
        paged_kernel = statistics.mean(a.elapsed_time(b) for a, b in evs) * 1e3
        shipped(0)
        prepared = [prepared_args(pool, sm_scale, bs, hkv) for pool in pools]
        attn_us, red_us = attention_kernel_us(torch, prepared, min(4 * n, 192))
        floor = {
            "us_per_call": terms,
            "eager_kernel_us": {"read": round(read_kernel, 3), "paged_read": round(paged_kernel, 3),
                                "attention": round(attn_us, 3), "reducer": round(red_us, 3)},
            "dependent_launch_us": round(terms["read+empty"] - terms["read"], 3),
            "shipped_over_two_launch_floor_us": round(terms["shipped"] - terms["read+empty"], 3),
            "shipped_over_paged_floor_us": round(terms["shipped"] - terms["paged_read+reduce_read"], 3),
            "hbm_frac": {k: round(nbytes / (v * 1e-6) / 1e9 / HBM_PEAK_GBS, 4) for k, v in terms.items()},
            "algorithmic_bytes": nbytes,
            "num_splits": splits,
        }
        log(f"[bench] c2-floor ctx{ctx}: " + ", ".join(f"{k} {v:.2f}" for k, v in terms.items())
            + f" us/call; eager read {read_kernel:.2f}, paged read {paged_kernel:.2f}, attention {attn_us:.2f},"
            + f" reducer {red_us:.2f} us")
        res[f"ctx{ctx}"] = floor
        del pools, bufs
        torch.cuda.empty_cache()
    c2 = res["ctx2048"]
    out = common_fields(args, "C2 call vs the floor of a call of its bytes (us/call)", c2["us_per_call"]["shipped"],
                        "us/call", c2["us_per_call"]["shipped"] * 1e-3, False,
                        {"workload": "c2-floor-b8-hq16-hkv2-d128-bs32", "kv_pools": args.pools})
    out.update(res)
    out["xcd_of_workgroup"] = {"grid": 256, "round_robin": all(x == i % 8 for i, x in enumerate(xcc)),
                               "first16": xcc[:16]}
    return out


TIMELINE_PHASES = ("wave start", "block-table entry arrived", "K/V loads issued", "K landed, QK done", "softmax done",
                   "PV issued", "units done", "wave-merge barrier passed", "partials issued", "partials acknowledged")


def timeline_reader():
    """(read, clear) for the measurement build's per-wave stamp array: read()
    copies it to the host as uint64 [workgroups, 8 waves, 16 slots]."""
    import ctypes

    import numpy as np

    from flashdec_amd import _lib

    lib = _lib.load_library()
    if not hasattr(lib, "fd_timeline_buffer"):
        raise RuntimeError("the timeline workloads need libflashdec_timeline.so (FLASHDEC_AMD_LIB points elsewhere)")
    lib.fd_timeline_buffer.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.POINTER(ctypes.c_uint64)]
    lib.fd_timeline_buffer.restype = ctypes.c_int
    ptr, nbytes = ctypes.c_void_p(), ctypes.c_uint64()
    assert lib.fd_timeline_buffer(ctypes.byref(ptr), ctypes.byref(nbytes)) == 0
    hip = ctypes.CDLL("libamdhip64.so")
    hip.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
    hip.hipMemcpy.restype = ctypes.c_int
    hip.hipMemset.argtypes = [ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t]
    hip.hipMemset.restype = ctypes.c_int
    host = np.zeros(nbytes.value // 8, dtype=np.uint64)

    def read():
        assert hip.hipMemcpy(host.ctypes.data, ptr.value, host.nbytes, 2) == 0  # device to host
        return host.reshape(-1, 8, 16).copy()

    def clear():
        assert hip.hipMemset(ptr.value, 0, host.nbytes) == 0

    return read, clear


def run_c2_timeline(torch, dev, args):
    """Per-wave timeline of the C2 attention kernel, from libflashdec_timeline.so.

    That library is the decode library built with -DFD_TIMELINE: lane 0 of
    every wave of the MFMA row kernel writes s_memrealtime (100 MHz) at ten
    phase boundaries (TIMELINE_PHASES) into a device array.  For ctx 2048
    and 1024 on the headline pools, a graph of one call per pool is replayed
    30 times; after each replay the last call's stamps are read back.  Every
    stamp is reported relative to the earliest wave start of its call:
    p10 / median / p90 / max over the 30 calls' waves, and the median time of
    each phase.  The stamps' own stores and waits perturb the kernel slightly:
    the graph's per-call time with them is reported beside the figures.
    """
    import numpy as np

    import flashdec_amd as fd
    from flashdec_amd import _lib

    read, _ = timeline_reader()
    batch, hq, hkv, d, bs = 8, 16, 2, 128, 32
    sm_scale = 1.0 / math.sqrt(d)
    res = {}
    for ctx in (2048, 1024):
        pools = build_pools(torch, args.pools, batch, ctx, hq, hkv, d, bs, dev)
        splits = _lib.paged_decode_plan(batch, hq, hkv, d, ctx)
        grid = batch * hkv * splits

        def call(i):
            q, k, v, table, lens, out = pools[i % len(pools)]
            fd.paged_decode_attention_into(q, k, v, table, lens, out, sm_scale=sm_scale)

        us_call = graph_p50_us(torch, dev, call, len(pools), samples=60)
        graph = torch.cuda.CUDAGraph()
        side = torch.cuda.Stream(dev)
        side.wait_stream(torch.cuda.current_stream(dev))
        with torch.cuda.stream(side):
            call(0)
            side.synchronize()
            with torch.cuda.graph(graph, stream=side):
                for i in range(len(pools)):
                    call(i)
        torch.cuda.current_stream(dev).wait_stream(side)
        rel = []
        for _ in range(30):
            graph.replay()
            torch.cuda.synchronize()
            st = read()[:grid, :4, : len(TIMELINE_PHASES)].reshape(grid * 4, -1).astype(np.int64)
            rel.append((st - st[:, 0].min()) * 10)  # ns
        rel = np.concatenate(rel)
        phases = {}
        for k, name in enumerate(TIMELINE_PHASES):
            col = rel[:, k]
            phases[name] = {"p10": float(np.percentile(col, 10)), "median": float(np.median(col)),
                            "p90": float(np.percentile(col, 90)), "max": float(col.max())}
        steps = {f"{TIMELINE_PHASES[k]} -> {TIMELINE_PHASES[k + 1]}": float(np.median(rel[:, k + 1] - rel[:, k]))
                 for k in range(len(TIMELINE_PHASES) - 1)}
        log(f"[bench] c2-timeline ctx{ctx} ({grid * 4} waves x 30 calls; instrumented call {us_call:.2f} us):")
        for name, v in phases.items():
            log(f"[bench]   {name:28s} p10 {v['p10']:6.0f}  median {v['median']:6.0f}  p90 {v['p90']:6.0f}  "
                f"max {v['max']:6.0f} ns")
        res[f"ctx{ctx}"] = {"instrumented_us_per_call": round(us_call, 3), "stamps_ns": phases,
                            "median_phase_ns": steps, "waves": grid * 4, "calls": 30}
        del pools
        torch.cuda.empty_cache()
    c2 = res["ctx2048"]
    out = common_fields(args, "C2 attention kernel: median wave end after the first wave start (ns)",
                        c2["stamps_ns"]["partials acknowledged"]["median"], "ns",
                        c2["instrumented_us_per_call"] * 1e-3, False,
                        {"workload": "c2-timeline-b8-hq16-hkv2-d128-bs32", "kv_pools": args.pools})
    out.update(res)
    return out


def run_c4_timeline(torch, dev, args):
    """Per-wave timeline of the C4 shared-prefix cascade kernel, from libflashdec_timeline.so.

    The C4 prefix workload's pools (16 requests on one 4096-token prefix,
    tails U{1..512}, seed 1701, 40 pools) through the cascade call; a graph of
    one call per pool is replayed 30 times, the stamp array cleared before
    each replay and read after it (the last call's stamps).  Every wave of the
    cascade kernel writes the phase stamps of the C2 timeline, the end of each
    of its 16-token units, and its role.  Reported per role (prefix, tail), in
    ns after the call's first wave start: p10 / median / p90 / max of every
    phase and unit end over the 30 calls' waves; the instrumented call's time
    beside them.
    """
    import numpy as np

    from flashdec_amd import cascade

    read, clear = timeline_reader()
    hq, hkv, d, bs = 16, 2, 128, 32
    sm_scale = 1.0 / math.sqrt(d)
    tails = np.random.default_rng(1701).integers(1, 513, size=16)
    lens = [4096 + int(t) for t in tails]
    pools = decode_pools(torch, dev, lens, hq, hkv, d, bs, 40, 1701, prefix_blocks=128)
    groups = [cascade.build_cascade_groups(p[3], p[4], bs, hq, hkv) for p in pools]

    def call(i):
        q, k, v, table, sl, o = pools[i % len(pools)]
        cascade.paged_decode_attention_cascade_into(q, k, v, table, sl, o, groups[i % len(pools)], sm_scale=sm_scale)

    us_call = graph_p50_us(torch, dev, call, len(pools), samples=60)
    prep = cascade_prepared(torch, pools[0], groups[0], sm_scale, bs, hkv)
    graph = torch.cuda.CUDAGraph()
    side = torch.cuda.Stream(dev)
    side.wait_stream(torch.cuda.current_stream(dev))
    with torch.cuda.stream(side):
        call(0)
        side.synchronize()
        with torch.cuda.graph(graph, stream=side):
            for i in range(len(pools)):
                call(i)
    torch.cuda.current_stream(dev).wait_stream(side)
    names = TIMELINE_PHASES + tuple(f"unit {u} done" for u in range(4)) + ("unit 4+ done",)
    per_role = {1: [], 2: []}
    for _ in range(30):
        torch.cuda.synchronize()
        clear()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        st = read()
        role = st[:, :, 15]
        live = role > 0
        t0 = st[:, :, 0][live].astype(np.int64).min()
        rel = (st[:, :, :15].astype(np.int64) - t0) * 10  # ns
        rel[st[:, :, :15] == 0] = -1  # phase not reached (units past the wave's last)
        for r in (1, 2):
            per_role[r].append(rel[role == r])
    res = {}
    for r, label in ((1, "prefix"), (2, "tail")):
        rel = np.concatenate(per_role[r])
        phases = {}
        for k, name in enumerate(names):
            col = rel[:, k][rel[:, k] >= 0]
            if col.size == 0:
                continue
            phases[name] = {"waves": int(col.size), "p10": float(np.percentile(col, 10)),
                            "median": float(np.median(col)), "p90": float(np.percentile(col, 90)),
                            "max": float(col.max())}
        log(f"[bench] c4-timeline {label} role ({rel.shape[0] // 30} waves x 30 calls; instrumented call "
            f"{us_call:.2f} us):")
        for name, v in phases.items():
            log(f"[bench]   {name:28s} p10 {v['p10']:6.0f}  median {v['median']:6.0f}  p90 {v['p90']:6.0f}  "
                f"max {v['max']:6.0f} ns  ({v['waves'] // 30} waves)")
        res[label] = {"waves": rel.shape[0] // 30, "stamps_ns": phases}
    out = common_fields(args, "C4 shared-prefix cascade kernel: median prefix-role wave end after the first wave "
                        "start (ns)", res["prefix"]["stamps_ns"]["partials acknowledged"]["median"], "ns",
                        us_call * 1e-3, False,
                        {"workload": "c4-timeline-shared-prefix-16x4096+U512", "kv_pools": len(pools),
                         "tail_splits": prep[0].num_splits, "prefix_splits": prep[1].prefix_splits,
                         "chunk_rows": prep[1].chunk_rows})
    out["instrumented_us_per_call"] = round(us_call, 3)
    out.update(res)
    return out


def run_ragged(torch, dev, args):
    """C4: B32 Hq16 Hkv2 D128 bf16, seq_lens ~ logU[128, 32768] (seed 1701)."""
    return run_decode_variant(torch, dev, args, "ragged-b32-logU128-32768", ragged_lengths(32, 1701), 3, 1701,
                              ragged=True)


def run_prefix(torch, dev, args):
    """C4 prefix: 16 requests share a 128-block (4096-token) prefix, private tails ~ U{1..512}."""
    import numpy as np

    tails = np.random.default_rng(1701).integers(1, 513, size=16)
    lens = [4096 + int(t) for t in tails]
    return run_decode_variant(torch, dev, args, "shared-prefix-16x4096+U512", lens, 40, 1701, prefix_blocks=128)


def run_prefix_large(torch, dev, args):
    """Shared prefix at scale: 64 requests share a 512-block (16384-token) prefix, private tails ~ U{1..512}."""
    import numpy as np

    tails = np.random.default_rng(7).integers(1, 513, size=64)
    lens = [16384 + int(t) for t in tails]
    return run_decode_variant(torch, dev, args, "shared-prefix-64x16384+U512", lens, 3, 7, prefix_blocks=512)


def run_prefix_sweep(torch, dev, args):
    """Shared-prefix cascade over chunk rows x prefix splits at four sizes (sharers x prefix tokens, tails
    ~ U{1..512}, seed 1701): the sweep behind the library's chunk-rows and prefix-split plans."""
    import numpy as np

    from flashdec_amd import cascade

    hq, hkv, d, bs = 16, 2, 128, 32
    sm = 1.0 / math.sqrt(d)
    shapes = [(16, 4096, 40, (4, 8, 16, 32)), (32, 8192, 10, (4, 8, 16, 32)), (64, 16384, 3, (2, 4, 8, 16)),
              (128, 16384, 2, (1, 2, 4, 8))]
    results = []
    for n, prefix, npools, sweep in shapes:
        tails = np.random.default_rng(1701).integers(1, 513, size=n)
        lens = [prefix + int(t) for t in tails]
        pools = decode_pools(torch, dev, lens, hq, hkv, d, bs, npools, 1701, prefix // bs)
        groups = [cascade.build_cascade_groups(p[3], p[4], bs, hq, hkv) for p in pools]
        plan_rows = cascade.plan_chunk_rows(groups[0], hq, hkv)
        for rows in (16, 32):
            times = {}
            for sp in sweep:
                def fn(i, sp=sp, rows=rows):
                    q, k, v, t, sl, o = pools[i % len(pools)]
                    cascade.paged_decode_attention_cascade_into(q, k, v, t, sl, o, groups[i % len(pools)],
                                                                sm_scale=sm, prefix_splits=sp, chunk_rows=rows)
                times[sp] = round(graph_ms_per_call(torch, dev, fn, 200 if n <= 32 else 40) * 1e3, 2)
            log(f"[bench] prefix-sweep {n}x{prefix} rows {rows}: "
                + ", ".join(f"{sp}: {t:.2f}" for sp, t in times.items()) + f" us/call (plan: rows {plan_rows})")
            results.append({"sharers": n, "prefix": prefix, "chunk_rows": rows, "us_per_call": times,
                            "planned_chunk_rows": plan_rows})
        del pools, groups
        torch.cuda.empty_cache()
    return {"workload": "prefix-sweep", "unit": "us/call by prefix splits", "results": results}


def run_formats(torch, dev, args):
    """General-path formats (beyond the C2 shape): head_dim 64, more than 16 query heads per KV
    head, MHA, dim-major caches and 8-token blocks, each B16 x 8192 tokens, bf16, block size 32
    unless named, through the public API (library-planned splits).  3 rotating pools each."""
    import flashdec_amd as fd

    cases = [  # name, Hq, Hkv, D, layout, block size, kernel the library runs
        ("d128-g8-token-major", 16, 2, 128, "token_major", 32, "mfma"),
        ("d64-g8-token-major", 16, 2, 64, "token_major", 32, "mfma"),
        ("d64-g7-token-major (Qwen2.5-0.5B heads)", 14, 2, 64, "token_major", 32, "mfma"),
        ("d128-g32-token-major", 64, 2, 128, "token_major", 32, "mfma, two 16-column blocks per wave"),
        ("d64-g71-token-major (MQA)", 71, 1, 64, "token_major", 32, "mfma, 3 head blocks of two column blocks"),
        ("d128-mha-token-major (B4)", 16, 16, 128, "token_major", 32, "mfma"),
        ("d128-g8-dim-major", 16, 2, 128, "dim_major", 32, "mfma dim-major, K staged through LDS"),
        ("d64-g8-dim-major", 16, 2, 64, "dim_major", 32, "mfma dim-major, K staged through LDS"),
        ("d128-g8-token-major-bs8", 16, 2, 128, "token_major", 8, "mfma"),
        ("d128-g8-dim-major-bs8", 16, 2, 128, "dim_major", 8, "mfma dim-major, K staged through LDS"),
    ]
    lines = []
    for name, hq, hkv, d, layout, bs, kernel in cases:
        batch = 4 if hq == hkv else 16
        lens = [8192] * batch
        pools = decode_pools(torch, dev, lens, hq, hkv, d, bs, 3, 31)
        if layout == "dim_major":
            pools = [(q, k.transpose(2, 3).contiguous(), v.transpose(2, 3).contiguous(), t, sl, o)
                     for q, k, v, t, sl, o in pools]

        def fn(i, pools=pools, layout=layout):
            q, k, v, table, sl, o = pools[i % len(pools)]
            fd.paged_decode_attention_into(q, k, v, table, sl, o, kv_layout=layout)

        ms = graph_ms_per_call(torch, dev, fn, 60)
        kv = sum(lens) * hkv * d * 2 * 2
        log(f"[bench] formats {name}: {ms * 1e3:.2f} us/call, K/V {kv / (ms * 1e-3) / 1e12:.2f} TB/s ({kernel})")
        lines.append({"case": name, "block_size": bs, "us_per_call": round(ms * 1e3, 2), "kv_bytes": kv,
                      "kv_tb_per_s": round(kv / (ms * 1e-3) / 1e12, 3), "kernel": kernel})
        del pools
    out = common_fields(args, "paged-decode us/call over general-path formats, B16 x 8192 tokens bf16",
                        lines[0]["us_per_call"], "us", lines[0]["us_per_call"] * 1e-3, False,
                        {"workload": "formats-b16-ctx8192", "block_size": "32 unless the case names 8"})
    out["cases"] = lines
    return out


def vllm_hook_call(torch, dev, batch, ctx, n_pools, seed, hq=16, hkv=2, d=128, bs=16):
    """``fn(i)``: the vLLM CUSTOM hook's launch on pool ``i % n_pools`` -- vLLM's 5-D NHD cache
    ``[blocks, 2, bs, kv_heads, d]``, every row at ``ctx`` tokens with its current token appended in
    the launch (slot of position ctx - 1), the split count as the hook picks it.  Returns
    (fn, splits, pools)."""
    import flashdec_amd  # noqa: F401  (loads the library)
    from flashdec_amd.paged_decode import _vllm_paged_decode_attention_into
    from flashdec_amd.vllm_splits import _AUTO_MIN_SPLIT_TOKENS, _select_num_splits

    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    pools = []
    for q, k, v, table, sl, o in decode_pools(torch, dev, [ctx] * batch, hq, hkv, d, bs, n_pools, seed):
        kv = torch.empty((k.shape[0], 2, bs, hkv, d), device=dev, dtype=k.dtype)
        kv[:, 0].copy_(k.permute(0, 2, 1, 3))
        kv[:, 1].copy_(v.permute(0, 2, 1, 3))
        del k, v
        pos = sl.long() - 1
        slots = table.long().gather(1, (pos // bs).unsqueeze(1)).squeeze(1) * bs + pos % bs
        ak = torch.randn((batch, hkv, d), device=dev).to(kv.dtype)
        av = torch.randn((batch, hkv, d), device=dev).to(kv.dtype)
        pools.append((q, ak, av, kv, table, sl, o, slots))
    splits = _select_num_splits(0, num_reqs=batch, num_kv_heads=hkv, logical_blocks=-(-ctx // bs),
                                target_programs=cus, auto_min_tokens=_AUTO_MIN_SPLIT_TOKENS, block_size=bs)
    ws = (torch.empty((batch, hq, splits, d), device=dev), torch.empty((batch, hq, splits), device=dev),
          torch.empty((batch, hq, splits), device=dev))

    def fn(i):
        q, ak, av, kv, table, sl, o, slots = pools[i % len(pools)]
        _vllm_paged_decode_attention_into(q, ak, av, kv, table, sl, o, slots, *ws, num_reqs=batch,
                                          num_q_heads=hq, num_kv_heads=hkv, head_dim=d, block_size=bs,
                                          sm_scale=d ** -0.5, num_splits=splits, max_seq_len=ctx)

    return fn, splits, pools


def run_vllm(torch, dev, args):
    """The vLLM CUSTOM hook's launch at the reference's published vLLM shapes: B8, Hq16/Hkv2/D128
    bf16, block size 16, vLLM's 5-D NHD cache ``[blocks, 2, 16, kv_heads, 128]``, every row at
    ctx 1024 or 2048 with its current token appended in the launch (slot of position len - 1),
    splits as the hook picks them (power of two nearest one workgroup per CU, >= 128 tokens each).
    8 rotating pools."""
    hq, hkv, d, bs, batch = 16, 2, 128, 16, 8
    lines = []
    for ctx in (1024, 2048):
        fn, splits, _ = vllm_hook_call(torch, dev, batch, ctx, 8, 41 + ctx)
        ms = graph_ms_per_call(torch, dev, fn, args.steps)
        algo = batch * ctx * hkv * d * 2 * 2 + 2 * batch * hq * d * 2 + 4 * batch * (ctx // bs) + 4 * batch
        log(f"[bench] vllm B8 ctx{ctx} bs16 fused append: {ms * 1e3:.2f} us/call, splits {splits}, "
            f"{algo / (ms * 1e-3) / 1e9:.1f} GB/s")
        lines.append({"ctx": ctx, "us_per_call": round(ms * 1e3, 2), "num_splits": splits,
                      "algorithmic_bytes": algo, "gb_per_s": round(algo / (ms * 1e-3) / 1e9, 1)})
        del fn
    out = common_fields(args, "vLLM CUSTOM hook decode us/call, B8 Hq16/Hkv2/D128 bf16 bs16 fused append",
                        lines[1]["us_per_call"], "us", lines[1]["us_per_call"] * 1e-3, False,
                        {"workload": "vllm-hook-b8-bs16-fused-append", "block_size": bs})
    out["cases"] = lines
    return out


# The reference's published p50s (ms, one RTX 5070, CUDA events around each eager call) for the
# rows the ref-shapes workload repeats.  FlashDec's own column of each summary.
REF_GROUPED_MS = {  # benchmarks/results/flashinfer_paged_decode_baseline_summary.md:24-39, full-length rows
    (1, 128): {"float16": 0.015616, "bfloat16": 0.016096},
    (16, 1024): {"float16": 0.176128, "bfloat16": 0.181664},
    (16, 8192): {"float16": 1.014976, "bfloat16": 1.050496},
    (64, 4096): {"float16": 2.562368, "bfloat16": 2.606080},
}
REF_DEFAULT_MS = {  # benchmarks/results/paged_decode_default_profile_summary.md:16-23, lengths ~ U{L/2..L}
    (1, 128): {"float16": 0.015328, "bfloat16": 0.038176},
    (16, 1024): {"float16": 0.155520, "bfloat16": 0.160864},
    (16, 8192): {"float16": 0.884576, "bfloat16": 0.928064},
    (64, 4096): {"float16": 1.934560, "bfloat16": 1.961216},
}
REF_VLLM_MS = {  # benchmarks/results/vllm_qwen_attention_summary.md:20-24
    (1, 128): 0.009952, (1, 1024): 0.013792, (4, 1024): 0.017888, (8, 1024): 0.024192, (8, 2048): 0.038528,
}
# benchmarks/results/multi_layer_transaction_summary.md:57: bf16 l2_b16_c1024, fused_cuda append and
# Triton decode -- the token's wall-clock p50, and its decode's device time per layer
REF_TOKEN_MS = {"token": 3.407861, "decode_layer": 0.133703}
REF_ROPE_APPEND_MS = {  # benchmarks/results/rope_kv_append_backends_summary.md:36-41, fused_cuda column
    "default": (16, 1024, {"float16": 1.436736, "bfloat16": 1.447424}),
    "large_batch": (64, 1024, {"float16": 3.419392, "bfloat16": 2.448480}),
    "long_context": (16, 4096, {"float16": 1.465536, "bfloat16": 1.076192}),
}


def event_p50_ms(torch, fn, warmup=20, repeat=100):
    """p50 ms of ``fn()`` timed as the reference times its rows: HIP events recorded around each
    eager call, a synchronisation after each (flashdec/benchmark.py:149-173)."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    times = []
    for _ in range(repeat):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        fn()
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b))
    return statistics.median(times)


def flushed_p50_ms(torch, dev, fn, reps=200, warmup=25):
    """p50 ms of ``fn()`` timed as the reference times its vLLM rows with Triton's do_bench
    (benchmarks/run_vllm_attention_microbench.py:230-241; Triton 3.6, not importable here): before
    each call a large buffer is zeroed so that the call starts with cold caches (Triton clears 256 MB;
    512 MiB here, more than MI355X's 256 MB Infinity Cache), HIP events record around each call, and
    the host does not wait between calls, so the launch's host work overlaps the clear."""
    flush = torch.empty(512 * 2**20 // 4, dtype=torch.int32, device=dev)
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(reps)]
    for a, b in evs:
        flush.zero_()
        a.record()
        fn()
        b.record()
    torch.cuda.synchronize()
    return statistics.median(a.elapsed_time(b) for a, b in evs)


def run_ref_shapes(torch, dev, args):
    """The reference's own published benchmark rows, repeated on MI355X with this library.

    - grouped decode, Hq32/Hkv8/D128, block size 32, token-major, fp16 and bf16, through
      ``paged_decode_attention_into`` (library-planned splits): every row at its full length (the
      FlashInfer-baseline rows) and lengths ~ U{L/2..L} (the default-configuration profile);
    - the vLLM hook's launch at the small Qwen shapes (B1 ctx128, B1 ctx1024, B4 ctx1024; block 16,
      fused current-token append) beside the B8 rows;
    - the whole ``rope_paged_kv_append(..., append_backend="fused_cuda")`` call (Hq32/Hkv8/D128,
      block 32, base 10000) on a one-layer cache seeded with the row's context, one token per call;
    - the multi-layer transaction token: a 2-layer ``DecodeEngine`` step at B16 ctx1024 (wall-clock
      p50 per token, synchronised around each).
    Every row is timed with the reference's method for it: events around each eager call with a
    synchronisation after each, p50 of 100 after 20 warm-ups (``event_p50_us``: the grouped,
    default-profile and RoPE + append rows), or Triton's do_bench (``flushed_p50_us``: the vLLM
    rows).  The decode and vLLM rows carry both, and the headline's method beside them (p50 of
    graph replays over rotating pools that together exceed the 256 MB Infinity Cache where the
    shape allows)."""
    import numpy as np
    import flashdec_amd as fd
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.rope import rope_paged_kv_append

    hq, hkv, d, bs = 32, 8, 128, 32
    dtypes = {"float16": torch.float16, "bfloat16": torch.bfloat16}
    rows = []
    probes = load_probes()
    sink = torch.zeros(256, dtype=torch.int32, device=dev)
    for kind, table in (("full", REF_GROUPED_MS), ("default", REF_DEFAULT_MS)):
        for (batch, ctx), ref in table.items():
            if kind == "full":
                lens = [ctx] * batch
            else:
                rng = np.random.default_rng(1000 + batch + ctx)
                lens = [int(x) for x in rng.integers(max(1, ctx // 2), ctx + 1, size=batch)]
            kv_bytes = sum(lens) * hkv * d * 2 * 2
            n_pools = max(3, min(48, -(-640 * 2**20 // kv_bytes)))
            algo = kv_bytes + 2 * batch * hq * d * 2 + 4 * batch * (-(-ctx // bs)) + 4 * batch
            for dname, dt in dtypes.items():
                pools = decode_pools(torch, dev, lens, hq, hkv, d, bs, n_pools, 77 + batch + ctx, dtype=dt)

                def fn(i, pools=pools):
                    q, k, v, tab, sl, o = pools[i % len(pools)]
                    fd.paged_decode_attention_into(q, k, v, tab, sl, o, sm_scale=d ** -0.5)

                counter = iter(range(10**9))
                ev_ms = event_p50_ms(torch, lambda: fn(next(counter)))
                fl_ms = flushed_p50_ms(torch, dev, lambda: fn(next(counter)))
                graph_us = graph_p50_us(torch, dev, fn, n_pools, samples=120, warmup=24)
                line = {"rows": kind, "batch": batch, "ctx": ctx, "dtype": dname, "pools": n_pools,
                        "event_p50_us": round(ev_ms * 1e3, 2), "flushed_p50_us": round(fl_ms * 1e3, 2),
                        "graph_p50_us": round(graph_us, 2),
                        "algorithmic_bytes": algo, "graph_gb_per_s": round(algo / (graph_us * 1e-6) / 1e9, 1),
                        "reference_rtx5070_us": round(ref[dname] * 1e3, 2),
                        "speedup_event": round(ref[dname] * 1e3 / (ev_ms * 1e3), 2)}
                if kind == "full" and dname == "bfloat16":
                    # the ceiling of a read of these bytes on this part: one non-temporal read of a
                    # buffer of the call's algorithmic bytes (the floor workload's probe), same method
                    n16 = (algo + 15) // 16 * 16
                    bufs = [torch.empty(n16, dtype=torch.uint8, device=dev) for _ in range(n_pools)]

                    def rd(i, bufs=bufs, n16=n16):
                        st = torch.cuda.current_stream(dev).cuda_stream
                        assert probes.fdp_stream_read(bufs[i % len(bufs)].data_ptr(), n16, sink.data_ptr(), st,
                                                      None, None) == 0

                    read_us = graph_p50_us(torch, dev, rd, n_pools, samples=120, warmup=24)
                    line["bare_read_graph_p50_us"] = round(read_us, 2)
                    line["bare_read_gb_per_s"] = round(algo / (read_us * 1e-6) / 1e9, 1)
                    log(f"[bench] ref-shapes bare read of B{batch} ctx{ctx}'s {algo} bytes: {read_us:.2f} us "
                        f"({line['bare_read_gb_per_s']} GB/s)")
                    del bufs, rd
                rows.append(line)
                log(f"[bench] ref-shapes decode {kind} B{batch} ctx{ctx} {dname}: event p50 {ev_ms * 1e3:.2f} us, "
                    f"flushed p50 {fl_ms * 1e3:.2f} us, graph p50 {graph_us:.2f} us ({line['graph_gb_per_s']} GB/s); reference "
                    f"{ref[dname] * 1e3:.2f} us on RTX 5070")
                del pools, fn
                torch.cuda.empty_cache()
    for (batch, ctx), ref in REF_VLLM_MS.items():
        fn, splits, pools = vllm_hook_call(torch, dev, batch, ctx, 8, 51 + batch + ctx)
        counter = iter(range(10**9))
        ev_ms = event_p50_ms(torch, lambda: fn(next(counter)))
        fl_ms = flushed_p50_ms(torch, dev, lambda: fn(next(counter)))
        graph_us = graph_p50_us(torch, dev, fn, len(pools), samples=120, warmup=24)
        rows.append({"rows": "vllm-hook", "batch": batch, "ctx": ctx, "dtype": "bfloat16", "num_splits": splits,
                     "event_p50_us": round(ev_ms * 1e3, 2), "flushed_p50_us": round(fl_ms * 1e3, 2),
                     "graph_p50_us": round(graph_us, 2), "reference_rtx5070_us": round(ref * 1e3, 2),
                     "speedup_flushed": round(ref / fl_ms, 2)})
        log(f"[bench] ref-shapes vllm hook B{batch} ctx{ctx}: event p50 {ev_ms * 1e3:.2f} us, flushed p50 "
            f"{fl_ms * 1e3:.2f} us, graph p50 {graph_us:.2f} us; reference {ref * 1e3:.2f} us on RTX 5070 (do_bench)")
        del fn, pools
    for name, (batch, ctx, ref) in REF_ROPE_APPEND_MS.items():
        for dname, dt in dtypes.items():
            steps = 20 + 100 + 1
            blocks = batch * (-(-(ctx + steps) // bs)) + 8
            cache = PagedKVCache(1, hkv, d, bs, blocks, dtype=dt, device=dev)
            ids = list(range(batch))
            for r in ids:
                cache.add_request(r)
            cache.seed_context(ids, ctx)
            gen = torch.Generator(device=dev)
            gen.manual_seed(91 + batch + ctx)
            q = torch.randn((batch, hq, d), device=dev, generator=gen).to(dt)
            k = torch.randn((batch, hkv, d), device=dev, generator=gen).to(dt)
            v = torch.randn((batch, hkv, d), device=dev, generator=gen).to(dt)
            ev_ms = event_p50_ms(torch, lambda: rope_paged_kv_append(cache, 0, ids, q, k, v,
                                                                      append_backend="fused_cuda"))
            rows.append({"rows": "rope-append", "case": name, "batch": batch, "ctx": ctx, "dtype": dname,
                         "event_p50_us": round(ev_ms * 1e3, 2), "reference_rtx5070_us": round(ref[dname] * 1e3, 2),
                         "speedup_event": round(ref[dname] / ev_ms, 2)})
            log(f"[bench] ref-shapes rope_paged_kv_append fused {name} B{batch} ctx{ctx} {dname}: event p50 "
                f"{ev_ms * 1e3:.2f} us; reference {ref[dname] * 1e3:.2f} us on RTX 5070")
            del cache
    # The multi-layer transaction token (benchmarks/run_multi_layer_engine.py:100-230): a 2-layer
    # engine, B16 with 1024 tokens of seeded context, Hq32/Hkv8/D128 bf16; one token = begin_step,
    # step_layer per layer (fused RoPE + append, then decode), commit_step, synchronised before and
    # after; wall-clock p50 over 100 tokens after 10, and the decode launches' device time per layer
    # (the library's timing hook) beside it.
    from flashdec_amd.engine import DecodeEngine

    layers, batch, ctx, warm, steps = 2, 16, 1024, 10, 100
    cache = PagedKVCache(layers, hkv, d, bs, batch * (-(-(ctx + warm + steps + 1) // bs)) + 8,
                         dtype=torch.bfloat16, device=dev)
    engine = DecodeEngine(cache, append_backend="fused_cuda", decode_backend="triton")
    ids = list(range(batch))
    for r in ids:
        engine.add_request(r)
    engine.admit()
    cache.seed_context(ids, ctx)
    gen = torch.Generator(device=dev)
    gen.manual_seed(4321)
    inputs = [[tuple(torch.randn(shape, device=dev, generator=gen).to(torch.bfloat16)
                     for shape in ((batch, hq, d), (batch, hkv, d), (batch, hkv, d))) for _ in range(layers)]
              for _ in range(8)]
    wall = []
    for s in range(warm + steps):
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        tx = engine.begin_step(ids)
        for layer in range(layers):
            engine.step_layer(tx, layer, *inputs[s % len(inputs)][layer])
        engine.commit_step(tx)
        torch.cuda.synchronize()
        wall.append((time.perf_counter() - t0) * 1e3)
    token_ms = statistics.median(wall[warm:])
    # the decode launch of one such layer, timed through the library's hook around exactly its kernels
    tq, tk, tv = inputs[0][0]
    pool = (tq, cache.k_cache[0], cache.v_cache[0], cache.block_tables(ids).to(dev),
            cache.seq_lens_tensor(ids).to(dev), torch.empty_like(tq))
    attn_us, red_us = attention_kernel_us(torch, [prepared_args(pool, d ** -0.5, bs, hkv)], 100)
    rows.append({"rows": "multi-layer-token", "layers": layers, "batch": batch, "ctx": ctx, "dtype": "bfloat16",
                 "wall_p50_ms": round(token_ms, 4), "decode_kernels_us_per_layer": round(attn_us + red_us, 2),
                 "reference_rtx5070_token_ms": REF_TOKEN_MS["token"],
                 "reference_rtx5070_decode_device_ms_per_layer": REF_TOKEN_MS["decode_layer"],
                 "speedup_token": round(REF_TOKEN_MS["token"] / token_ms, 2)})
    log(f"[bench] ref-shapes multi-layer token L{layers} B{batch} ctx{ctx} bf16: wall p50 {token_ms:.3f} ms/token, "
        f"decode kernels {attn_us + red_us:.1f} us/layer; reference {REF_TOKEN_MS['token']:.3f} ms/token, decode "
        f"{REF_TOKEN_MS['decode_layer'] * 1e3:.1f} us/layer on RTX 5070")
    del engine, cache
    head = next(r for r in rows if r["rows"] == "full" and r["batch"] == 16 and r["ctx"] == 8192
                and r["dtype"] == "bfloat16")
    out = common_fields(args, "reference benchmark rows on MI355X: grouped decode B16 ctx8192 Hq32/Hkv8/D128 bf16 "
                        "(us/call, reference timing method)", head["event_p50_us"], "us",
                        head["event_p50_us"] * 1e-3, False, {"workload": "reference-benchmark-rows"})
    out["rows"] = rows
    return out



def run_engine_prefix(torch, dev, args):
    """36-layer DecodeEngine steps over a shared prefix: B64 rows attached to one resident
    16384-token prefix, private tails ~ U{64..512}, Hq16 Hkv2 D128 bf16.  Two step graphs on the
    same engine and schedule: the cascade (the engine's default here) and the per-row decode with
    cached K/V loads."""
    import numpy as np

    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine

    layers, batch, hq, hkv, d, bs, prefix = 36, 64, 16, 2, 128, 32, 16384
    steps = max(20, args.engine_steps // 2)
    tails = np.random.default_rng(77).integers(64, 513, size=batch)
    pb = prefix // bs
    width = pb + (int(tails.max()) + 2 * steps + 64 + bs - 1) // bs
    cache = PagedKVCache(layers, hkv, d, bs, max_blocks=pb + batch * (width - pb), dtype=torch.bfloat16,
                         device=dev, prefix_cache_capacity_blocks=pb)
    gen = torch.Generator(device=dev)
    gen.manual_seed(113)
    for layer in range(layers):
        cache.k_cache[layer].normal_(generator=gen)
        cache.v_cache[layer].normal_(generator=gen)
    cache.enable_graph_metadata(batch, width)
    engine = DecodeEngine(cache)
    shape = (layers, pb, hkv, bs, d)
    engine.register_prefix("sys", torch.empty(shape, device=dev, dtype=torch.bfloat16).normal_(generator=gen),
                           torch.empty(shape, device=dev, dtype=torch.bfloat16).normal_(generator=gen))
    ids = list(range(batch))
    for rid in ids:
        engine.add_request(rid)
    engine.admit(ids, prefix_id="sys")
    for rid, t in zip(ids, tails):
        cache.seed_context([rid], int(t))
    log(f"[bench] engine-prefix: {layers} layers, B{batch} sharing {prefix} tokens, tails U{{64..512}}")
    result = {}
    for name, cascade in (("cascade", True), ("per_row", False)):
        sg = engine.capture_step_graph(batch, hq, base=1e6, cascade=cascade)
        sg.q.normal_(generator=gen)
        sg.k.normal_(generator=gen)
        sg.v.normal_(generator=gen)

        def step(sg=sg):
            tx = engine.begin_step(ids)
            engine.step_graph(tx, sg)
            engine.commit_step(tx)

        for _ in range(10):
            step()
        torch.cuda.synchronize()
        start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        start.record()
        for _ in range(steps):
            step()
        stop.record()
        torch.cuda.synchronize()
        result[name] = start.elapsed_time(stop) / steps
        log(f"[bench] engine-prefix {name}: {result[name]:.3f} ms/step")
        del sg
    out = common_fields(args, "36-layer DecodeEngine step ms over a shared 16384-token prefix, B64",
                        round(result["cascade"], 4), "ms/step", result["cascade"], False,
                        {"workload": "engine-prefix-36l-b64-16384", "layers": layers, "batch": batch,
                         "prefix_tokens": prefix, "tails": "U{64..512}", "steps": steps, "path": "cascade graph"})
    out["tokens_per_s"] = round(batch / (result["cascade"] * 1e-3), 1)
    out["per_row_path"] = {"ms_per_step": round(result["per_row"], 4), "kv_loads": "plain (kv_reuse)"}
    return out


def run_engine(torch, dev, args):
    """C5: 36-layer DecodeEngine step, B64 Hq16 Hkv2 D128 bf16, context 8192, abort every 100th step."""
    from flashdec_amd.cache import PagedKVCache
    from flashdec_amd.engine import DecodeEngine

    layers, batch, hq, hkv, d, bs, ctx = 36, 64, 16, 2, 128, 32, 8192
    steps = args.engine_steps
    # room for the warm-ups, the timed steps, the separate-RoPE comparison steps and the eager steps
    n_eager, warm_eager = 20, 5
    width = (ctx + 3 * 20 + 3 * steps + 2 + n_eager + warm_eager + bs - 1) // bs
    cache = PagedKVCache(layers, hkv, d, bs, max_blocks=batch * width, dtype=torch.bfloat16, device=dev)
    gen = torch.Generator(device=dev)
    gen.manual_seed(109)
    for layer in range(layers):
        cache.k_cache[layer].normal_(generator=gen)
        cache.v_cache[layer].normal_(generator=gen)
    cache.enable_graph_metadata(batch, width)
    engine = DecodeEngine(cache)
    ids = list(range(batch))
    for rid in ids:
        engine.add_request(rid)
    engine.admit()
    cache.seed_context(ids, ctx)
    log(f"[bench] engine: {layers} layers, B{batch}, context {ctx}, cache {cache.k_cache.numel() * 4 / 2**30:.1f} GiB")
    sg = engine.capture_step_graph(batch, hq, base=1e6)
    sg.q.normal_(generator=gen)
    sg.k.normal_(generator=gen)
    sg.v.normal_(generator=gen)

    def graph_step():
        tx = engine.begin_step(ids)
        engine.step_graph(tx, sg)
        engine.commit_step(tx)

    def abort_step(bad_layer):
        before = (cache.num_used_blocks, cache.seq_lens_tensor(ids).cpu())
        tx = engine.begin_step(ids)
        try:
            for layer in range(layers):
                q = sg.q[layer][..., :-1] if layer == bad_layer else sg.q[layer]
                engine.step_layer(tx, layer, q, sg.k[layer], sg.v[layer], base=1e6)
        except ValueError:
            pass
        else:
            raise RuntimeError("the malformed layer input was accepted")
        after = (cache.num_used_blocks, cache.seq_lens_tensor(ids).cpu())
        return before[0] == after[0] and torch.equal(before[1], after[1])

    # warm-up: the host runs ahead of the replays, so the first steps also
    # grow the pinned staging pool of the per-step metadata copies
    warm = 20
    for _ in range(warm):
        graph_step()
    # and the eager path the timed aborts take (its first launches load kernels)
    if not abort_step(1):
        raise RuntimeError("warm-up abort did not roll back cleanly")
    torch.cuda.synchronize()
    committed = 0
    rollbacks_ok = 0
    aborts = 0
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    start.record()
    for i in range(steps):
        if i % 100 == 99:
            aborts += 1
            rollbacks_ok += abort_step((i // 100) % layers)
        else:
            graph_step()
            committed += 1
    stop.record()
    torch.cuda.synchronize()
    wall_s = time.perf_counter() - t0
    device_ms = start.elapsed_time(stop)
    ms_per_step = device_ms / steps
    separate = None
    if sg.fused_rope:
        # the same steps with RoPE + append as its own kernel per layer
        sg_sep = engine.capture_step_graph(batch, hq, base=1e6, fuse_rope=False)
        sg_sep.q.copy_(sg.q)
        sg_sep.k.copy_(sg.k)
        sg_sep.v.copy_(sg.v)

        def graph_step_sep():
            tx_ = engine.begin_step(ids)
            engine.step_graph(tx_, sg_sep)
            engine.commit_step(tx_)

        # the same schedule as the timed loop above: every 100th step aborts
        n_sep = steps
        for _ in range(warm):
            graph_step_sep()
        torch.cuda.synchronize()
        committed_sep = warm
        start.record()
        for i in range(n_sep):
            if i % 100 == 99:
                abort_step((i // 100) % layers)
            else:
                graph_step_sep()
                committed_sep += 1
        stop.record()
        torch.cuda.synchronize()
        separate = start.elapsed_time(stop) / n_sep
    else:
        committed_sep = 0
    # the same graph steps with cos/sin evaluated inside the kernels (the
    # cache's rope_tables off) instead of read from the cache's table
    cache.rope_tables = False
    sg_eval = engine.capture_step_graph(batch, hq, base=1e6)
    cache.rope_tables = True
    assert sg_eval.cos_sin_table is None and sg.cos_sin_table is not None
    sg_eval.q.copy_(sg.q)
    sg_eval.k.copy_(sg.k)
    sg_eval.v.copy_(sg.v)

    def graph_step_eval():
        tx_ = engine.begin_step(ids)
        engine.step_graph(tx_, sg_eval)
        engine.commit_step(tx_)

    for _ in range(warm):
        graph_step_eval()
    torch.cuda.synchronize()
    start.record()
    for _ in range(steps):
        graph_step_eval()
    stop.record()
    torch.cuda.synchronize()
    eval_ms = start.elapsed_time(stop) / steps
    committed_sep += warm + steps
    log(f"[bench] engine: graph steps with cos/sin evaluated in the kernels (no table): {eval_ms:.3f} ms/step")
    # the same steps without a graph: step_layer per layer, as the reference's
    # engine runs (after layer 0, RoPE + append inside the decode launch)

    def eager_step():
        tx_ = engine.begin_step(ids)
        for layer in range(layers):
            engine.step_layer(tx_, layer, sg.q[layer], sg.k[layer], sg.v[layer], base=1e6)
        engine.commit_step(tx_)

    ctx_eager = ctx + warm + committed + committed_sep  # the rows' length when the eager steps start
    for _ in range(warm_eager):
        eager_step()
    torch.cuda.synchronize()
    t1 = time.perf_counter()
    start.record()
    for _ in range(n_eager):
        eager_step()
    stop.record()
    torch.cuda.synchronize()
    eager_ms = start.elapsed_time(stop) / n_eager
    eager_wall_ms = (time.perf_counter() - t1) * 1e3 / n_eager
    committed_eager = warm_eager + n_eager
    log(f"[bench] engine: eager steps (step_layer per layer): {eager_ms:.3f} ms/step, wall {eager_wall_ms:.3f} "
        f"(context {ctx_eager + warm_eager}, after the graph steps)")
    # per-layer attention kernel, measured on the same shapes through the timing hook
    from flashdec_amd import paged_decode as pd

    tx = engine.begin_step(ids)
    meta = cache.graph_metadata(batch)  # this transaction's metadata lives in the arena
    prepared = []
    for layer in range(4):
        # the launch the graph replays: with fused RoPE the raw q and this
        # step's K/V row (stored to its slot, which the abort below frees)
        args_ = pd._lib.PagedDecodeArgs()
        q_in = sg.q[layer] if sg.fused_rope else sg.q_rot[layer]
        pd._fill_common(args_, q_in, cache.k_cache[layer], cache.v_cache[layer],
                        pd._cache_strides(cache.k_cache[layer], 2, 3), pd._cache_strides(cache.v_cache[layer], 2, 3),
                        meta.block_tables, meta.eff_lens, sg.out[layer], hkv, bs, 1.0 / math.sqrt(d))
        args_.num_blocks = cache.max_blocks
        args_.max_seq_len = width * bs
        acc, mx, sm, _ = pd._auto_workspace(q_in, hkv, sg.num_splits, pd._lib.current_stream_handle(dev))
        pd._fill_workspace(args_, acc, mx, sm, sg.num_splits)
        if sg.fused_rope:
            pd._fill_append(args_, sg.k[layer], sg.v[layer], meta.slots)
            args_.rotary_dim = sg.rotary_dim
            args_.rope_base = sg.base
            if sg.cos_sin_table is not None:
                args_.rope_cos_sin_table = sg.cos_sin_table.data_ptr()
                args_.rope_table_rows = sg.cos_sin_table.shape[1]
        prepared.append((args_, pd._lib.current_stream_handle(dev)))
    attn_us, red_us = attention_kernel_us(torch, prepared, 16)
    engine.abort_step(tx)
    # K+V bytes one layer's decode reads at the end
    kv_layer = (ctx + warm + committed + committed_sep + committed_eager) * batch * hkv * d * 2 * 2
    log(f"[bench] engine: {ms_per_step:.3f} ms/step over {steps} steps ({committed} committed, {aborts} aborted, "
        f"{rollbacks_ok} clean rollbacks); wall {wall_s * 1e3 / steps:.3f} ms/step; attention kernel {attn_us:.1f} us"
        f" per layer, reducer {red_us:.2f} us")
    out = common_fields(args, "36-layer DecodeEngine step ms, B64 ctx8192 Qwen2.5-3B attention shape (C5)",
                        round(ms_per_step, 4), "ms/step", ms_per_step, False,
                        {"workload": "engine-36l-b64-ctx8192", "layers": layers, "batch": batch, "context": ctx,
                         "steps": steps, "committed_steps": committed, "aborted_steps": aborts,
                         "clean_rollbacks": rollbacks_ok, "num_splits": sg.num_splits,
                         "fused_rope": sg.fused_rope, "kernels_per_layer": 2 if sg.fused_rope else 3,
                         "timing": "events around the whole loop; graph-replayed steps, eager abort steps"})
    out["steps"] = steps
    out["tokens_per_s"] = round(committed * batch / (device_ms * 1e-3), 1)
    out["wall_ms_per_step"] = round(wall_s * 1e3 / steps, 4)
    out["eager_path"] = {"ms_per_step": round(eager_ms, 4), "wall_ms_per_step": round(eager_wall_ms, 4),
                         "steps": n_eager, "context_at_start": ctx_eager + warm_eager,
                         "note": "begin_step, 36 x step_layer, commit_step; no graph; measured after the graph "
                                 "steps, so at a longer context than the graph line"}
    out["rope_cos_sin"] = {"table": "the cache's own (PagedKVCache.rope_table), the default: bit-exact to apply_rope",
                           "no_table_ms_per_step": round(eval_ms, 4),
                           "no_table_note": "rope_tables off: cos/sin evaluated in the kernels (float64, rounded "
                                            "once), same graph steps without aborts"}
    if separate is not None:
        out["separate_rope_kernel_path"] = {"ms_per_step": round(separate, 4), "kernels_per_layer": 3,
                                            "steps": steps}
        log(f"[bench] engine: RoPE + append as its own kernel: {separate:.3f} ms/step")
    out["roofline"] = {"bound": "hbm", "kernel_us_mean": round(attn_us, 2), "reducer_us_mean": round(red_us, 3),
                       "algorithmic_bytes_per_layer": kv_layer,
                       "achieved": round(kv_layer / (attn_us * 1e-6) / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                       "frac": round(kv_layer / (attn_us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)}
    return out


def main():
    args = parse_args()
    if args.gpus != 1:
        print(
            f"bench.py runs on exactly one GPU; --gpus {args.gpus} is not supported "
            "(the decode path shards per request / KV head with no exchange).",
            file=sys.stderr,
        )
        sys.exit(2)

    # the CPU leg first: its worker processes start before this process touches the GPU
    cpu_res = None
    if args.workload == "decode" and not args.no_cpu and not args.profile_kernels:
        cpu_res = cpu_baseline(args.cpu_seconds)

    import torch

    import flashdec_amd as fd
    from flashdec_amd import _lib

    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    if args.workload in ("c2-timeline", "c4-timeline"):
        # the measurement build of the library, with the per-wave stamps
        from flashdec_amd import _build

        if not _build.TIMELINE_LIB_PATH.exists():
            raise RuntimeError(f"{_build.TIMELINE_LIB_PATH} is not built: run __graft_entry__.build()")
        os.environ["FLASHDEC_AMD_LIB"] = str(_build.TIMELINE_LIB_PATH)
    _lib.load_library()
    if args.workload != "decode":
        run = {"c2-floor": run_c2_floor, "c2-timeline": run_c2_timeline, "c4-timeline": run_c4_timeline, "rope": run_rope, "ragged": run_ragged, "prefix": run_prefix, "prefix-large": run_prefix_large,
               "prefix-sweep": run_prefix_sweep, "engine": run_engine, "engine-prefix": run_engine_prefix, "formats": run_formats,
               "vllm": run_vllm, "ref-shapes": run_ref_shapes}[args.workload]
        print(json.dumps(run(torch, dev, args)), flush=True)
        return
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
    # warm-up: at least --warmup calls and at least 100 ms of calls
    t_warm = time.perf_counter()
    warm_calls = 0
    while warm_calls < args.warmup or time.perf_counter() - t_warm < 0.1:
        n = max(len(pools), args.warmup - warm_calls)
        back_to_back(torch, _lib, prepared, n)
        warm_calls += n
    warmup_ms = (time.perf_counter() - t_warm) * 1e3
    log(f"[bench] warmup: {warm_calls} calls in {warmup_ms:.0f} ms")

    def capture(n_calls):
        g = torch.cuda.CUDAGraph()
        cap = torch.cuda.Stream(dev)
        cap.wait_stream(stream)
        with torch.cuda.stream(cap):
            call(0)  # the capture stream's split workspace exists before capture
            cap.synchronize()
            with torch.cuda.graph(g, stream=cap):
                for i in range(n_calls):
                    call(i)
        stream.wait_stream(cap)
        torch.cuda.synchronize()
        g.replay()  # untimed replay (first-replay setup)
        torch.cuda.synchronize()
        return g

    # (1) exactly K steps in one graph, replayed once between synchronisations
    graph = capture(args.steps)
    t_start = torch.cuda.Event(enable_timing=True)
    t_stop = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t_start.record(stream)
    graph.replay()
    t_stop.record(stream)
    torch.cuda.synchronize()
    total_ms = t_start.elapsed_time(t_stop)
    single_ms = total_ms / args.steps
    log(f"[bench] graph: {args.steps} calls in {total_ms:.3f} ms -> {single_ms * 1e3:.2f} us/call")

    # (2) p50 over samples: a graph of one call per pool (one rotation over
    # the pools), replayed back to back with events between the replays
    sample_graph = capture(len(pools))
    n_samples = 240
    marks = [torch.cuda.Event(enable_timing=True) for _ in range(n_samples + 1)]
    torch.cuda.synchronize()
    marks[0].record(stream)
    for i in range(n_samples):
        sample_graph.replay()
        marks[i + 1].record(stream)
    torch.cuda.synchronize()
    per_call = sorted(marks[i].elapsed_time(marks[i + 1]) / len(pools) for i in range(n_samples))
    ms_per_step = statistics.median(per_call)
    log(f"[bench] p50 over {n_samples} samples of {len(pools)} calls: {ms_per_step * 1e3:.2f} us/call "
        f"(p10 {per_call[n_samples // 10] * 1e3:.2f}, p90 {per_call[9 * n_samples // 10] * 1e3:.2f})")

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

    # the C2 config names ctx1024 too: the same call on 48 pools at ctx1024,
    # timed the same way, rides along in the line
    companion = None
    if (batch, ctx) == (8, 2048):
        pools_1k = build_pools(torch, args.pools, batch, 1024, hq, hkv, d, bs, dev)

        def call_1k(i):
            q, k, v, table, lens, out = pools_1k[i % len(pools_1k)]
            fd.paged_decode_attention_into(q, k, v, table, lens, out, sm_scale=sm_scale)

        us_1k = graph_p50_us(torch, dev, call_1k, len(pools_1k))
        prepared_1k = [prepared_args(pool, sm_scale, bs, hkv) for pool in pools_1k]
        attn_1k, red_1k = attention_kernel_us(torch, prepared_1k, min(4 * len(pools_1k), 192))
        nb_1k = algorithmic_bytes(batch, 1024, hq, hkv, d, bs)
        companion = {
            "us_per_call": round(us_1k, 3),
            "value": round(nb_1k / (us_1k * 1e-6) / 1e9, 2),
            "unit": "GB/s",
            "hbm_frac": round(nb_1k / (us_1k * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "num_splits": prepared_1k[0][0].num_splits,
            "kernel_us_mean": round(attn_1k, 3),
            "reducer_us_mean": round(red_1k, 3),
            "roofline_frac": round(nb_1k / (attn_1k * 1e-6) / 1e9 / HBM_PEAK_GBS, 4),
            "algorithmic_bytes_per_call": nb_1k,
        }
        log(f"[bench] ctx1024: {us_1k:.2f} us/call, attention kernel {attn_1k:.2f} us, reducer {red_1k:.2f} us")

    achieved = nbytes / (kernel_ms * 1e-3) / 1e9
    traffic, traffic_meta = load_traffic()
    if traffic_meta is not None and traffic_meta.get("algorithmic_bytes_per_call") != nbytes:
        # the committed counters are for the headline shape only
        traffic, traffic_meta = None, None
    traffic_src = None if traffic_meta is None else os.path.relpath(TRAFFIC_SUMMARY, ROOT)
    if traffic is not None:
        traffic = int(round(traffic))
    value = nbytes / (ms_per_step * 1e-3) / 1e9
    cpu = None
    if cpu_res is not None:
        torch_res, numpy_res, threads = cpu_res
        c2 = torch_res["C2"]
        cpu = {
            "value": c2["gb_per_s"],
            "unit": "GB/s",
            "cores": c2["threads"],
            "kind": "port",
            "sample": f"fp32 torch-CPU restatement of paged_reference.py:92-125 in its per-(sequence, query-head) "
                      f"loop (oracle/torch_loop.py) on the full B8 ctx2048 call (bf16 inputs upcast per head, as "
                      f"the reference does), torch.set_num_threads({threads}) (os.cpu_count() "
                      f"{os.cpu_count()}, capped at the box's {CPU_THREAD_CAP}-thread share), one synchronous call "
                      f"at a time, p50 of {c2['calls']} calls after 3 warm-ups: {c2['us_per_call']:.0f} us/call",
            "torch_get_num_threads": c2["threads"],
            "os_cpu_count": os.cpu_count(),
            "cpu_model": cpu_model(),
            "configs": torch_res,
            "numpy_oracle": {
                "kind": "port",
                "sample": "numpy oracle (oracle/attention.py) with a call's (row, KV head) pairs shared by worker "
                          "processes (one BLAS thread each); each call one synchronised unit between two barriers "
                          "that the parent and every worker pass, p50 after 3 warm-ups",
                "configs": numpy_res,
            },
        }
        log(f"[bench] cpu torch loop: C2 {c2['us_per_call'] / 1e3:.2f} ms/call ({c2['threads']} threads), "
            f"C1 {torch_res['C1']['us_per_call'] / 1e3:.2f} ms/call; numpy oracle C2 "
            f"{numpy_res['C2']['us_per_call'] / 1e3:.2f} ms/call ({numpy_res['C2']['processes']} processes)")

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "us_per_call": round(ms_per_step * 1e3, 3),
        "p50_samples": n_samples,
        "calls_per_sample": len(pools),
        "single_replay_ms_per_step": round(single_ms, 6),
        "warmup_ms": round(warmup_ms, 1),
        "warmup_calls": warm_calls,
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
            "timing": "ms_per_step/value: p50 over 240 back-to-back replays of a graph of one call per pool, "
                      "hipEvents between replays; single_replay_ms_per_step: a graph of exactly K calls replayed "
                      "once between synchronisations",
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
            "kernel_timing": "eager back-to-back calls: the library records HIP events around exactly the "
                             "attention dispatch (hipExtLaunchKernel), which a captured graph cannot carry per "
                             "kernel; the rocprofv3 kernel trace of the graph replays is in profiles/",
            "reducer_us_mean": round(statistics.mean(red_ms) * 1e3, 3),
            "algorithmic_bytes_per_call": nbytes,
            "traffic_source": traffic_src,
        },
        "cpu_baseline": cpu,
    }
    if companion is not None:
        result["ctx1024"] = companion
    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
