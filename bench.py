#!/usr/bin/env python3
"""Benchmark of the exact-search hot path on one MI355X.

Default: exact top-10 cosine over 1,000,000 x 384 fp32 (the 1,000-centre
Gaussian mixture, sigma 0.3, normalised), batches of 1024 queries, queries
and results resident in HBM.  Prints ONE JSON line whose value is the batch
throughput; the same line carries the batch-1 throughput, the p50/p95
single-query latency at 100,000 x 384 and, unless --quick, one entry per
other configuration (int8 prefilter, IVF-flat, IVF-PQ).

  python bench.py [--steps K] [--warmup W] [--batch B] [--workload flat|int8|ivf|ivfpq]

Every workload first checks a sample of queries against the CPU oracle
(bit-identical results) and stops if they differ.  Throughput is timed with
no per-kernel synchronisation; kernel durations for the roofline come from
a separate pass with HIP events recorded on the stream the kernels run on.
The CPU baseline of each line is the oracle's restatement of the route the
reference's CPU path takes for that configuration (no GPU context:
FlatGPUSearch.swift:63-94, 754-779, 1003-1037), timed on a bounded sample on
this host's cores in the same run; each baseline records the CPU model,
nproc, NUMA layout and the threads it used.
"""
from __future__ import annotations

import argparse
import json
import os
import re
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

HBM_PEAK_GBS = 8000.0
FP32_MFMA_TFLOPS = 157.3
BF16_MFMA_TFLOPS = 2500.0  # dense
METRIC = "queries/sec exact top-10 @1M×384 fp32 (batch 1/1024); p50 single-query µs @100k"
CPU_THREADS = min(16, os.cpu_count() or 1)  # the host's CPU share of one GPU


def host_info() -> dict:
    """CPU model, logical CPUs, NUMA nodes and the threads a baseline uses."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    numa = []
    for node in sorted(Path("/sys/devices/system/node").glob("node[0-9]*")):
        try:
            numa.append(f"{node.name}: cpus {(node / 'cpulist').read_text().strip()}")
        except OSError:
            pass
    return {"cpu_model": model, "nproc": os.cpu_count(), "numa": numa,
            "threads_used": CPU_THREADS,
            "note": "worker threads sized to the CPU share of one GPU on this host (16)"}


def cpu_line(value, unit, cores, sample, kind="port"):
    return {"value": round(value, 2), "unit": unit, "cores": cores, "kind": kind, "sample": sample,
            "host": host_info()}


def sha(*arrays) -> str:
    import hashlib

    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(a).tobytes())
    return h.hexdigest()


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def percentile_nearest_rank(samples, p):
    """LatencyDistribution.swift:154-160: index ceil(p n) - 1."""
    s = sorted(samples)
    idx = max(0, min(len(s) - 1, int(np.ceil(p * len(s))) - 1))
    return s[idx]


def measured_traffic(kernel: str, workload: str):
    """HBM bytes per launch from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/hbm_traffic.md), or None."""
    path = ROOT / "profiles" / "hbm_traffic.md"
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if len(cells) >= 4 and cells[0] == kernel and cells[1] == workload:
            try:
                return int(float(cells[2]) + float(cells[3]))
            except ValueError:
                return None
    return None


def roofline_hbm(kernel, workload, bytes_per_launch, avg_s):
    gbs = bytes_per_launch / avg_s / 1e9
    return {"bound": "hbm", "achieved": round(gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
            "frac": round(gbs / HBM_PEAK_GBS, 4), "traffic": measured_traffic(kernel, workload),
            "kernel": kernel, "avg_launch_us": round(avg_s * 1e6, 2),
            "bytes_per_launch": int(bytes_per_launch)}


def roofline_mfma(kernel, workload, flops_per_launch, avg_s, peak=None):
    peak = peak or FP32_MFMA_TFLOPS
    tf = flops_per_launch / avg_s / 1e12
    return {"bound": "mfma", "achieved": round(tf, 2), "peak": peak, "unit": "TFLOP/s",
            "frac": round(tf / peak, 4), "traffic": measured_traffic(kernel, workload),
            "kernel": kernel, "avg_launch_us": round(avg_s * 1e6, 2),
            "flops_per_launch": int(flops_per_launch)}


def timed(step, steps, warmup, hip):
    for w in range(warmup):
        step(w)
    hip.synchronize()
    t0 = time.perf_counter()
    for s in range(steps):
        step(s)
    hip.synchronize()
    return time.perf_counter() - t0


def kernel_avg(ctx, step, reps, names, hip):
    """Average event-timed duration (s) per launch of each named kernel."""
    ctx.timing_reset()
    ctx.timing(True)
    for s in range(reps):
        step(s)
    hip.synchronize()
    ctx.timing(False)
    out = {}
    for name in names:
        ms, cnt = ctx.timing_read(name)
        out[name] = (ms / cnt / 1e3, cnt) if cnt else (None, 0)
    return out


def parity_flat(db, norms, queries, dist, ids, k, metric):
    from oracle import oracle

    od, oi, counts = oracle.flat_search_batch(db, norms, queries, k, metric, threads=CPU_THREADS)
    for i in range(queries.shape[0]):
        kk = int(counts[i])
        if not np.array_equal(od[i, :kk], dist[i, :kk]):
            raise SystemExit(f"parity gate failed: query {i} distances differ from the oracle")
        redo = oracle.distances_for_ids(db, norms, queries[i], ids[i, :kk], metric)
        if not np.array_equal(redo, dist[i, :kk]):
            raise SystemExit(f"parity gate failed: query {i} ids do not carry their distances")


# ---------------------------------------------------------------------------
# Flat exact scan (T1/T2, C2)
# ---------------------------------------------------------------------------

def bench_flat(args, ctx):
    import meltan_amd as M
    from meltan_amd import hip, workloads
    from oracle import oracle

    n, dim, k, B = args.n, 384, 10, args.batch
    metric = M.METRIC_COSINE
    log(f"flat: generating {n} x {dim} mixture corpus")
    nq_pool = max(1024, B)
    db, q = workloads.mixture_1m_384(nq=nq_pool, n=n)
    data_sha = sha(db, q)
    corpus = ctx.upload(db)
    norms = oracle.row_norms(db)
    gd, gi = corpus.flat_search(q[:8], k, metric)
    parity_flat(db, norms, q[:8], gd, gi, k, metric)
    gd, gi = corpus.flat_search(q[:64], k, metric)  # batched path
    parity_flat(db, norms, q[:64], gd, gi, k, metric)
    log("flat: parity gate passed (8 single and 64 batched queries bit-identical to the oracle)")

    dq = hip.DeviceArray.from_numpy(q)
    dd = hip.DeviceArray((nq_pool, k), np.float32)
    di = hip.DeviceArray((nq_pool, k), np.uint32)
    stream = hip.Stream()

    def make_step(b):
        def step(s):
            off = (s * b) % (nq_pool - b + 1)
            corpus.flat_search_device(dq.offset(off * dim), b, k, metric, dd.offset(off * k),
                                      di.offset(off * k), stream.handle)
        return step

    res = {}
    for b, steps, warmup in ((B, args.steps, args.warmup), (1, 200, 20)):
        step = make_step(b)
        elapsed = timed(step, steps, warmup, hip)
        reps = min(steps, 20)
        kt = kernel_avg(ctx, step, reps, ["flat_bound", "flat_gemm", "flat_merge", "flat_scan"], hip)
        if kt["flat_gemm"][1] and kt["flat_bound"][1]:
            # Split-bf16 contraction: two bf16 MFMA products per fp32
            # product (query hi and lo parts against the row's hi part).
            # achieved = algorithmic flops (2 B n d) / launch time against
            # the dense bf16 peak; the issued rate is twice it.
            avg, launches = kt["flat_gemm"]
            flops = 2.0 * (b * reps / launches) * n * dim
            roof = roofline_mfma("flat_gemm_bf16x2<384,cosine,4,bounded>", f"flat_{n}x{dim}_b{b}",
                                 flops, avg, peak=BF16_MFMA_TFLOPS)
            roof["issued_tflops"] = round(2 * flops / avg / 1e12, 2)
            roof["issued_frac"] = round(2 * flops / avg / 1e12 / BF16_MFMA_TFLOPS, 4)
            roof["bound_pass_us"] = round(kt["flat_bound"][0] * 1e6, 2)
            roof["merge_avg_us"] = round(kt["flat_merge"][0] * 1e6, 2) if kt["flat_merge"][1] else None
        elif kt["flat_gemm"][1]:
            avg, launches = kt["flat_gemm"]
            flops = 2.0 * (b * reps / launches) * n * dim  # queries per launch x n x d
            roof = roofline_mfma("flat_gemm_f32<384,cosine>", f"flat_{n}x{dim}_b{b}", flops, avg)
            roof["merge_avg_us"] = round(kt["flat_merge"][0] * 1e6, 2) if kt["flat_merge"][1] else None
        else:
            avg, launches = kt["flat_scan"]
            per = b * reps / max(launches, 1)
            # The event pair brackets the scan and its threshold merge.
            roof = roofline_hbm("flat_scan_f4<6> + flat_fast_merge<6>", f"flat_{n}x{dim}_b{b}",
                                per * n * (dim * 4 + 4), avg)
        res[b] = {"qps": b * steps / elapsed, "ms_per_step": elapsed / steps * 1e3, "steps": steps,
                  "warmup": warmup, "roofline": roof}
        log(f"flat: batch {b}: {res[b]['qps']:.1f} queries/s, {roof['kernel']} "
            f"{roof['achieved']} {roof['unit']} ({roof['frac']:.3f} of peak)")

    extra = {}
    if not args.quick:
        extra["c1"] = bench_single_queries(args, ctx, "c1")
        extra["c2"] = bench_single_queries(args, ctx, "c2")

    cpu = cpu1 = None
    if not args.no_cpu:
        # T2: a batch without a GPU context goes query by query through
        # HostBatchWork.run -- the int8 bounded scan, mode 0, at n >= 16384
        # (FlatGPUSearch.swift:1024-1036) -- across the cores.
        nsample = args.cpu_queries
        log(f"flat: CPU baseline (host batch route) on {nsample} queries, {CPU_THREADS} threads")
        planes = oracle.int8_build(db)
        t0 = time.perf_counter()
        _, _, _, route = oracle.host_batch_search(db, norms, planes, q[:nsample], k, metric,
                                                  cores=CPU_THREADS, threads=CPU_THREADS)
        dt = time.perf_counter() - t0
        del planes
        cpu = cpu_line(nsample / dt, "queries/s", CPU_THREADS,
                       f"{nsample} queries of the same batch workload through HostBatchWork.run "
                       f"(FlatGPUSearch.swift:1003-1037): {int(route.sum())} took the int8 "
                       f"BoundedExactScan (mode 0, adaptive and proven exact), one query per "
                       f"thread; {dt:.2f} s")
        # T1: one query alone, n > 40960 and no GPU: the fp32
        # ParallelFlatScan with min(cores, 32, n / 2048) slices on the cores.
        nq1 = 24
        t0 = time.perf_counter()
        for i in range(nq1):
            oracle.flat_search(db, norms, q[i], k, metric, cores=CPU_THREADS, threads=CPU_THREADS)
        dt = time.perf_counter() - t0
        cpu1 = cpu_line(nq1 / dt, "queries/s", CPU_THREADS,
                        f"{nq1} single queries through ParallelFlatScan.search "
                        f"({min(CPU_THREADS, 32, n // 2048)} slices, FlatGPUSearch.swift:63-94), "
                        f"{dt:.2f} s")
    corpus.release()
    main_b = res[B]
    out = {
        "metric": METRIC,
        "value": round(main_b["qps"], 2),
        "unit": "queries/s",
        "n_gpus": 1,
        "steps": main_b["steps"],
        "warmup": main_b["warmup"],
        "ms_per_step": round(main_b["ms_per_step"], 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (1,000-centre Gaussian mixture, seeded; meltan_amd/workloads.py)",
        "config": {"workload": f"exact flat top-{k} cosine, {n}x{dim} fp32, batch {B}",
                   "n": n, "dim": dim, "k": k, "batch": B, "metric": "cosine"},
        "roofline": main_b["roofline"],
        "cpu_baseline": cpu,
        "batch1": {"qps": round(res[1]["qps"], 2), "ms_per_query": round(res[1]["ms_per_step"], 4),
                   "roofline": res[1]["roofline"], "cpu_baseline": cpu1},
        "data_sha256": {"corpus+queries": data_sha},
    }
    out.update(extra)
    if "c2" in extra:  # the metric's single-query latency at 100k, end to end
        out["p50_us_100k"] = extra["c2"]["p50_us"]
        out["p95_us_100k"] = extra["c2"]["p95_us"]
        out["kernel_p50_us_100k"] = extra["c2"]["kernel_p50_us"]
    return out


def bench_single_queries(args, ctx, which):
    """C1 (10,000 x 384) or C2 (100,000 x 384): exact cosine top-10, one
    query per call.  p50/p95 through the host-pointer C ABI (query upload,
    kernels, results back: PCIe included), the kernel-only p50 (HIP events
    around the scan and its merge, on their stream), and for C2 the batch-32
    and batch-1024 host-API throughput; the CPU baseline is the reference's
    single-query host route on this host."""
    import meltan_amd as M
    from meltan_amd import workloads
    from oracle import oracle

    k, metric = 10, M.METRIC_COSINE
    if which == "c1":
        db, q = workloads.flat_10k(1000)
        desc = "exact flat top-10 cosine, 10000x384, batch 1"
    else:
        db, q = workloads.flat_100k(1024)
        desc = "exact flat top-10 cosine, 100000x384, batch 1 (also 32, 1024)"
    n = db.shape[0]
    c = ctx.upload(db)
    norms = oracle.row_norms(db)
    gd, gi = c.flat_search(q[:4], k, metric)
    parity_flat(db, norms, q[:4], gd, gi, k, metric)
    for i in range(50):
        c.flat_search(q[i:i + 1], k, metric)
    lat = []
    t_all = time.perf_counter()
    for i in range(1000):
        t = time.perf_counter()
        c.flat_search(q[i % q.shape[0]:i % q.shape[0] + 1], k, metric)
        lat.append((time.perf_counter() - t) * 1e6)
    t_all = time.perf_counter() - t_all
    kern = []
    ctx.timing(True)
    for i in range(300):
        ctx.timing_reset()
        c.flat_search(q[i % q.shape[0]:i % q.shape[0] + 1], k, metric)
        ms, cnt = ctx.timing_read("flat_scan")
        if cnt:
            kern.append(ms * 1e3)
    ctx.timing(False)
    p50k = percentile_nearest_rank(kern, 0.5)
    out = {"workload": desc,
           "p50_us": round(percentile_nearest_rank(lat, 0.5), 2),
           "p95_us": round(percentile_nearest_rank(lat, 0.95), 2),
           "qps_host_api": round(1000 / t_all, 1),
           "kernel_p50_us": round(p50k, 2),
           "kernel_roofline": roofline_hbm("flat_scan_f4<6> + flat_fast_merge<6>",
                                           f"flat_{n}x384_b1", n * (384 * 4 + 4), p50k / 1e6),
           "data_sha256": sha(db, q)}
    if which == "c2":
        for b in (32, 1024):
            t = time.perf_counter()
            reps = 10
            for r in range(reps):
                c.flat_search(q[:b], k, metric)
            out[f"qps_batch{b}_host_api"] = round(b * reps / (time.perf_counter() - t), 1)
    if not args.no_cpu:
        # A single query without a GPU context: n < 16384 or n > 40960 takes
        # the fp32 ParallelFlatScan with min(cores, 32, n / 2048) slices
        # (FlatGPUSearch.swift:63-94).
        slices = max(1, min(CPU_THREADS, 32, n // 2048))
        lat_cpu = []
        for i in range(100 if which == "c1" else 40):
            t = time.perf_counter()
            oracle.flat_search(db, norms, q[i], k, metric, cores=CPU_THREADS, threads=slices)
            lat_cpu.append((time.perf_counter() - t) * 1e6)
        out["cpu_baseline"] = cpu_line(
            percentile_nearest_rank(lat_cpu, 0.5), "us p50 per query", slices,
            f"{len(lat_cpu)} single queries through ParallelFlatScan.search, {slices} slices "
            f"on {slices} threads, p50 by nearest rank (LatencyDistribution.swift:154-160)")
        if which == "c2":
            planes = oracle.int8_build(db)
            t0 = time.perf_counter()
            oracle.host_batch_search(db, norms, planes, q[:256], k, metric, cores=CPU_THREADS,
                                     threads=CPU_THREADS)
            out["cpu_baseline_batch"] = cpu_line(
                256 / (time.perf_counter() - t0), "queries/s", CPU_THREADS,
                "256 queries through HostBatchWork.run (int8 BoundedExactScan, mode 0, at "
                "n >= 16384), one query per thread")
    log(f"{which}: p50 {out['p50_us']} us (kernels {out['kernel_p50_us']} us)")
    c.release()
    return out


# ---------------------------------------------------------------------------
# Tier crossover (FlatGPUSearch.swift:31-95, BENCHMARKS.md:193-199)
# ---------------------------------------------------------------------------

def bench_tiers(args, ctx):
    """Single-query latency of the four flat tiers across corpus sizes at
    dim 384, k 24, cosine (the reference's crossover measurement): the
    device fp32 scan and the device int8 bounded scan (mode 0) through the
    host-pointer C ABI (query upload and results back included), and the
    host fp32 ParallelFlatScan and host int8 BoundedExactScan restated in
    the oracle (the CPU baselines of those tiers, 16 host threads).  p50 by
    nearest rank; the crossovers are where one tier's p50 drops below
    another's."""
    import meltan_amd as M
    from meltan_amd import workloads
    from oracle import oracle

    dim, k, metric = 384, 24, M.METRIC_COSINE
    sizes = [128, 256, 512, 1024, 4096, 16384, 20480, 24576, 32768, 50000, 100000, 262144,
             400000, 600000, 800000, 1000000]
    log("tiers: generating 1,000,000 x 384 N(0,1) normalised rows (prefixes per size)")
    db_all = workloads.gauss_rows(1001, sizes[-1], dim, True)
    q = workloads.gauss_rows(1002, 64, dim, True)
    rows = []
    for n in sizes:
        db = db_all[:n]
        c = ctx.upload(db)
        norms = oracle.row_norms(db)

        def p50(fn, reps):
            lat = []
            for i in range(reps):
                t = time.perf_counter()
                fn(i % q.shape[0])
                lat.append((time.perf_counter() - t) * 1e6)
            return round(percentile_nearest_rank(lat, 0.5), 2)

        for i in range(20):
            c.flat_search(q[i:i + 1], k, metric)
        row = {"n": n, "gpu_fp32_us": p50(lambda i: c.flat_search(q[i:i + 1], k, metric), 300)}
        if n >= 16384:
            for i in range(10):
                c.int8_search(q[i:i + 1], k, metric, mode=0)
            row["gpu_int8_us"] = p50(lambda i: c.int8_search(q[i:i + 1], k, metric, mode=0), 200)
        if not args.no_cpu:
            slices = max(1, min(CPU_THREADS, 32, n // 2048))
            row["host_fp32_us"] = p50(lambda i: oracle.flat_search(
                db, norms, q[i], k, metric, cores=CPU_THREADS, threads=slices),
                40 if n <= 100000 else 10)
            row["host_fp32_threads"] = slices
            if n >= 16384:
                planes = oracle.int8_build(db)
                row["host_int8_us"] = p50(lambda i: oracle.int8_search(
                    db, norms, planes, q[i], k, metric, cores=CPU_THREADS, mode=0),
                    20 if n <= 100000 else 4)
                del planes
        rows.append(row)
        log(f"tiers: n {n}: " + ", ".join(f"{a} {b}" for a, b in row.items() if a != "n"))
        c.release()

    def first(pred):
        for r in rows:
            if pred(r):
                return r["n"]
        return None

    cross = {"gpu_fp32_below_host_fp32_from_n": first(
        lambda r: "host_fp32_us" in r and r["gpu_fp32_us"] < r["host_fp32_us"]),
        "gpu_int8_below_gpu_fp32_from_n": first(
        lambda r: "gpu_int8_us" in r and r["gpu_int8_us"] < r["gpu_fp32_us"])}
    return {"workload": f"single-query tiers, exact top-{k} cosine, dim {dim}, N(0,1) rows",
            "rows": rows, "crossover": cross}


# ---------------------------------------------------------------------------
# int8 prefilter + fp32 rerank (C3)
# ---------------------------------------------------------------------------

def bench_int8(args, ctx):
    """C3: the int8 prefilter + fp32 rerank at 1M x 384, batch 1 and 1024,
    in both modes: mode 1 (the configuration's literal form: top-100 by the
    int8 keys, then the exact top-10 of those) and mode 0 (the reference's
    BoundedExactScan: adaptive budget with the lower-bound proof, exact)."""
    import meltan_amd as M
    from meltan_amd import hip, workloads
    from oracle import oracle

    n, dim, k, budget = 1_000_000, 384, 10, 100
    metric = M.METRIC_COSINE
    log("int8: 1M x 384 mixture, top-100 prefilter then rerank to top-10")
    db, q = workloads.mixture_1m_384(nq=1024, n=n)
    corpus = ctx.upload(db)
    norms = oracle.row_norms(db)
    planes = oracle.int8_build(db)
    for mode in (1, 0):
        gd, gi, _ = corpus.int8_search(q[:2], k, metric, mode=mode, budget=budget)
        bd, bi, _ = corpus.int8_search(q[:64], k, metric, mode=mode, budget=budget)
        for i in range(2):
            od, oi, _ = oracle.int8_search(db, norms, planes, q[i], k, metric, cores=CPU_THREADS,
                                           mode=mode, budget=budget)
            for rd, ri in ((gd, gi), (bd, bi)):
                if not np.array_equal(rd[i, :len(od)], od):
                    raise SystemExit(f"int8 parity gate failed (mode {mode})")
                if mode == 1 and not np.array_equal(ri[i, :len(oi)], oi):
                    raise SystemExit("int8 parity gate failed (mode 1 ids)")
    cpu = {}
    if not args.no_cpu:
        # The reference's CPU int8 path is BoundedExactScan (mode 0); the
        # oracle's restatement scans a query on one thread.
        t0 = time.perf_counter()
        for i in range(8):
            oracle.int8_search(db, norms, planes, q[i], k, metric, cores=CPU_THREADS, mode=0)
        dt = time.perf_counter() - t0
        cpu[1] = cpu_line(8 / dt, "queries/s", 1,
                          f"8 single queries through BoundedExactScan.search (mode 0) restated, "
                          f"one thread per query, {dt:.2f} s")
        t0 = time.perf_counter()
        oracle.host_batch_search(db, norms, planes, q[:128], k, metric, cores=CPU_THREADS,
                                 threads=CPU_THREADS)
        dt = time.perf_counter() - t0
        cpu[1024] = cpu_line(128 / dt, "queries/s", CPU_THREADS,
                             f"128 queries through HostBatchWork.run (BoundedExactScan, mode 0), "
                             f"one query per thread, {dt:.2f} s")
    del planes
    dq = hip.DeviceArray.from_numpy(q)
    dd = hip.DeviceArray((1024, k), np.float32)
    di = hip.DeviceArray((1024, k), np.uint32)
    stream = hip.Stream()
    out = {"workload": f"int8 prefilter top-{budget} + exact rerank top-{k}, cosine, {n}x{dim}",
           "data_sha256": sha(db, q)}
    for mode in (1, 0):
        for b, steps in ((1, 100), (1024, 10)):
            def step(s, b=b, mode=mode):
                off = (s * b) % (1024 - b + 1)
                corpus.int8_search_device(dq.offset(off * dim), b, k, metric, mode, budget,
                                          dd.offset(off * k), di.offset(off * k), stream.handle)
            elapsed = timed(step, steps, 2, hip)
            kt = kernel_avg(ctx, step, min(steps, 10),
                            ["int8_scan", "int8_bound", "int8_gemm", "int8_merge"], hip)
            if (b == 1 and not kt["int8_scan"][1]) or (b > 1 and not kt["int8_gemm"][1]):
                roof = None
            elif b == 1:
                # The collect launch streams every row's codes and planes once;
                # the bound launch before it reads a sixteenth of them.
                # Bytes of one launch: every row's codes and planes (a
                # mode-0 query may take several launches, one per round).
                avg, launches = kt["int8_scan"]
                roof = roofline_hbm("int8_collect<6>", f"int8_{n}x{dim}_b{b}", n * (dim + 12), avg)
                roof["launches_per_query"] = round(launches / min(steps, 10), 2)
                roof["bound_pass_us"] = round(kt["int8_bound"][0] * 1e6, 2) if kt["int8_bound"][1] else None
            else:
                # The batch is a 1024 x 1e6 x 384 int8 contraction on i8 MFMA
                # (dense peak 5.0 POP/s) with the key epilogue fused into it.
                avg, launches = kt["int8_gemm"]
                ops = 2.0 * b * n * dim
                roof = {"bound": "mfma", "achieved": round(ops / avg / 1e12, 2), "peak": 5000.0,
                        "unit": "TOP/s", "frac": round(ops / avg / 1e12 / 5000.0, 5),
                        "traffic": measured_traffic("int8_gemm<12>", f"int8_{n}x{dim}_b{b}"),
                        "kernel": "int8_gemm<12,cosine,bounded>", "avg_launch_us": round(avg * 1e6, 2),
                        "ops_per_launch": int(ops),
                        "bound_pass_us": round(kt["int8_bound"][0] * 1e6, 2) if kt["int8_bound"][1] else None,
                        "merge_avg_us": round(kt["int8_merge"][0] * 1e6, 2) if kt["int8_merge"][1] else None,
                        "scan_launches": kt["int8_scan"][1], "gemm_launches": launches}
            key = f"batch{b}" if mode == 1 else f"mode0_batch{b}"
            out[key] = {"qps": round(b * steps / elapsed, 1), "roofline": roof,
                        "mode": "fixed budget 100, no proof" if mode == 1 else
                                "adaptive budget with the lower-bound proof (exact)",
                        "cpu_baseline": cpu.get(b)}
            log(f"int8: mode {mode} batch {b}: {out[key]['qps']} queries/s")
    corpus.release()
    return out


# ---------------------------------------------------------------------------
# IVF-flat (C4)
# ---------------------------------------------------------------------------

def bench_ivf(args, ctx):
    import meltan_amd as M
    from meltan_amd import hip, workloads
    from oracle import oracle

    n, dim, nlist, k, B = 1_000_000, 128, 4096, 10, 1024
    log("ivf: 1M x 128 mixture, device k-means (10 iterations), nlist 4096")
    db, q = workloads.mixture_1m_128(nq=B)
    corpus = ctx.upload(db)
    t = time.perf_counter()
    cents = corpus.kmeans(nlist, 10, M.METRIC_L2)
    t_km = time.perf_counter() - t
    t = time.perf_counter()
    ivf = corpus.ivf_flat_build(cents, M.METRIC_L2)
    t_build = time.perf_counter() - t
    off, ids = ivf.lists()
    sizes = np.diff(off)
    part = oracle.IVFPartition.__new__(oracle.IVFPartition)
    part.metric, part.dim, part.count, part.nlist = M.METRIC_L2, dim, n, nlist
    part.centroids, part.cnorms = cents, oracle.row_norms(cents)
    part.offsets, part.list_ids = off, ids
    part.packed = np.ascontiguousarray(db[ids])
    part.packed_norms = oracle.row_norms(part.packed)
    dq = hip.DeviceArray.from_numpy(q)
    dd = hip.DeviceArray((B, k), np.float32)
    di = hip.DeviceArray((B, k), np.uint32)
    stream = hip.Stream()
    out = {"workload": f"IVF-flat L2 top-{k}, {n}x{dim}, nlist {nlist}, batch {B}",
           "kmeans_s": round(t_km, 3), "build_s": round(t_build, 3),
           "data_sha256": sha(db, q)}
    for nprobe in (4, 8, 32):
        gd, gi, gp = ivf.search(q, k, nprobe, want_probes=True)
        for i in (0, 1):
            od, oi, op = part.search(q[i], k, nprobe)
            if not (np.array_equal(gp[i], op) and np.array_equal(gd[i, :len(od)], od)):
                raise SystemExit("IVF parity gate failed")
        cand_rows = int(sum(sizes[gp[i]].sum() for i in range(B)))
        probed = np.unique(gp[:B].ravel())
        list_rows = int(sizes[probed].sum())

        def step(s, nprobe=nprobe):
            ivf.search_device(dq.ptr, B, k, nprobe, dd.ptr, di.ptr, stream.handle)
        elapsed = timed(step, 5, 1, hip)
        kt = kernel_avg(ctx, step, 3, ["ivf_probe", "ivf_lm", "ivf_scan"], hip)
        # The list-major scan reads every probed list once per batch: its
        # algorithmic bytes are the distinct probed lists' rows, norms and
        # ids; it forms cand_rows (query, row) dots of 2 dim flop each.
        avg, _ = kt["ivf_lm"]
        roof = roofline_hbm("ivf_lm_scan<2> + ivf_lm_merge<2>", f"ivf_{n}x{dim}_np{nprobe}_b{B}",
                            list_rows * (dim * 4 + 4 + 4), avg)
        roof["pair_tflops"] = round(2.0 * dim * cand_rows / avg / 1e12, 2)
        roof["probe_pass_us"] = round(kt["ivf_probe"][0] * 1e6, 2) if kt["ivf_probe"][1] else None
        # The rest of the call: the kernels that group the (query, probe)
        # pairs by list, the status read and any proof retries.
        roof["outside_scan_us"] = (round((kt["ivf_scan"][0] - avg) * 1e6, 2)
                                   if kt["ivf_scan"][1] else None)
        out[f"nprobe{nprobe}"] = {
            "qps": round(B * 5 / elapsed, 1),
            "candidates_per_query": round(cand_rows / B, 1),
            "distinct_lists": int(probed.size),
            "roofline": roof}
        if not args.no_cpu:
            # IVFFlatSearch.search per query (scanProbedLists,
            # IVFFlatSearch.swift:214-291) over the same lists, queries
            # spread over the cores.
            import concurrent.futures as cf

            t0 = time.perf_counter()
            with cf.ThreadPoolExecutor(CPU_THREADS) as ex:
                list(ex.map(lambda i: part.search(q[i], k, nprobe), range(B)))
            dt = time.perf_counter() - t0
            out[f"nprobe{nprobe}"]["cpu_baseline"] = cpu_line(
                B / dt, "queries/s", CPU_THREADS,
                f"{B} queries through scanProbedLists restated (probes, exact dots.c-order "
                f"scan of the probed lists, (distance, id) top-k), one query per thread, "
                f"{dt:.2f} s")
        log(f"ivf: nprobe {nprobe}: {out[f'nprobe{nprobe}']['qps']} queries/s")
    ivf.release()
    corpus.release()
    return out


# ---------------------------------------------------------------------------
# IVF-PQ (C5)
# ---------------------------------------------------------------------------

def bench_ivfpq(args, ctx):
    import meltan_amd as M
    from meltan_amd import hip, workloads
    from oracle import oracle

    n = args.pq_n
    dim, nlist, m, nprobe, kadc, rer, B = 96, 8192, 48, 16, 100, 10, 1024
    log(f"ivfpq: {n} x 96 mixture, nlist {nlist}, M {m} x 8 bit, nprobe {nprobe}")
    db, q, _ = workloads.mixture_10m_96(nq=B, n=n)
    data_sha = sha(db, q)
    train = workloads.mixture_10m_96_train()
    tc = ctx.upload(train)
    t = time.perf_counter()
    coarse, books = tc.ivfpq_train(nlist, m, args.pq_iters, M.METRIC_INNER_PRODUCT)
    t_train = time.perf_counter() - t
    tc.release()
    corpus = ctx.upload(db)
    t = time.perf_counter()
    pq = corpus.ivfpq_build(coarse, books, M.METRIC_INNER_PRODUCT)
    t_build = time.perf_counter() - t
    gs, gi = pq.search(q[:4], kadc, nprobe, rerank_k=rer)
    codes, assign = pq.codes()
    offsets, ids = oracle.ivf_lists(assign, nlist)
    for i in range(4):
        os_, oi = oracle.ivfpq_search(coarse, books, codes, offsets, ids, M.METRIC_INNER_PRODUCT, q[i], kadc,
                                      nprobe, rows=db, rerank_k=rer)
        if not (np.array_equal(gs[i], os_) and np.array_equal(gi[i], oi)):
            raise SystemExit("IVF-PQ parity gate failed")
    # recall@10 of the reranked results against the exact inner-product top-10
    nrec = 256
    _, exact = corpus.flat_search(q[:nrec], rer, M.METRIC_INNER_PRODUCT)
    _, got = pq.search(q[:nrec], kadc, nprobe, rerank_k=rer)
    recall = float(np.mean([len(set(got[i]) & set(exact[i])) / rer for i in range(nrec)]))
    cpu = {}
    if not args.no_cpu:
        import concurrent.futures as cf

        ncpu = 1024
        for rr in (0, rer):
            t0 = time.perf_counter()
            with cf.ThreadPoolExecutor(CPU_THREADS) as ex:
                list(ex.map(lambda i: oracle.ivfpq_search(
                    coarse, books, codes, offsets, ids, M.METRIC_INNER_PRODUCT, q[i], kadc, nprobe,
                    rows=db if rr else None, rerank_k=rr), range(ncpu)))
            dt = time.perf_counter() - t0
            cpu[rr] = cpu_line(ncpu / dt, "queries/s", CPU_THREADS,
                               f"{ncpu} queries through _IVFPQIndex.search restated (probes, "
                               f"residual LUTs, sequential ADC, BoundedSortedList)"
                               f"{' plus the exact rerank' if rr else ''}, one query per thread, "
                               f"{dt:.2f} s")
    sizes = np.diff(offsets)
    probes = [oracle.ivfpq_probe(coarse, q[i], nprobe, M.METRIC_INNER_PRODUCT)[0] for i in range(B)]
    cand_per_query = float(np.mean([sizes[p].sum() for p in probes]))
    del codes, db
    dq = hip.DeviceArray.from_numpy(q)
    dd = hip.DeviceArray((B, kadc), np.float32)
    di = hip.DeviceArray((B, kadc), np.uint32)
    stream = hip.Stream()
    out = {"workload": f"IVF-PQ ADC IP, {n}x{dim}, nlist {nlist}, M {m}, nprobe {nprobe}, "
                       f"top-{kadc} then exact rerank to {rer}, batch {B}",
           "training": f"mans_ivfpq_train on 262,144 mixture rows (seed 5003), {args.pq_iters} "
                       f"iterations (coarse and per subspace), inner product",
           "train_s": round(t_train, 3), "build_s": round(t_build, 3),
           "candidates_per_query": round(cand_per_query, 1),
           f"recall@{rer}_nprobe{nprobe}": round(recall, 4),
           "data_sha256": data_sha}
    for rerank in (0, rer):
        def step(s, rerank=rerank):
            pq.search_device(dq.ptr, B, kadc, nprobe, rerank, dd.ptr, di.ptr, stream.handle)
        elapsed = timed(step, 5, 1, hip)
        kt = kernel_avg(ctx, step, 3, ["ivfpq_probe", "ivfpq_scan"], hip)
        avg, _ = kt["ivfpq_scan"]
        key = "adc_rerank" if rerank else "adc"
        # The event pair brackets the scan launch (with its work-item plan);
        # the probe selection before it is timed on its own.
        roof = roofline_hbm("ivfpq_scan", f"ivfpq_{n}x{dim}_b{B}", B * cand_per_query * (m + 4), avg)
        roof["probe_pass_us"] = round(kt["ivfpq_probe"][0] * 1e6, 2) if kt["ivfpq_probe"][1] else None
        out[key] = {"qps": round(B * 5 / elapsed, 1), "roofline": roof, "cpu_baseline": cpu.get(rerank)}
        log(f"ivfpq: {key}: {out[key]['qps']} queries/s")
    pq.release()
    corpus.release()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--batch", type=int, default=1024)
    ap.add_argument("--n", type=int, default=1_000_000)
    ap.add_argument("--pq-n", type=int, default=10_000_000)
    ap.add_argument("--pq-iters", type=int, default=20,
                    help="IVF-PQ training iterations (IVFPQConfiguration's default is 20)")
    ap.add_argument("--workload", default="flat", choices=["flat", "int8", "ivf", "ivfpq", "tiers"])
    ap.add_argument("--quick", action="store_true", help="flat only, no 100k or per-config extras")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-queries", type=int, default=128)
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="first copy MIB MiB device to device (a plain copy kernel of known size, "
                         "the scale for rocprofv3 FETCH_SIZE / WRITE_SIZE counts)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: every scan here runs on a single MI355X and this build "
              "has no multi-GPU path; the sharded design is documented alongside the code.",
              file=sys.stderr)
        sys.exit(2)
    import meltan_amd as M

    ctx = M.Context(0)
    if args.calibrate_copy > 0:
        from meltan_amd import hip

        nb = args.calibrate_copy << 20
        src, dst = hip.DeviceArray(nb, np.uint8), hip.DeviceArray(nb, np.uint8)
        dst.copy_from(src)
        hip.synchronize()
        log(f"calibration copy: {nb} bytes device to device")
        src.free()
        dst.free()
    if args.workload == "flat":
        out = bench_flat(args, ctx)
        if not args.quick:
            for name, fn in (("int8", bench_int8), ("ivf", bench_ivf), ("ivfpq", bench_ivfpq)):
                try:
                    out[name] = fn(args, ctx)
                except SystemExit:
                    raise
                except Exception as exc:  # a failed extra must not hide the main line
                    out[name] = {"error": f"{type(exc).__name__}: {exc}"}
    else:
        fn = {"int8": bench_int8, "ivf": bench_ivf, "ivfpq": bench_ivfpq,
              "tiers": bench_tiers}[args.workload]
        out = {"metric": METRIC, "workload": args.workload}
        out.update(fn(args, ctx))
    print(json.dumps(out), flush=True)


if __name__ == "__main__":
    main()
