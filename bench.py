#!/usr/bin/env python3
"""Headline benchmark of the wmma_ops MI355X hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu]

Metric: "FP16 GEMM TFLOPS (% MFMA peak) @4096^3; W4A16 M=1 HBM GB/s".
A step is one wmma_ops_amd.matmul of the 4096^3 FP16 GEMM: A[4096,4096] and
B[4096,4096] fp16 ~ N(0,1) (seed 43), fp32 output, inputs resident in HBM.  W warmup
steps, then K timed steps between two synchronisations; `value` = 2*M*N*K / time.
The W4A16 M=1 decode figures (configs[3], K=4096, N in {4096, 14336}, G=128) ride along
in the same JSON line: weights rotate over > 512 MB so the 256 MB MALL cannot hold them,
and launches are replayed from a HIP graph so the figure is kernel time, not host
dispatch.  The CPU baseline (rank 0, N=1) is the oracle's fp32 torch.matmul on the host
cores over a bounded sample of the same 4096^3 workload.

Prints ONE JSON line.  One GPU only: --gpus N with N > 1 exits with a message.
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

PEAK_FP16_FLOPS = 2.5e15   # MI355X dense FP16 MFMA (published)
PEAK_HBM_BPS = 8.0e12      # MI355X HBM3E (published)
M = N = K = 4096
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_f16f32_4096_traffic.json")


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-w4a16", action="store_true", help="skip the W4A16 decode figures")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    return ap.parse_args()


def time_events(fn, reps):
    """Mean duration (ms) of fn() measured with one event pair per launch on the current
    stream (the stream the C-ABI launches on)."""
    import torch

    pairs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
             for _ in range(reps)]
    for s, e in pairs:
        s.record()
        fn()
        e.record()
    torch.cuda.synchronize()
    return statistics.mean(s.elapsed_time(e) for s, e in pairs)


def gemm_bench(wo, steps, warmup):
    import torch

    g = torch.Generator().manual_seed(42 + 1)
    A = torch.randn(M, K, generator=g).half().cuda()
    B = torch.randn(K, N, generator=g).half().cuda()
    for _ in range(warmup):
        wo.matmul(A, B)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        C = wo.matmul(A, B)
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / steps
    ms_kernel = time_events(lambda: wo.matmul(A, B), max(steps, 20))
    # parity spot check of the benchmarked output (a 256-row slab against the fp32 CPU oracle)
    from oracle import gemm as og

    err = og.max_rel_err(C[:256], og.gemm_ref(A[:256].cpu(), B.cpu()))
    return ms_step, ms_kernel, err


def w4a16_bench(wo, Nw):
    """M=1 W4A16 decode: graph-replayed launches over rotating weight copies (> 512 MB)."""
    import numpy as np
    import torch

    from oracle import gemm as og
    from oracle import int4 as oi

    Kw, G = 4096, 128
    A, q, s, z = oi.make_inputs(1, Kw, Nw, G, seed=42 + 3)
    pk0 = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    sd = torch.from_numpy(s).cuda()
    zd = torch.from_numpy(oi.pack_zeros(z)).cuda()
    Ad = A.cuda()
    algo_bytes = Kw * Nw // 2 + (Kw // G) * Nw * 2 + (Kw // G) * Nw // 2 + 2 * Kw + 4 * Nw
    copies = max(2, math.ceil(600e6 / algo_bytes))
    pks = [pk0.clone() for _ in range(copies)]
    sds = [sd.clone() for _ in range(copies)]
    zds = [zd.clone() for _ in range(copies)]
    Y0 = wo.matmul_int4(Ad, pk0, sd, zd, G)
    err = og.max_rel_err(Y0, oi.w4a16_ref(A, q, s, z, G))
    torch.cuda.synchronize()
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(3):  # warm the allocator on the side stream before capture
            wo.matmul_int4(Ad, pks[i % copies], sds[i % copies], zds[i % copies], G)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    outs = []
    with torch.cuda.graph(graph):
        for i in range(copies):
            outs.append(wo.matmul_int4(Ad, pks[i], sds[i], zds[i], G))
    graph.replay()
    torch.cuda.synchronize()
    assert torch.equal(outs[0], Y0), "graph replay differs from eager"
    reps = 5
    ts = []
    for _ in range(reps):
        s0, e0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        graph.replay()
        e0.record()
        torch.cuda.synchronize()
        ts.append(s0.elapsed_time(e0) / copies)
    assert torch.equal(outs[-1], outs[0]), "graph replays differ"
    ms = statistics.median(ts)
    return {"N": Nw, "K": Kw, "G": G, "bytes": algo_bytes, "us_per_call": round(ms * 1e3, 3),
            "GBps": round(algo_bytes / (ms * 1e-3) / 1e9, 1),
            "hbm_frac": round(algo_bytes / (ms * 1e-3) / PEAK_HBM_BPS, 4),
            "rotation_copies": copies, "max_rel_err": float(f"{err:.3e}")}


def cpu_baseline(seconds):
    """The oracle's fp32 torch.matmul on host cores, on a bounded sample of 4096^3 calls."""
    import torch

    from oracle import gemm as og

    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    g = torch.Generator().manual_seed(42 + 1)
    A = torch.randn(M, K, generator=g).half()
    B = torch.randn(K, N, generator=g).half()
    og.gemm_ref(A, B)  # warm-up
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        og.gemm_ref(A, B)
        times.append(time.perf_counter() - t0)
        if len(times) >= 50:
            break
    t = statistics.median(times)
    return {"value": round(2.0 * M * N * K / t / 1e12, 4), "unit": "TFLOPS", "cores": threads,
            "kind": "port",
            "sample": f"{len(times)} calls of torch.matmul(A.float(), B.float()) at 4096^3 "
                      f"(oracle.gemm.gemm_ref), median {t * 1e3:.1f} ms"}


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); every GPU box "
              "in this build has one MI355X. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    import wmma_ops_amd as wo

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    ms_step, ms_kernel, err = gemm_bench(wo, args.steps, args.warmup)
    flops = 2.0 * M * N * K
    tflops = flops / (ms_step * 1e-3) / 1e12
    achieved = flops / (ms_kernel * 1e-3) / 1e12
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    line = {
        "metric": "FP16 GEMM TFLOPS (% MFMA peak) @4096^3; W4A16 M=1 HBM GB/s",
        "value": round(tflops, 2),
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16",
        "data": "synthetic (seeded N(0,1) fp16 inputs, fp32 output)",
        "config": {"workload": "fp16 GEMM C[4096,4096] fp32 = A[4096,4096] @ B[4096,4096] "
                               "(configs[1], wmma_ops_amd.matmul)",
                   "M": M, "N": N, "K": K, "plan": wo.gemm_plan(M, N, K)},
        "pct_mfma_peak": round(100.0 * tflops * 1e12 / PEAK_FP16_FLOPS, 2),
        "max_rel_err": float(f"{err:.3e}"),
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_FP16_FLOPS / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved * 1e12 / PEAK_FP16_FLOPS, 4), "traffic": traffic,
                     "kernel": "gemm_tiled_kernel<256,256,2,2,true>",
                     "kernel_us": round(ms_kernel * 1e3, 2)},
    }
    if not args.no_w4a16:
        line["w4a16_m1"] = [w4a16_bench(wo, n) for n in (4096, 14336)]
    if not args.no_cpu:
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
