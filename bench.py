#!/usr/bin/env python3
"""Benchmarks of the wmma_ops MI355X hot path.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-w4a16]
    python bench.py --workload NAME      # one JSON line per case of one config family
    python bench.py --suite              # every config family (one JSON line per case)

Default run (the driver's contract): ONE JSON line for the headline metric of
BASELINE.json, "FP16 GEMM TFLOPS (% MFMA peak) @4096^3; W4A16 M=1 HBM GB/s".
A step is one wmma_ops_amd.matmul of the 4096^3 FP16 GEMM: A[4096,4096] and
B[4096,4096] fp16 ~ N(0,1) (seed 42 + 1), fp32 output, inputs resident in HBM.  The same
step first runs for 100 ms of GPU time (the clock ramps up under sustained load: timed
from idle, the first tens of launches run 10-15% slower), then W warmup steps, then K
timed steps between two synchronisations; `value` = 2*M*N*K / time.
`roofline.achieved` divides the same FLOPs by the kernel's mean duration measured with
HIP events on the stream the kernel is launched on (the current stream).  The W4A16 M=1
decode figures (configs[3], K=4096, N in {4096, 14336}, G=128) ride along in the same
line, each with the time a plain streaming read of the same byte count takes in its
fastest launch shape in the same run (`read_floor`); the CPU baseline (N=1 only) is the oracle on the host cores over bounded samples
of the same workloads: fp32 torch.matmul at 4096^3 (`value`), the W4A16 M=1 dequant +
matmul at N=14336, and fp32 SDPA on 2 heads of configs[4].

Workload families (--workload):
  gemm       configs[0..1]: M=N=K in {512,1024,2048,4096} and 4096x4096x2048
  epilogue   configs[1]: C = 2.0*A@B + 0.5*C, out-of-place and in-place, 1024^3/4096^3
  skinny     configs[2]: M in {1,16,64,128} x N in {4096,11008,14336}, K=4096; K=14336,N=4096;
             and M=32 on the same shapes
  ragged     N or K off a multiple of 8 (4096x4100x4096, 2048x32001x4096, M = 1..4096): the
             repacked product path, the element-wise in-place path and the aligned neighbour
             shape; shapes off the 256 grid (M = 4100..8200, N = 4352..14336): the planner's
             two-part plans against one launch -- in one process (inputs not rotated)
  w4a16      configs[3]: M in {1,16,128,2048} x N in {4096,14336}, K=4096, G=128
  flash      configs[4]: [4,32,4096,128], causal and non-causal, forward and backward; with
             8 K/V heads (GQA); head dims 64 and 256; a packed variable-length batch
  flash_operands  configs[4] non-causal forward and backward on all-ones inputs (the power
             limit's share of the random-input figures)
  decode     flash attention with 1-16 queries against 4096-32768 keys (MHA and 8 K/V heads,
             D 128 / 256): the split-key-range forward against the one-pass forward
  bwd_gqa    flash-attention backward with 4-8 K/V heads at 1024-4096 tokens: the
             grouped-query split of the dK/dV kernel against the unsplit backward
  copy       a plain 256 MiB device copy (calibrates the rocprofv3 byte counters)
  mfma_ceiling  the matrix pipe's sustained rate with register operands and no memory
             traffic (libwmma_calib.so): the ceiling the GEMM main loop is held against;
             and the 4096^3 GEMM itself on random and on constant operands
  lds_read   the LDS read rate of ds_read_b128 and ds_read_b64_tr_b16 (contiguous and in the
             flash forward's V-fragment pattern), the LDS side of the MFMA kernels
  l2_read    the activation stage of the small-M LDS-DMA GEMMs alone: 64-row x 128-byte
             blocks from L2 into LDS, 4 or 8 waves, 7, 3 or no blocks in flight
  read_floor a plain streaming read of the W4A16 M=1 weight sizes and of 1 GiB in several
             launch shapes, graph replayed over rotating buffers: the floor of the
             HBM-bound kernels (the fastest shape)
  vendor     torch.mm (hipBLASLt/rocBLAS, fp32 and fp16 output) and torch's flash SDPA on
             the same shapes, for comparison
HBM-bound cases rotate their inputs over more than 512 MB (twice the 256 MB MALL) so the
bytes really come from HBM; microsecond-scale kernels are replayed from a HIP graph.

One GPU only: --gpus N with N > 1 exits with a message.
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
ROTATE_BYTES = 600e6       # > 2 x 256 MB MALL
M = N = K = 4096
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "gemm_f16f32_4096_traffic.json")
METRIC = "FP16 GEMM TFLOPS (% MFMA peak) @4096^3; W4A16 M=1 HBM GB/s"
TILE_NAMES = ["64x64", "128x64", "256x64", "128x128", "256x128", "256x256"]


def parse():
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[1])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--no-w4a16", action="store_true", help="skip the W4A16 decode figures")
    ap.add_argument("--cpu-seconds", type=float, default=12.0)
    ap.add_argument("--workload", choices=sorted(FAMILIES), help="one config family")
    ap.add_argument("--suite", action="store_true", help="every config family")
    ap.add_argument("--quick", action="store_true",
                    help="with --workload/--suite: two calls per case, no settle phase and no "
                         "graph capture -- for rocprofv3 counter passes; its times are not "
                         "the benchmark")
    return ap.parse_args()


# ---------------------------------------------------------------------------- timing --
SETTLE_MS = 100.0  # sustained load before any timing: the GPU's clock ramps up over ~50 ms
QUICK = False      # --quick: few launches per case (counter collection), see parse()


def settle(fn, ms=SETTLE_MS):
    """Runs fn(i) back to back until `ms` of GPU time have passed, so that the timed calls
    that follow see the clock a sustained workload runs at, not the idle one."""
    import torch

    if QUICK:
        return
    spent, i = 0.0, 0
    while spent < ms:
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for _ in range(16):
            fn(i)
            i += 1
        e.record()
        e.synchronize()
        spent += s.elapsed_time(e)


def time_batches(fn, calls, batches=5):
    """Median over `batches` of (event-timed batch of `calls` back-to-back calls)/calls,
    in ms.  fn(i) runs call i (so inputs can rotate)."""
    import torch

    if QUICK:
        calls, batches = min(calls, 2), 1
    settle(fn)
    torch.cuda.synchronize()
    out = []
    for _ in range(batches):
        s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s.record()
        for i in range(calls):
            fn(i)
        e.record()
        torch.cuda.synchronize()
        out.append(s.elapsed_time(e) / calls)
    return statistics.median(out)


def time_graph(fn, copies, batches=5):
    """Per-call time (ms) of `copies` calls fn(0..copies-1) captured in one HIP graph and
    replayed `batches` times (median); returns (ms, outputs of the captured calls)."""
    import torch

    if QUICK:  # no capture: counter passes see plain launches
        return time_batches(fn, 2), [fn(0)]
    stream = torch.cuda.Stream()
    stream.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(stream):
        for i in range(min(copies, 3)):
            fn(i)
    torch.cuda.current_stream().wait_stream(stream)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    outs = []
    with torch.cuda.graph(graph):
        for i in range(copies):
            outs.append(fn(i))
    graph.replay()
    torch.cuda.synchronize()
    settle(lambda i: graph.replay())
    ts = []
    for _ in range(batches):
        s0, e0 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        s0.record()
        graph.replay()
        e0.record()
        torch.cuda.synchronize()
        ts.append(s0.elapsed_time(e0) / copies)
    return statistics.median(ts), outs


def line(**kw):
    print(json.dumps(kw), flush=True)


class ClockSampler:
    """Samples the GPU's current gfx clock (MHz) and socket power (W) from the SMU's metrics
    table (amdsmi, `current_gfxclk` / `current_socket_power`) every ~5 ms on a host thread
    while the block runs.  `summary()` gives the medians over the samples, or None when
    amdsmi is not available (the field is then null in the JSON)."""

    def __init__(self, device_index=0):
        self.samples = []
        self._stop = False
        self._h = None
        try:
            import amdsmi

            amdsmi.amdsmi_init()
            self._smi = amdsmi
            self._h = amdsmi.amdsmi_get_processor_handles()[device_index]
        except Exception:  # noqa: BLE001 - optional instrumentation
            self._h = None

    def _run(self):
        while not self._stop:
            try:
                m = self._smi.amdsmi_get_gpu_metrics_info(self._h)
                clk, pw = m.get("current_gfxclk"), m.get("current_socket_power")
                if isinstance(clk, (int, float)):
                    self.samples.append((float(clk), float(pw) if isinstance(pw, (int, float)) else None))
            except Exception:  # noqa: BLE001
                pass
            time.sleep(0.005)

    def __enter__(self):
        import threading

        if self._h is not None:
            self._t = threading.Thread(target=self._run, daemon=True)
            self._t.start()
        return self

    def __exit__(self, *exc):
        self._stop = True
        if self._h is not None:
            self._t.join()
        return False

    def summary(self):
        if not self.samples:
            return None
        clk = statistics.median(c for c, _ in self.samples)
        pw = [p for _, p in self.samples if p is not None]
        return {"sclk_MHz": clk, "socket_power_W": statistics.median(pw) if pw else None,
                "samples": len(self.samples)}


def sustained_clock(fn, seconds=0.6):
    """The gfx clock and socket power a sustained run of fn(i) holds: fn back to back for
    `seconds` after the settle phase, sampled by ClockSampler (medians)."""
    import torch

    settle(fn)
    with ClockSampler() as cs:
        t_end = time.perf_counter() + seconds
        i = 0
        while time.perf_counter() < t_end:
            for _ in range(32):
                fn(i)
                i += 1
            torch.cuda.synchronize()
    return cs.summary()


def roofline(nbytes, flops, ms):
    """The binding roofline of a case: the larger of its HBM time (bytes / 8 TB/s) and its
    matrix-pipe time (FLOPs / 2.5 PFLOP/s), as a fraction of the measured time, with each
    fraction beside it."""
    t = ms * 1e-3
    f_hbm = nbytes / PEAK_HBM_BPS / t
    f_mfma = flops / PEAK_FP16_FLOPS / t
    return {"bound": "hbm" if f_hbm >= f_mfma else "mfma", "roofline_frac": round(max(f_hbm, f_mfma), 4),
            "frac_hbm": round(f_hbm, 4), "frac_mfma": round(f_mfma, 4)}


def copies_for(nbytes):
    return max(2, math.ceil(ROTATE_BYTES / max(nbytes, 1)))


ALLCLOSE_RTOL = 1e-3      # elementwise check beside the max-relative bar:
ALLCLOSE_ATOL_REL = 1e-4  # |Y - ref| <= 1e-3 |ref| + 1e-4 max|ref| for every element


def parity(Y, ref, atol_rel=ALLCLOSE_ATOL_REL):
    """The error metrics of a parity spot check against the fp32 oracle: max|Y-ref| /
    max|ref| (the bar, 1e-3), the relative L2 error and an elementwise allclose with
    rtol ALLCLOSE_RTOL and atol atol_rel * max|ref| (reported beside it).  A path whose
    error is bounded against max|ref| rather than per element (the W4A16 decode at M <= 2,
    which subtracts the zero point through fp32 sums of the activations) passes the bar
    as its atol."""
    import torch

    from oracle import gemm as og

    Y, ref = Y.detach().float().cpu(), ref.detach().float().cpu()
    m = float(ref.abs().max()) if ref.numel() else 0.0
    return {"max_rel_err": float(f"{og.max_rel_err(Y, ref):.3e}"),
            "rel_l2": float(f"{og.rel_l2_err(Y, ref):.3e}"),
            "allclose": bool(torch.allclose(Y, ref, rtol=ALLCLOSE_RTOL, atol=atol_rel * m)),
            "allclose_atol_rel": atol_rel}


# ------------------------------------------------------------------------ families --
def fam_gemm(wo):
    import torch

    from oracle import gemm as og

    for (m, n, k) in [(512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048),
                      (4096, 4096, 4096), (4096, 4096, 2048)]:
        g = torch.Generator().manual_seed(42 + (0 if m == 512 else 1))
        A = torch.randn(m, k, generator=g).half()
        B = torch.randn(k, n, generator=g).half()
        Ad, Bd = A.cuda(), B.cuda()
        calls = 200 if m <= 1024 else 50
        ms = time_batches(lambda i: wo.matmul(Ad, Bd), calls)
        par = parity(wo.matmul(Ad[:256], Bd), og.gemm_ref(A[:256], B))
        fl = 2.0 * m * n * k
        line(family="gemm", M=m, N=n, K=k, plan=wo.gemm_plan(m, n, k), us=round(ms * 1e3, 2),
             TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
             frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4), **par)


def fam_epilogue(wo):
    import torch

    from oracle import gemm as og

    for s in (1024, 4096):
        g = torch.Generator().manual_seed(42 + 1)
        A = torch.randn(s, s, generator=g).half()
        B = torch.randn(s, s, generator=g).half()
        C = torch.randn(s, s, generator=g)
        Ad, Bd, Cd = A.cuda(), B.cuda(), C.cuda()
        calls = 200 if s <= 1024 else 50
        fl = 2.0 * s * s * s
        ref = og.gemm_ref(A[:256], B, 2.0, 0.5, C[:256])
        ms = time_batches(lambda i: wo.gemm(Ad, Bd, 2.0, 0.5, Cd), calls)
        err = og.max_rel_err(wo.gemm(Ad, Bd, 2.0, 0.5, Cd)[:256], ref)
        line(family="epilogue", mode="out_of_place", M=s, N=s, K=s, us=round(ms * 1e3, 2),
             TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
             frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4),
             max_rel_err=float(f"{err:.3e}"))
        Ci = Cd.clone()
        ms = time_batches(lambda i: wo.gemm_inplace(Ad, Bd, Ci, 2.0, 0.5), calls)
        Ci = Cd.clone()
        wo.gemm_inplace(Ad, Bd, Ci, 2.0, 0.5)
        err = og.max_rel_err(Ci[:256], ref)
        line(family="epilogue", mode="in_place", M=s, N=s, K=s, us=round(ms * 1e3, 2),
             TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
             frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4),
             max_rel_err=float(f"{err:.3e}"))


def fam_skinny(wo):
    import torch

    from oracle import gemm as og

    # configs[2], plus M = 32 (between its rows: the skinny kernel's two-block form)
    shapes = [(m, n, 4096) for m in (1, 16, 64, 128) for n in (4096, 11008, 14336)] + \
             [(m, 4096, 14336) for m in (1, 16, 64, 128)] + \
             [(32, n, 4096) for n in (4096, 11008, 14336)] + [(32, 4096, 14336)]
    for (m, n, k) in shapes:
        g = torch.Generator().manual_seed(42 + 2)
        A = torch.randn(m, k, generator=g).half()
        B = (torch.randn(k, n, generator=g) * 0.02).half()
        nbytes = 2 * m * k + 2 * k * n + 4 * m * n
        cp = copies_for(nbytes)
        As = [A.cuda() for _ in range(cp)]
        Bs = [B.cuda() for _ in range(cp)]
        C0 = wo.matmul(As[0], Bs[0])
        ms, outs = time_graph(lambda i: wo.matmul(As[i % cp], Bs[i % cp]), cp)
        assert torch.equal(outs[0], C0), "graph replay differs from eager"
        par = parity(C0, og.gemm_ref(A, B))
        line(family="skinny", M=m, N=n, K=k, plan=wo.gemm_plan(m, n, k), us=round(ms * 1e3, 2),
             bytes=nbytes, GBps=round(nbytes / (ms * 1e-3) / 1e9, 1),
             TFLOPS=round(2.0 * m * n * k / (ms * 1e-3) / 1e12, 2),
             **roofline(nbytes, 2.0 * m * n * k, ms), rotation_copies=cp, timing="graph replay",
             **par)
        del As, Bs, outs


def fam_ragged(wo):
    """GEMMs whose B rows (N not a multiple of 8) or A rows (K not) break 16-byte vectors,
    three ways in one process: the product path (wo.matmul: the operand is repacked into a
    zero-padded copy in the workspace, then the vector kernels run), the same call through
    the C-ABI with only the split-K workspace (the element-wise kernels read the operand in
    place), and the aligned neighbour shape (N or K rounded up to 8) for the repack's cost.
    Then shapes off the 256 grid: the planner's two-part plans against one launch."""
    import ctypes

    import torch

    from oracle import gemm as og

    L = ctypes.CDLL(wo.LIBRARY_PATH)
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    L.wmma_gemm_f16f32.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32,
                                   f32, f32, i32, vp, sz, vp]
    stream = torch.cuda.current_stream().cuda_stream
    for (m, n, k) in [(4096, 4100, 4096), (4096, 4096, 4100), (2048, 32001, 4096),
                      (1024, 4100, 4096), (128, 4100, 4096), (16, 4100, 4096), (1, 4100, 4096),
                      (1, 4096, 4100)]:
        g = torch.Generator().manual_seed(42 + 5)
        A = torch.randn(m, k, generator=g).half()
        B = (torch.randn(k, n, generator=g) * 0.02).half()
        Ad, Bd = A.cuda(), B.cuda()
        fl = 2.0 * m * n * k
        calls = 20 if fl > 1e11 else 100
        plan = wo.gemm_plan(m, n, k)
        ws = torch.empty(max(plan[7], 1), dtype=torch.uint8, device="cuda")
        C = torch.empty(m, n, device="cuda")

        def inplace(i):
            rc = L.wmma_gemm_f16f32(Ad.data_ptr(), k, Bd.data_ptr(), n, None, n, C.data_ptr(), n,
                                    m, n, k, 1.0, 0.0, -1, ws.data_ptr(), plan[7], stream)
            assert rc == 0

        n8, k8 = (n + 7) // 8 * 8, (k + 7) // 8 * 8
        # same random values, zero padded (all-zero operands would run faster than random
        # ones: the board's power limit holds the clock less)
        A8 = torch.zeros(m, k8, dtype=torch.half, device="cuda")
        B8 = torch.zeros(k8, n8, dtype=torch.half, device="cuda")
        A8[:, :k] = Ad
        B8[:k, :n] = Bd
        rows = min(m, 64)
        ref = og.gemm_ref(A[:rows], B)
        for path, fn in (("repack", lambda i: wo.matmul(Ad, Bd)), ("in place", inplace),
                         ("aligned neighbour", lambda i: wo.matmul(A8, B8))):
            ms = time_batches(fn, calls)
            if path == "repack":
                err = og.max_rel_err(wo.matmul(Ad, Bd)[:rows], ref)
            elif path == "in place":
                inplace(0)
                err = og.max_rel_err(C[:rows], ref)
            else:
                err = None
            shape = (m, n8, k8) if path == "aligned neighbour" else (m, n, k)
            line(family="ragged", path=path, M=shape[0], N=shape[1], K=shape[2],
                 plan=wo.gemm_plan(*shape), us=round(ms * 1e3, 2),
                 TFLOPS=round(2.0 * shape[0] * shape[1] * shape[2] / (ms * 1e-3) / 1e12, 1),
                 max_rel_err=None if err is None else float(f"{err:.3e}"))
        del Ad, Bd, A8, B8, C, ws
    # Off the 256 grid: the planner's plan (two launches where it splits off an edge)
    # against the faster one-launch plan of the 256x256 and 128x128 tiles (matmul_tiled:
    # one launch, no split), timed in one process.
    for (m, n, k) in [(4100, 4096, 4096), (5000, 4096, 4096), (8200, 4096, 4096),
                      (4096, 4352, 4096), (2560, 14336, 4096), (4096, 14336, 4096),
                      (7000, 4096, 4096)]:
        g = torch.Generator().manual_seed(42 + 6)
        A = torch.randn(m, k, generator=g).half()
        B = torch.randn(k, n, generator=g).half()
        Ad, Bd = A.cuda(), B.cuda()
        fl = 2.0 * m * n * k
        ms = time_batches(lambda i: wo.matmul(Ad, Bd), 10)
        err = og.max_rel_err(wo.matmul(Ad, Bd)[-64:], og.gemm_ref(A[-64:], B))
        one = min((time_batches(lambda i: wo.matmul_tiled(Ad, Bd, cfg), 10), cfg) for cfg in (5, 3))
        line(family="ragged", path="planner", M=m, N=n, K=k, plan=wo.gemm_plan(m, n, k),
             us=round(ms * 1e3, 2), TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
             max_rel_err=float(f"{err:.3e}"))
        line(family="ragged", path="one launch", M=m, N=n, K=k, tile=TILE_NAMES[one[1]],
             us=round(one[0] * 1e3, 2), TFLOPS=round(fl / (one[0] * 1e-3) / 1e12, 1))
        del Ad, Bd


def w4a16_case(wo, m, n, use_graph=True, layout=None):
    """configs[3] W4A16 case: M = m, K = 4096, N = n, G = 128.  layout: "fused" (weights,
    scales and zeros in one run per 16 columns, prepack_int4_fused: the decode layout, the
    default for m <= 4) or "sliced" (prepack_int4 + slice-major parameters, the default for
    larger m).  Same bytes either way."""
    import torch

    from oracle import gemm as og
    from oracle import int4 as oi

    kw, G = 4096, 128
    layout = layout or ("fused" if m <= 4 else "sliced")
    A, q, s, z = oi.make_inputs(m, kw, n, G, seed=42 + 3)
    # one-time layout conversions (outside the timed region)
    qd, s0, z0 = (torch.from_numpy(x).cuda() for x in (oi.pack_gptq(q), s, oi.pack_zeros(z)))
    Ad = A.cuda()
    nbytes = kw * n // 2 + (kw // G) * n * 2 + (kw // G) * n // 2 + 2 * m * kw + 4 * m * n
    cp = copies_for(nbytes)
    if layout == "fused":
        f0 = wo.prepack_int4_fused(qd, s0, z0, G)
        fs = [f0.clone() for _ in range(cp)]
        Y0 = wo.matmul_int4_fused(Ad, f0, G)
        fn = lambda i: wo.matmul_int4_fused(Ad, fs[i % cp], G)
    else:
        pk0 = wo.prepack_int4(qd)
        sd, zd = wo.prepack_int4_params(s0, z0)
        pks = [pk0.clone() for _ in range(cp)]
        sds = [sd.clone() for _ in range(cp)]
        zds = [zd.clone() for _ in range(cp)]
        Y0 = wo.matmul_int4(Ad, pk0, sd, zd, G)
        fn = lambda i: wo.matmul_int4(Ad, pks[i % cp], sds[i % cp], zds[i % cp], G)
    decode_m2 = m <= 2 and wo.w4a16_plan(m, n, kw, G)[0] == 0
    par = parity(Y0, oi.w4a16_ref(A, q, s, z, G), atol_rel=1e-3 if decode_m2 else ALLCLOSE_ATOL_REL)
    if use_graph:
        ms, outs = time_graph(fn, cp)
        assert torch.equal(outs[0], Y0), "graph replay differs from eager"
    else:
        ms = time_batches(fn, 2 * cp)
    fl = 2.0 * m * n * kw
    return {"M": m, "N": n, "K": kw, "G": G, "bytes": nbytes, "us_per_call": round(ms * 1e3, 3),
            "GBps": round(nbytes / (ms * 1e-3) / 1e9, 1),
            "TFLOPS": round(fl / (ms * 1e-3) / 1e12, 2), **roofline(nbytes, fl, ms),
            "rotation_copies": cp, "layout": layout,
            "timing": "graph replay" if use_graph else "stream launches", **par}


def fam_w4a16(wo):
    for m in (1, 16, 128, 2048):
        for n in (4096, 14336):
            r = w4a16_case(wo, m, n, use_graph=m <= 128)
            r["family"] = "w4a16"
            line(**r)


def fam_flash(wo):
    import torch

    from oracle import attention as oatt
    from oracle import gemm as og

    B, H, S, D = 4, 32, 4096, 128
    # configs[4] (multi-head), then the same with 8 key/value heads (grouped-query attention,
    # the extension of the documented API; same FLOPs, a quarter of the K/V bytes)
    for Hkv in (H, 8):
        Q, Kt, V = oatt.make_inputs(B, H, S, D, seed=42 + 4, Hkv=Hkv)
        Qd, Kd, Vd = Q.cuda(), Kt.cuda(), V.cuda()
        g = H // Hkv
        for causal in (False, True):
            ms = time_batches(lambda i: wo.flash_attention(Qd, Kd, Vd, causal, 1.0 / math.sqrt(D)), 10)
            O = wo.flash_attention(Qd, Kd, Vd, causal, 1.0 / math.sqrt(D))
            ref = oatt.sdpa_ref(Q[0:1, 0:g], Kt[0:1, 0:1], V[0:1, 0:1], causal)
            par = parity(O[0:1, 0:g], ref)
            fl = 4.0 * B * H * S * S * D if not causal else 4.0 * B * H * D * S * (S + 1) / 2
            line(family="flash", B=B, H=H, Hkv=Hkv, S=S, D=D, causal=causal, us=round(ms * 1e3, 1),
                 TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
                 frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4), **par)
            # backward pass (dQ, dK, dV from dO): FLOPs counted as 2.5x the forward's (the five
            # matrix products of the gradient; the kernels also recompute S and dP once more)
            sc = 1.0 / math.sqrt(D)
            O, lse = wo.flash_attention_forward(Qd, Kd, Vd, causal, sc)
            dO = torch.randn(B, H, S, D, generator=torch.Generator().manual_seed(77)).half()
            dOd = dO.cuda()
            msb = time_batches(lambda i: wo.flash_attention_backward(dOd, Qd, Kd, Vd, O, lse, causal, sc), 5)
            grads = wo.flash_attention_backward(dOd, Qd, Kd, Vd, O, lse, causal, sc)
            ref = oatt.sdpa_bwd_ref(Q[0:1, 0:g], Kt[0:1, 0:1], V[0:1, 0:1], dO[0:1, 0:g], causal, sc)
            errb = max(og.max_rel_err(x[0:1, 0:y.shape[1]].float(), y) for x, y in zip(grads, ref))
            flb = 2.5 * fl
            line(family="flash_bwd", B=B, H=H, Hkv=Hkv, S=S, D=D, causal=causal,
                 us=round(msb * 1e3, 1), TFLOPS=round(flb / (msb * 1e-3) / 1e12, 1),
                 frac_mfma_peak=round(flb / (msb * 1e-3) / PEAK_FP16_FLOPS, 4),
                 max_rel_err=float(f"{errb:.3e}"))
            del O, lse, dOd, grads
        del Qd, Kd, Vd
    # other head dims: D = 64 and D = 256 at the same B, H, S
    for D2 in (64, 256):
        Q, Kt, V = oatt.make_inputs(B, H, S, D2, seed=42 + 4)
        Qd, Kd, Vd = Q.cuda(), Kt.cuda(), V.cuda()
        for causal in (False, True):
            ms = time_batches(lambda i: wo.flash_attention(Qd, Kd, Vd, causal), 10)
            O = wo.flash_attention(Qd, Kd, Vd, causal)
            err = og.max_rel_err(O[0:1, 0:1].float(), oatt.sdpa_ref(Q[0:1, 0:1], Kt[0:1, 0:1], V[0:1, 0:1], causal))
            fl = 4.0 * B * H * S * S * D2 if not causal else 4.0 * B * H * D2 * S * (S + 1) / 2
            line(family="flash", B=B, H=H, S=S, D=D2, causal=causal, us=round(ms * 1e3, 1),
                 TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
                 frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4),
                 max_rel_err=float(f"{err:.3e}"))
            O, lse = wo.flash_attention_forward(Qd, Kd, Vd, causal)
            dOd = torch.randn(B, H, S, D2, generator=torch.Generator().manual_seed(77)).half().cuda()
            msb = time_batches(lambda i: wo.flash_attention_backward(dOd, Qd, Kd, Vd, O, lse, causal), 5)
            grads = wo.flash_attention_backward(dOd, Qd, Kd, Vd, O, lse, causal)
            ref = oatt.sdpa_bwd_ref(Q[0:1, 0:1], Kt[0:1, 0:1], V[0:1, 0:1], dOd[0:1, 0:1].cpu(), causal)
            errb = max(og.max_rel_err(x[0:1, 0:1].float(), y) for x, y in zip(grads, ref))
            line(family="flash_bwd", B=B, H=H, S=S, D=D2, causal=causal, us=round(msb * 1e3, 1),
                 TFLOPS=round(2.5 * fl / (msb * 1e-3) / 1e12, 1),
                 frac_mfma_peak=round(2.5 * fl / (msb * 1e-3) / PEAK_FP16_FLOPS, 4),
                 max_rel_err=float(f"{errb:.3e}"))
            del O, lse, dOd, grads
        del Qd, Kd, Vd
    # CPU baseline: fp32 SDPA on the host cores (forward, and forward + autograd backward)
    # over a bounded sample of (batch, head) slices of the same workload
    if not QUICK:
        for causal in (False, True):
            line(family="flash_cpu", causal=causal, **cpu_flash_sample(causal, 3.0, backward=True))
    # packed variable-length batch (flash_attention_varlen): six ragged sequences, 16384
    # tokens, 32 query / 8 key-value heads; FLOPs counted per sequence
    lens = [1024, 3072, 2048, 4096, 512, 5632]
    Hkv = 8
    cu = torch.tensor([0] + [sum(lens[:i + 1]) for i in range(len(lens))], dtype=torch.int32)
    g = torch.Generator().manual_seed(42 + 4)
    q = torch.randn(sum(lens), H, D, generator=g).half()
    k = torch.randn(sum(lens), Hkv, D, generator=g).half()
    v = torch.randn(sum(lens), Hkv, D, generator=g).half()
    qd, kd, vd, cud = q.cuda(), k.cuda(), v.cuda(), cu.cuda()
    for causal in (False, True):
        run = lambda i: wo.flash_attention_varlen(qd, kd, vd, cud, cud, max(lens), max(lens), causal,
                                                  1.0 / math.sqrt(D))
        ms = time_batches(run, 10)
        O = run(0)
        a, e = cu[0].item(), cu[1].item()   # first sequence checked against the oracle
        ref = oatt.sdpa_varlen_ref(q[a:e], k[a:e], v[a:e], cu[:2], cu[:2], causal)
        err = og.max_rel_err(O[a:e].float(), ref)
        fl = sum((4.0 * H * S_ * S_ * D) if not causal else 4.0 * H * D * S_ * (S_ + 1) / 2
                 for S_ in lens)
        line(family="flash", varlen=lens, H=H, Hkv=Hkv, D=D, causal=causal, us=round(ms * 1e3, 1),
             TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
             frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4),
             max_rel_err=float(f"{err:.3e}"))


def fam_decode(wo):
    """Flash attention on decoding shapes (few queries against many keys): the product path
    (wo.flash_attention: key range split over more workgroups, grouped-query heads packed
    into one sequence per K/V head) against the one-pass forward through the C-ABI without a
    workspace.  Both replayed from a HIP graph over K/V rotated past the MALL; bytes = the
    K and V read once (+ Q and O), HBM roofline."""
    import ctypes

    import torch

    from oracle import attention as oatt
    from oracle import gemm as og

    L = ctypes.CDLL(wo.LIBRARY_PATH)
    vp, i32, f32 = ctypes.c_void_p, ctypes.c_int, ctypes.c_float
    L.wmma_flash_attn_fwd_lse.argtypes = [vp] * 5 + [i32] * 6 + [f32, i32, vp]
    for (B, H, Hkv, Sq, Sk, D) in [(1, 32, 32, 1, 4096, 128), (1, 32, 8, 1, 8192, 128),
                                   (1, 32, 8, 1, 32768, 128), (8, 32, 8, 1, 4096, 128),
                                   (1, 32, 32, 16, 4096, 128), (1, 16, 16, 1, 4096, 256)]:
        Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=42 + 7, Sk=Sk, Hkv=Hkv)
        nbytes = 2 * 2 * B * Hkv * Sk * D + 2 * 2 * B * H * Sq * D
        cp = copies_for(nbytes)
        Qd = Q.cuda()
        Ks = [K.cuda() for _ in range(cp)]
        Vs = [V.cuda() for _ in range(cp)]
        ref = oatt.sdpa_ref(Q[:1, :4], oatt.expand_kv(K, H)[:1, :4], oatt.expand_kv(V, H)[:1, :4])

        def one(i):
            O = torch.empty_like(Qd)
            rc = L.wmma_flash_attn_fwd_lse(Qd.data_ptr(), Ks[i % cp].data_ptr(), Vs[i % cp].data_ptr(),
                                           O.data_ptr(), None, B, H, Hkv, Sq, Sk, D, 1.0 / math.sqrt(D), 0,
                                           torch.cuda.current_stream().cuda_stream)
            assert rc == 0
            return O

        for path, fn in (("split", lambda i: wo.flash_attention(Qd, Ks[i % cp], Vs[i % cp])),
                         ("one pass", one)):
            ms, outs = time_graph(fn, cp)
            err = og.max_rel_err(outs[0][:1, :4].float().cpu(), ref)
            line(family="decode", path=path, B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D,
                 us=round(ms * 1e3, 2), bytes=nbytes, GBps=round(nbytes / (ms * 1e-3) / 1e9, 1),
                 frac_hbm=round(nbytes / PEAK_HBM_BPS / (ms * 1e-3), 4), rotation_copies=cp,
                 timing="graph replay", max_rel_err=float(f"{err:.3e}"))
        del Ks, Vs


def fam_bwd_gqa(wo):
    """Flash-attention backward with few key/value heads (grouped-query attention, short
    sequences): the product path (wo.flash_attention_backward: the group's query heads split
    over more dK/dV workgroups, partial sums added by a second kernel) against the unsplit
    backward through the C-ABI with only the row-statistics workspace, in one process."""
    import ctypes

    import torch

    from oracle import attention as oatt

    L = ctypes.CDLL(wo.LIBRARY_PATH)
    vp, i32, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    L.wmma_flash_attn_bwd_workspace_size.restype = sz
    L.wmma_flash_attn_bwd_workspace_size.argtypes = [i32] * 3
    L.wmma_flash_attn_bwd.argtypes = [vp] * 10 + [sz] + [i32] * 6 + [f32, i32, vp]
    for (B, H, Hkv, S, D, causal) in [(1, 32, 8, 2048, 128, True), (1, 32, 8, 2048, 128, False),
                                      (1, 16, 4, 1024, 128, True), (2, 32, 4, 1024, 128, True),
                                      (1, 32, 8, 4096, 128, True)]:
        Q, K, V = oatt.make_inputs(B, H, S, D, seed=42 + 8, Hkv=Hkv)
        g = torch.Generator().manual_seed(43)
        dO = torch.randn(B, H, S, D, generator=g).half().cuda()
        Qd, Kd, Vd = Q.cuda(), K.cuda(), V.cuda()
        O, lse = wo.flash_attention_forward(Qd, Kd, Vd, causal)
        fl = 2.5 * 4.0 * B * H * D * (S * (S + 1) / 2 if causal else S * S)
        base = L.wmma_flash_attn_bwd_workspace_size(B, H, S)
        ws = torch.empty(base, dtype=torch.uint8, device="cuda")
        dQ, dK, dV = torch.empty_like(Qd), torch.empty_like(Kd), torch.empty_like(Vd)

        def unsplit(i):
            rc = L.wmma_flash_attn_bwd(dO.data_ptr(), Qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(),
                                       O.data_ptr(), lse.data_ptr(), dQ.data_ptr(), dK.data_ptr(),
                                       dV.data_ptr(), ws.data_ptr(), base, B, H, Hkv, S, S, D,
                                       1.0 / math.sqrt(D), 1 if causal else 0,
                                       torch.cuda.current_stream().cuda_stream)
            assert rc == 0

        for path, fn in (("split", lambda i: wo.flash_attention_backward(dO, Qd, Kd, Vd, O, lse, causal)),
                         ("unsplit", unsplit)):
            ms = time_batches(fn, 5)
            line(family="bwd_gqa", path=path, B=B, H=H, Hkv=Hkv, S=S, D=D, causal=causal,
                 us=round(ms * 1e3, 1), TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
                 frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4))
        del ws, dQ, dK, dV


def fam_flash_operands(wo):
    """configs[4] non-causal, forward and backward, on all-ones Q, K, V (and dO): the same
    kernels and traffic with operand bits that never switch -- against the random-input
    lines of the flash family, how far the board's power limit holds these kernels on
    random data.  A family of its own so that the flash family's kernel trace holds only
    random-input launches."""
    import torch

    B, H, S, D = 4, 32, 4096, 128
    ones = torch.ones(B, H, S, D, dtype=torch.float16, device="cuda")
    fl = 4.0 * B * H * S * S * D
    ms = time_batches(lambda i: wo.flash_attention(ones, ones, ones, False), 10)
    line(family="flash", B=B, H=H, S=S, D=D, causal=False, operands="all ones", us=round(ms * 1e3, 1),
         TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1), frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4))
    O, lse = wo.flash_attention_forward(ones, ones, ones, False)
    msb = time_batches(lambda i: wo.flash_attention_backward(ones, ones, ones, ones, O, lse, False), 5)
    line(family="flash_bwd", B=B, H=H, S=S, D=D, causal=False, operands="all ones", us=round(msb * 1e3, 1),
         TFLOPS=round(2.5 * fl / (msb * 1e-3) / 1e12, 1),
         frac_mfma_peak=round(2.5 * fl / (msb * 1e-3) / PEAK_FP16_FLOPS, 4))


def fam_vendor(wo):
    """The vendor libraries torch dispatches to on the same inputs, for comparison (not
    this library's code): torch.mm fp16 x fp16 with fp32 output (out_dtype) and with fp16
    output (hipBLASLt / rocBLAS), and torch's flash scaled_dot_product_attention on
    configs[4] (the FLASH_ATTENTION backend only; reported unavailable otherwise)."""
    import torch

    for (m, n, k) in [(2048, 2048, 2048), (4096, 4096, 4096), (4096, 4096, 2048)]:
        g = torch.Generator().manual_seed(42 + 1)
        Ad = torch.randn(m, k, generator=g).half().cuda()
        Bd = torch.randn(k, n, generator=g).half().cuda()
        fl = 2.0 * m * n * k
        for out in ("f32", "f16"):
            if out == "f32":
                fn = lambda i: torch.mm(Ad, Bd, out_dtype=torch.float32)
            else:
                fn = lambda i: torch.mm(Ad, Bd)
            ms = time_batches(fn, 50)
            line(family="vendor_gemm", M=m, N=n, K=k, out=out, library="torch.mm (hipBLASLt/rocBLAS)",
                 us=round(ms * 1e3, 2), TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
                 frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4))
            # this library on the same inputs, timed the same way
            if out == "f32":
                ms2 = time_batches(lambda i: wo.matmul(Ad, Bd), 50)
                line(family="vendor_gemm", M=m, N=n, K=k, out=out, library="wmma_ops_amd.matmul",
                     us=round(ms2 * 1e3, 2), TFLOPS=round(fl / (ms2 * 1e-3) / 1e12, 1),
                     frac_mfma_peak=round(fl / (ms2 * 1e-3) / PEAK_FP16_FLOPS, 4))
        del Ad, Bd
    # Microsecond shapes, both libraries captured in a HIP graph and replayed (launch gaps
    # out of the figure): the small squares of configs[0..1] with the inputs resident, and
    # the few-row shapes of configs[2] with the inputs rotated over > 512 MB as in `skinny`.
    small = [(512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048)] + \
            [(m, 4096, 4096) for m in (1, 16, 32, 64, 128)] + [(128, 14336, 4096)]
    for (m, n, k) in small:
        g = torch.Generator().manual_seed(42 + 2)
        A = torch.randn(m, k, generator=g).half()
        B = (torch.randn(k, n, generator=g) * 0.02).half()
        nbytes = 2 * m * k + 2 * k * n + 4 * m * n
        cp = copies_for(nbytes) if m <= 128 and m < n else 2
        As = [A.cuda() for _ in range(cp)]
        Bs = [B.cuda() for _ in range(cp)]
        fl = 2.0 * m * n * k
        for lib, fn in (("torch.mm (hipBLASLt/rocBLAS)",
                         lambda i: torch.mm(As[i % cp], Bs[i % cp], out_dtype=torch.float32)),
                        ("wmma_ops_amd.matmul", lambda i: wo.matmul(As[i % cp], Bs[i % cp]))):
            ms, _ = time_graph(fn, cp if cp > 2 else 20)
            line(family="vendor_gemm_small", M=m, N=n, K=k, out="f32", library=lib,
                 us=round(ms * 1e3, 2), TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
                 GBps=round(nbytes / (ms * 1e-3) / 1e9, 1), rotation_copies=cp,
                 timing="graph replay")
        del As, Bs
    # 4096^3 fp32-output on all-ones operands (the operand bits never switch, so the board's
    # power limit holds the clock less): both kernels' pipelines without the data's energy.
    Ad = torch.ones(4096, 4096, dtype=torch.float16, device="cuda")
    Bd = torch.ones(4096, 4096, dtype=torch.float16, device="cuda")
    fl = 2.0 * 4096 ** 3
    for lib, fn in (("torch.mm (hipBLASLt/rocBLAS)", lambda i: torch.mm(Ad, Bd, out_dtype=torch.float32)),
                    ("wmma_ops_amd.matmul", lambda i: wo.matmul(Ad, Bd))):
        ms = time_batches(fn, 50)
        line(family="vendor_gemm", M=4096, N=4096, K=4096, out="f32", operands="all ones", library=lib,
             us=round(ms * 1e3, 2), TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
             frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4))
    del Ad, Bd
    from torch.nn.attention import SDPBackend, sdpa_kernel

    B, H, S, D = 4, 32, 4096, 128
    g = torch.Generator().manual_seed(42 + 4)
    Q, Kt, V = (torch.randn(B, H, S, D, generator=g).half().cuda() for _ in range(3))
    for causal in (False, True):
        fl = 4.0 * B * H * S * S * D if not causal else 4.0 * B * H * D * S * (S + 1) / 2
        try:
            with sdpa_kernel(SDPBackend.FLASH_ATTENTION):
                fn = lambda i: torch.nn.functional.scaled_dot_product_attention(Q, Kt, V, is_causal=causal)
                ms = time_batches(fn, 5)
            line(family="vendor_flash", B=B, H=H, S=S, D=D, causal=causal,
                 library="torch SDPA (FLASH_ATTENTION backend)", us=round(ms * 1e3, 1),
                 TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1))
        except RuntimeError as e:
            line(family="vendor_flash", causal=causal, library="torch SDPA", unavailable=str(e)[:200])


def fam_copy(wo):
    """Plain device copy of a known size: the calibration for rocprofv3's FETCH_SIZE and
    WRITE_SIZE counters (bytes the counters report per byte actually copied)."""
    import torch

    nbytes = 256 << 20
    x = torch.ones(nbytes, dtype=torch.uint8, device="cuda")
    y = torch.empty_like(x)
    ms = time_batches(lambda i: y.copy_(x), 10)
    line(family="copy", bytes=nbytes, us=round(ms * 1e3, 1),
         GBps_read_plus_write=round(2 * nbytes / (ms * 1e-3) / 1e9, 1))


def calib_lib():
    """The calibration kernels (include/wmma_calib.h): bench.py's measuring instruments."""
    import ctypes

    L = ctypes.CDLL(os.path.join(ROOT, "wmma_ops_amd", "libwmma_calib.so"))
    vp, i32 = ctypes.c_void_p, ctypes.c_int
    L.wmma_calib_mfma_ceiling.argtypes = [i32, i32, vp, vp, vp]
    L.wmma_calib_mfma_ceiling_flops.argtypes = [i32, i32]
    L.wmma_calib_mfma_ceiling_flops.restype = ctypes.c_double
    L.wmma_calib_read_stream.argtypes = [vp, ctypes.c_size_t, i32, vp, vp]
    L.wmma_calib_read_stream_shape.argtypes = [vp, ctypes.c_size_t, i32, i32, vp, vp]
    L.wmma_calib_lds_read.argtypes = [i32, i32, i32, vp, vp]
    L.wmma_calib_lds_read_bytes.argtypes = [i32, i32]
    L.wmma_calib_lds_read_bytes.restype = ctypes.c_double
    sz = ctypes.c_size_t
    L.wmma_calib_l2_stage.argtypes = [i32, i32, i32, vp, sz, sz, i32, i32, vp, vp]
    L.wmma_calib_l2_stage_bytes.argtypes = [i32, i32]
    L.wmma_calib_l2_stage_bytes.restype = ctypes.c_double
    return L


def mfma_ceiling(calls=200, random_operands=True):
    """Sustained rate (FLOP/s) of v_mfma_f32_32x32x16_f16 on register operands, 512
    workgroups x 4 waves x 8 independent accumulators, ~1 ms launches back to back after
    the settle phase: the matrix pipe's ceiling on this board, clock and power limits
    included.  With random operands (fp16 N(0,1), as the GEMM's inputs) the operand bits
    switch from one MFMA to the next; with constant operands they do not, and the board
    draws less power."""
    import torch

    L = calib_lib()
    wgs, iters = 512, 4000
    sink = torch.zeros(wgs, device="cuda")
    ops = None
    if random_operands:
        g = torch.Generator().manual_seed(42)
        ops = torch.randn(wgs * 256 * 16 * 8, generator=g).half().cuda()
    st = torch.cuda.current_stream().cuda_stream
    run = lambda i: L.wmma_calib_mfma_ceiling(wgs, iters, ops.data_ptr() if ops is not None else None,
                                              sink.data_ptr(), st)
    assert run(0) == 0
    ms = time_batches(run, calls if not QUICK else 2, batches=3)
    return L.wmma_calib_mfma_ceiling_flops(wgs, iters) / (ms * 1e-3), ms


def fam_mfma_ceiling(wo):
    for rnd in (True, False):
        fl, ms = mfma_ceiling(random_operands=rnd)
        line(family="mfma_ceiling", operands="random N(0,1) fp16" if rnd else "constant",
             TFLOPS=round(fl / 1e12, 1), frac_mfma_peak=round(fl / PEAK_FP16_FLOPS, 4),
             us_per_launch=round(ms * 1e3, 1),
             config="512 workgroups x 4 waves, each wave 4000 x 8 independent "
                    "v_mfma_f32_32x32x16_f16 on register operands (no memory traffic)")
    # The same 4096^3 GEMM (same kernel, same memory traffic) on random and on constant
    # operands: a kernel limited by issue or memory runs both in the same time; a
    # power-limited one runs faster when the operand bits do not switch.
    import torch

    g = torch.Generator().manual_seed(42 + 1)
    for name in ("random N(0,1) fp16", "all ones", "all zeros"):
        if name.startswith("random"):
            A = torch.randn(4096, 4096, generator=g).half().cuda()
            B = torch.randn(4096, 4096, generator=g).half().cuda()
        else:
            v = 1.0 if name == "all ones" else 0.0
            A = torch.full((4096, 4096), v, dtype=torch.float16, device="cuda")
            B = torch.full((4096, 4096), v, dtype=torch.float16, device="cuda")
        ms = time_batches(lambda i: wo.matmul(A, B), 100 if not QUICK else 2)
        fl = 2.0 * 4096 ** 3
        line(family="gemm_operands", M=4096, N=4096, K=4096, operands=name, us=round(ms * 1e3, 2),
             TFLOPS=round(fl / (ms * 1e-3) / 1e12, 1),
             frac_mfma_peak=round(fl / (ms * 1e-3) / PEAK_FP16_FLOPS, 4))
        del A, B


def fam_lds_read(wo):
    """LDS read rate of the fragment-read patterns of the MFMA kernels (libwmma_calib.so):
    one workgroup of 8 waves per CU, each wave reading 8 KB per iteration of a 64 KB LDS
    buffer, ~0.3 ms launches back to back after the clock settles."""
    import torch

    L = calib_lib()
    wgs, iters = 256, 2000
    sink = torch.zeros(wgs, device="cuda")
    names = {0: "ds_read_b128, 1 KB contiguous per instruction",
             1: "ds_read_b64_tr_b16, 512 contiguous bytes per instruction",
             2: "ds_read_b64_tr_b16, flash forward V-fragment pattern (D = 128)"}
    nbytes = L.wmma_calib_lds_read_bytes(wgs, iters)
    for mode in (0, 1, 2):
        st = torch.cuda.current_stream().cuda_stream
        fn = lambda i: L.wmma_calib_lds_read(mode, wgs, iters, sink.data_ptr(), st)
        assert fn(0) == 0
        ms = time_batches(fn, 50 if not QUICK else 2, batches=3)
        line(family="lds_read", pattern=names[mode], us_per_launch=round(ms * 1e3, 1),
             TBps_chip=round(nbytes / (ms * 1e-3) / 1e12, 1),
             GBps_per_cu=round(nbytes / (ms * 1e-3) / 1e9 / wgs, 1),
             config=f"{wgs} workgroups x 8 waves x {iters} iterations x 8 KB")


def fam_l2_read(wo):
    """The activation stage of the small-M LDS-DMA GEMMs alone (libwmma_calib.so): 224
    workgroups (the W4A16 GEMM grid at M = 128, N = 14336) copy 64-row x 128-byte blocks of
    a 1 MB L2-resident buffer (rows 8 KB apart, as A at K = 4096) into LDS, 4 or 8 waves per
    workgroup, 7, 3 or no blocks in flight; and the same bytes as contiguous 8 KB blocks."""
    import torch

    L = calib_lib()
    wgs, iters, row_bytes = 224, 64, 8192
    nb = 128 * row_bytes
    src = torch.ones(nb // 2, dtype=torch.float16, device="cuda")
    sink = torch.zeros(wgs, device="cuda")
    nbytes = L.wmma_calib_l2_stage_bytes(wgs, iters)
    for strided, waves, depth in ((1, 4, 4), (1, 4, 8), (1, 4, 1), (1, 8, 4), (1, 8, 8), (1, 8, 1),
                                  (0, 4, 4), (0, 8, 4)):
        st = torch.cuda.current_stream().cuda_stream
        fn = lambda i: L.wmma_calib_l2_stage(waves, depth, strided, src.data_ptr(), nb, row_bytes,
                                             wgs, iters, sink.data_ptr(), st)
        assert fn(0) == 0
        ms = time_batches(fn, 400 if not QUICK else 2, batches=3)
        line(family="l2_read", pattern="64 rows x 128 B, rows 8 KB apart" if strided else
             "contiguous 8 KB blocks", waves=waves, blocks_in_flight=depth - 1,
             us_per_launch=round(ms * 1e3, 2), ns_per_block=round(ms * 1e6 / iters, 1),
             GBps_per_cu=round(nbytes / (ms * 1e-3) / 1e9 / wgs, 1),
             TBps_chip=round(nbytes / (ms * 1e-3) / 1e12, 2),
             config=f"{wgs} workgroups x {iters} blocks of 8 KB")


def read_floor_best(nbytes, shapes=((64, 16), (256, 2), (512, 2))):
    """(us, shape) of the fastest plain streaming read of nbytes (rounded down to 16) over
    the given launch shapes, graph-replayed over rotating buffers like the W4A16 figures."""
    import torch

    L = calib_lib()
    nb = nbytes // 16 * 16
    cp = copies_for(nb)
    bufs = [torch.empty(nb, dtype=torch.uint8, device="cuda").fill_(i & 255) for i in range(cp)]
    sink = torch.zeros(nb // 8192 + 1, device="cuda")
    best = None
    for threads, loads in shapes:
        def fn(i):
            rc = L.wmma_calib_read_stream_shape(bufs[i % cp].data_ptr(), nb, threads, loads,
                                                sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
            assert rc == 0

        ms, _ = time_graph(fn, cp)
        if best is None or ms < best[0]:
            best = (ms, f"{threads} threads x {loads} loads per lane")
    del bufs
    return best[0] * 1e3, best[1]


def fam_read_floor(wo):
    """Streaming reads of the W4A16 M=1 weight sizes (K=4096, N=4096 / 14336: 8 MiB, 28 MiB)
    and of 1 GiB in several launch shapes (threads per workgroup x 16-byte loads per lane),
    buffers rotated over > 512 MB and replayed from a HIP graph, like the W4A16 figures: the
    floor of an HBM-bound kernel reading that many bytes is the fastest shape's time."""
    import torch

    L = calib_lib()
    shapes = [(64, 16), (256, 2), (256, 4), (256, 8), (512, 2), (512, 4), (512, 8), (1024, 2),
              (1024, 4)]
    for nbytes in (4096 * 4096 // 2, 4096 * 14336 // 2, 1 << 30):
        cp = copies_for(nbytes)
        bufs = [torch.empty(nbytes, dtype=torch.uint8, device="cuda").fill_(i & 255) for i in range(cp)]
        sink = torch.zeros(nbytes // 8192 + 1, device="cuda")
        best = None
        for threads, loads in shapes:
            def fn(i):
                rc = L.wmma_calib_read_stream_shape(bufs[i % cp].data_ptr(), nbytes, threads, loads,
                                                    sink.data_ptr(), torch.cuda.current_stream().cuda_stream)
                assert rc == 0

            ms, _ = time_graph(fn, cp)
            line(family="read_floor", bytes=nbytes, threads=threads, loads_per_lane=loads,
                 us=round(ms * 1e3, 3), GBps=round(nbytes / (ms * 1e-3) / 1e9, 1),
                 frac_hbm=round(nbytes / (ms * 1e-3) / PEAK_HBM_BPS, 4), rotation_copies=cp)
            if best is None or ms < best[0]:
                best = (ms, threads, loads)
        line(family="read_floor_best", bytes=nbytes, us=round(best[0] * 1e3, 3),
             GBps=round(nbytes / (best[0] * 1e-3) / 1e9, 1),
             frac_hbm=round(nbytes / (best[0] * 1e-3) / PEAK_HBM_BPS, 4),
             shape=f"{best[1]} threads x {best[2]} loads per lane")
        del bufs


FAMILIES = {"gemm": fam_gemm, "epilogue": fam_epilogue, "skinny": fam_skinny, "ragged": fam_ragged,
            "w4a16": fam_w4a16, "flash": fam_flash, "copy": fam_copy,
            "mfma_ceiling": fam_mfma_ceiling, "read_floor": fam_read_floor, "lds_read": fam_lds_read,
            "l2_read": fam_l2_read,
            "flash_operands": fam_flash_operands, "decode": fam_decode, "bwd_gqa": fam_bwd_gqa,
            "vendor": fam_vendor}


# ------------------------------------------------------------------------ headline --
def gemm_clock_and_batches(wo):
    """The headline GEMM's sustained clock / power (ClockSampler) and its median of 5
    event-timed batches of 200 back-to-back calls (BASELINE.md's timing convention)."""
    import torch

    g = torch.Generator().manual_seed(42 + 1)
    A = torch.randn(M, K, generator=g).half().cuda()
    B = torch.randn(K, N, generator=g).half().cuda()
    fn = lambda i: wo.matmul(A, B)
    clock = sustained_clock(fn)
    ms = time_batches(fn, 200)
    return clock, {"us_per_call": round(ms * 1e3, 2),
                   "TFLOPS": round(2.0 * M * N * K / (ms * 1e-3) / 1e12, 1)}


def gemm_bench(wo, steps, warmup):
    import torch

    g = torch.Generator().manual_seed(42 + 1)
    A = torch.randn(M, K, generator=g).half().cuda()
    B = torch.randn(K, N, generator=g).half().cuda()
    settle(lambda i: wo.matmul(A, B))
    for _ in range(warmup):
        wo.matmul(A, B)
    torch.cuda.synchronize()
    # One event pair on the launch stream (torch's current stream, which the extension
    # launches on) brackets the timed region: its span / steps is the kernel's average
    # launch duration, back to back as in the timed steps.
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record()
    for _ in range(steps):
        C = wo.matmul(A, B)
    e1.record()
    torch.cuda.synchronize()
    ms_step = (time.perf_counter() - t0) * 1e3 / steps
    ms_kernel = e0.elapsed_time(e1) / steps
    # parity spot check of the benchmarked output (a 256-row slab against the fp32 CPU oracle)
    from oracle import gemm as og

    par = parity(C[:256], og.gemm_ref(A[:256].cpu(), B.cpu()))
    return ms_step, ms_kernel, par


def cpu_model() -> str:
    """The host CPU as /proc/cpuinfo describes it: model name, family / model / stepping
    (a virtualised host may report only a generic name), clock, and the widest x86 vector
    extension the matmul kernels can use."""
    info = {}
    try:
        with open("/proc/cpuinfo") as f:
            for ln in f:
                if ":" not in ln:
                    if info:
                        break  # first processor only
                    continue
                k, v = (x.strip() for x in ln.split(":", 1))
                info.setdefault(k, v)
    except OSError:
        return "unknown"
    flags = set(info.get("flags", "").split())
    simd = "avx512" if "avx512f" in flags else "avx2" if "avx2" in flags else "sse"
    return (f"{info.get('model name', 'unknown')} (family {info.get('cpu family', '?')}, model "
            f"{info.get('model', '?')}, stepping {info.get('stepping', '?')}, "
            f"{info.get('cpu MHz', '?')} MHz, {simd})")


def cpu_threads() -> int:
    """Host threads for the CPU baselines: the process's CPUs, at most 16 (the GPU box's
    share of one GPU)."""
    import torch

    threads = min(16, len(os.sched_getaffinity(0)))
    torch.set_num_threads(threads)
    return threads


def cpu_time(fn, seconds, max_calls=50):
    """Median wall time (s) of fn() after one warm-up, over at least 3 calls and about
    `seconds` of work."""
    fn()
    times = []
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or len(times) < 3:
        t0 = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t0)
        if len(times) >= max_calls:
            break
    return statistics.median(times), len(times)


def cpu_flash_sample(causal, seconds, backward=False):
    """fp32 SDPA of the oracle (oracle.attention.sdpa_ref; with backward=True also its
    autograd backward) on the host cores, over 2 (batch, head) slices of configs[4]
    ([4,32,4096,128]): a bounded sample of the flash workload, FLOPs counted as on the GPU."""
    import torch

    from oracle import attention as oatt

    threads = cpu_threads()
    S, D = 4096, 128
    Q, Kt, V = oatt.make_inputs(1, 2, S, D, seed=42 + 4)
    fl = 4.0 * 2 * S * S * D if not causal else 4.0 * 2 * D * S * (S + 1) / 2
    t, n = cpu_time(lambda: oatt.sdpa_ref(Q, Kt, V, causal), seconds, 10)
    out = {"value": round(fl / t / 1e12, 4), "unit": "TFLOPS", "cores": threads, "kind": "port",
           "sample": f"2 heads of [4,32,{S},{D}] (causal={causal}): {n} calls of "
                     f"oracle.attention.sdpa_ref, median {t * 1e3:.0f} ms"}
    if backward:
        dO = torch.randn(1, 2, S, D, generator=torch.Generator().manual_seed(77)).half()
        tb, nb = cpu_time(lambda: oatt.sdpa_bwd_ref(Q, Kt, V, dO, causal), seconds, 10)
        out["bwd_TFLOPS"] = round(2.5 * fl / tb / 1e12, 4)
        out["sample"] += f"; {nb} calls of sdpa_bwd_ref, median {tb * 1e3:.0f} ms"
    out["cpu_model"] = cpu_model()
    return out


def cpu_baseline(seconds):
    """The oracle on host cores, bounded samples of the headline workloads: fp32
    torch.matmul at 4096^3, the W4A16 M = 1 decode (GPTQ unpack, fp16((q - z) * s)
    dequantisation and matmul, N = 14336), and fp32 SDPA on 2 heads of configs[4]."""
    import torch

    from oracle import gemm as og
    from oracle import int4 as oi

    threads = cpu_threads()
    g = torch.Generator().manual_seed(42 + 1)
    A = torch.randn(M, K, generator=g).half()
    B = torch.randn(K, N, generator=g).half()
    t, n = cpu_time(lambda: og.gemm_ref(A, B), seconds)
    out = {"value": round(2.0 * M * N * K / t / 1e12, 4), "unit": "TFLOPS", "cores": threads,
           "kind": "port",
           "sample": f"{n} calls of torch.matmul(A.float(), B.float()) at 4096^3 "
                     f"(oracle.gemm.gemm_ref), median {t * 1e3:.1f} ms",
           "cpu_model": cpu_model(), "os_cpu_count": os.cpu_count()}
    # W4A16 decode: the time includes unpacking the packed GPTQ words and the dequantisation
    Aq, q, sc, z = oi.make_inputs(1, 4096, 14336, 128, seed=42 + 3)
    qw = oi.pack_gptq(q)
    nbytes = 4096 * 14336 // 2 + (4096 // 128) * 14336 * 2 + (4096 // 128) * 14336 // 2 + 2 * 4096 + 4 * 14336
    tw, nw = cpu_time(lambda: oi.w4a16_ref(Aq, oi.unpack_gptq(qw), sc, z, 128), seconds / 4, 10)
    out["w4a16_m1"] = {"value": round(nbytes / tw / 1e9, 3), "unit": "GB/s", "cores": threads,
                       "sample": f"{nw} calls of unpack_gptq + dequant + matmul at M=1, N=14336, "
                                 f"K=4096, G=128 (oracle.int4), median {tw * 1e3:.1f} ms"}
    fs = cpu_flash_sample(False, seconds / 4)
    fs.pop("cpu_model")
    out["flash"] = fs
    return out


def headline(wo, args):
    ms_step, ms_kernel, par = gemm_bench(wo, args.steps, args.warmup)
    flops = 2.0 * M * N * K
    tflops = flops / (ms_step * 1e-3) / 1e12
    achieved = flops / (ms_kernel * 1e-3) / 1e12
    traffic = None
    if os.path.exists(TRAFFIC_FILE):
        with open(TRAFFIC_FILE) as f:
            traffic = json.load(f).get("hbm_bytes_per_launch")
    plan = wo.gemm_plan(M, N, K)
    ceiling, _ = mfma_ceiling(calls=100)
    clock, batches = gemm_clock_and_batches(wo)
    sclk = clock["sclk_MHz"] * 1e6 if clock else None
    # dense FP16 MFMA peak at the measured clock: 256 CUs x 4096 FLOP per clock per CU
    peak_sclk = 256 * 4096 * sclk if sclk else None
    out = {
        "metric": METRIC,
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
                   "M": M, "N": N, "K": K, "plan": plan},
        "pct_mfma_peak": round(100.0 * tflops * 1e12 / PEAK_FP16_FLOPS, 2),
        **par,  # max_rel_err (the 1e-3 bar), rel_l2, allclose on a 256-row slab
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2),
                     "peak": PEAK_FP16_FLOPS / 1e12, "unit": "TFLOP/s",
                     "frac": round(achieved * 1e12 / PEAK_FP16_FLOPS, 4), "traffic": traffic,
                     "kernel": "gemm_mfma_kernel<256,256,32,2,4,4> (BMxBNxBK, waves MxN, stages)",
                     "kernel_us": round(ms_kernel * 1e3, 2),
                     # the matrix pipe's measured rate with register operands (no memory
                     # traffic) on this board, from libwmma_calib.so, in the same run
                     "ceiling": {"TFLOPS": round(ceiling / 1e12, 1),
                                 "frac": round(achieved * 1e12 / ceiling, 4),
                                 "what": "v_mfma_f32_32x32x16_f16 back to back, 512 workgroups "
                                         "x 4 waves x 8 accumulators, random fp16 register "
                                         "operands (bench.py --workload mfma_ceiling)"},
                     # the gfx clock this GEMM holds under sustained load (SMU metrics via
                     # amdsmi, median over ~0.6 s of back-to-back launches) and the dense
                     # FP16 peak at that clock (256 CUs x 4096 FLOP/clk)
                     "sclk_GHz": round(sclk / 1e9, 3) if sclk else None,
                     "peak_at_sclk": round(peak_sclk / 1e12, 1) if peak_sclk else None,
                     "frac_at_sclk": round(achieved * 1e12 / peak_sclk, 4) if peak_sclk else None,
                     "socket_power_W": clock["socket_power_W"] if clock else None},
        # BASELINE.md's convention: median of 5 event-timed batches of back-to-back calls
        "median_of_5_batches": batches,
    }
    if not args.no_w4a16:
        out["w4a16_m1"] = [w4a16_case(wo, 1, n) for n in (4096, 14336)]
        for r in out["w4a16_m1"]:
            # the same bytes read by a plain streaming kernel in its fastest launch shape, in
            # the same run (libwmma_calib.so): the floor of one launch reading that much
            fl_us, shape = read_floor_best(r["bytes"])
            r["read_floor"] = {"us": round(fl_us, 3), "shape": shape,
                               "frac": round(fl_us / r["us_per_call"], 4),
                               "what": "streaming read of the same byte count, fastest of "
                                       "64x16, 256x2, 512x2 threads x 16-byte loads per lane, "
                                       "graph-replayed over rotating buffers "
                                       "(bench.py --workload read_floor)"}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(out), flush=True)


def main():
    args = parse()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (asked for --gpus {args.gpus}); every GPU box "
              "in this build has one MI355X. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch

    import wmma_ops_amd as wo

    assert torch.cuda.is_available(), "bench.py needs a GPU"
    global QUICK
    QUICK = args.quick and bool(args.suite or args.workload)
    if args.suite:
        for name in ("gemm", "epilogue", "skinny", "ragged", "w4a16", "flash", "flash_operands",
                     "decode", "bwd_gqa"):
            FAMILIES[name](wo)
    elif args.workload:
        FAMILIES[args.workload](wo)
    else:
        headline(wo, args)


if __name__ == "__main__":
    main()
