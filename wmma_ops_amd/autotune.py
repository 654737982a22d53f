"""Autotuner for the GEMM dispatch table -- the MI355X counterpart of the reference's
autotune.py (:131-283), which times matmul_tiled configurations and emits the C++ of
select_tuned_tile.

    python -m wmma_ops_amd.autotune [--shapes baseline | M,N,K ...] [--emit PATH]
                                    [--report PATH] [--min-gain 0.03]

For every shape it times each plan the kernels can run -- the tiled LDS-DMA kernel with
every tile (WMMA_TILE_*) and K split 1, 2, 4, 8, 16, and for M <= 64 the streaming skinny
kernel with K splits 1..32 -- through the C-ABI (wmma_gemm_plan_custom,
wmma_gemm_f16f32_plan), next to the planner's own choice.  Every plan's output is checked
against the planner's (max relative error <= 1e-3) before it is timed.  Inputs are rotated
over more than 512 MB when one copy would fit in the 256 MB MALL, and each shape's work
runs for 30 ms (100 ms for the first) before its timings so the clock has settled; the
planner's own plan is timed in the same sweep.  A shape enters the emitted table when a
different plan beats the planner's by more than --min-gain, or when the compiled table
already holds it (the planner then reports the table's plan as its own); the table
(wmma_ops_amd/csrc/tuned_table.inc) is compiled into the planner, so a rebuild applies it.  Needs a GPU; it is a tool, not part of any compute path.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import statistics
import sys

ROOT = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(ROOT, "libwmma_ops_amd.so")
TABLE_PATH = os.path.join(ROOT, "csrc", "tuned_table.inc")

KERNEL_TILED, KERNEL_SKINNY = 0, 1
TILE_NAMES = ["64x64", "128x64", "256x64", "128x128", "256x128", "256x256"]
SKINNY_MAX_M = 64
ROTATE_BYTES = 600e6


class Plan(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int), ("tile_cfg", ctypes.c_int), ("tile_m", ctypes.c_int),
                ("tile_n", ctypes.c_int), ("split_k", ctypes.c_int), ("k_per_split", ctypes.c_int),
                ("grid", ctypes.c_int), ("workspace_bytes", ctypes.c_size_t),
                ("edge_dim", ctypes.c_int), ("edge_at", ctypes.c_int)]


def load_lib(path: str = LIB_PATH):
    lib = ctypes.CDLL(path)
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_last_error.restype = ctypes.c_char_p
    lib.wmma_gemm_plan_make.argtypes = [i32, i32, i32, i32, i32, ctypes.POINTER(Plan)]
    lib.wmma_gemm_plan_custom.argtypes = [i32, i32, i32, i32, i32, i32, ctypes.POINTER(Plan)]
    lib.wmma_gemm_f16f32_plan.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32,
                                          f32, f32, ctypes.POINTER(Plan), vp, sz, vp]
    return lib


def baseline_shapes():
    """BASELINE configs[0..2]: the square and rectangular GEMMs and the skinny set."""
    shapes = [(512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
              (4096, 4096, 2048)]
    shapes += [(m, n, 4096) for m in (1, 16, 64, 128) for n in (4096, 11008, 14336)]
    shapes += [(m, 4096, 14336) for m in (1, 16, 64, 128)]
    return shapes


def candidate_plans(lib, M, N, K):
    """Every (kernel, tile, split) the kernels accept for this shape, as Plan structs."""
    out = []
    for tile in range(len(TILE_NAMES)):
        for split in (1, 2, 4, 8, 16):
            p = Plan()
            if lib.wmma_gemm_plan_custom(M, N, K, KERNEL_TILED, tile, split, ctypes.byref(p)) == 0:
                out.append(p)
    if M <= SKINNY_MAX_M:
        for split in (1, 2, 3, 4, 5, 6, 8, 12, 16, 24, 32):
            p = Plan()
            if lib.wmma_gemm_plan_custom(M, N, K, KERNEL_SKINNY, -1, split, ctypes.byref(p)) == 0:
                out.append(p)
    # the same split can be reached from two requests (k_per_split rounding): keep one
    seen, uniq = set(), []
    for p in out:
        key = (p.kernel, p.tile_cfg, p.split_k)
        if key not in seen:
            seen.add(key)
            uniq.append(p)
    return uniq


def describe(p: Plan) -> str:
    name = "skinny" if p.kernel == KERNEL_SKINNY else TILE_NAMES[p.tile_cfg]
    edge = f" + edge {'rows' if p.edge_dim == 1 else 'cols'} from {p.edge_at}" if p.edge_dim else ""
    return f"{name} split {p.split_k}{edge}"


class Shape:
    """Device inputs of one shape (rotated copies when the working set fits the MALL)."""

    def __init__(self, torch, M, N, K, seed):
        g = torch.Generator().manual_seed(seed)
        A = torch.randn(M, K, generator=g).half()
        B = torch.randn(K, N, generator=g).half()
        nbytes = 2 * M * K + 2 * K * N
        self.copies = max(1, math.ceil(ROTATE_BYTES / nbytes)) if nbytes < 256e6 else 1
        self.A = [A.cuda() for _ in range(self.copies)]
        self.B = [B.cuda() for _ in range(self.copies)]
        self.C = torch.empty(M, N, device="cuda")
        self.M, self.N, self.K = M, N, K


def run(lib, torch, s: Shape, plan: Plan, ws, i: int, out=None):
    C = s.C if out is None else out
    rc = lib.wmma_gemm_f16f32_plan(s.A[i % s.copies].data_ptr(), s.K, s.B[i % s.copies].data_ptr(),
                                   s.N, None, s.N, C.data_ptr(), s.N, s.M, s.N, s.K, 1.0, 0.0,
                                   ctypes.byref(plan), ws.data_ptr() if ws is not None else None,
                                   plan.workspace_bytes, torch.cuda.current_stream().cuda_stream)
    if rc:
        raise RuntimeError(lib.wmma_last_error().decode())
    return C


def time_plan(lib, torch, s: Shape, plan: Plan, ws, batches=3, min_ms=2.0):
    """Median per-call time (us) over `batches` back-to-back batches of calls."""
    run(lib, torch, s, plan, ws, 0)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    run(lib, torch, s, plan, ws, 1)
    e1.record()
    e1.synchronize()
    calls = max(s.copies, min(400, int(min_ms / max(e0.elapsed_time(e1), 1e-3)) + 1))
    ts = []
    for _ in range(batches):
        e0.record()
        for i in range(calls):
            run(lib, torch, s, plan, ws, i)
        e1.record()
        e1.synchronize()
        ts.append(e0.elapsed_time(e1) * 1e3 / calls)
    return statistics.median(ts)


def settle(lib, torch, s: Shape, plan: Plan, ws, ms=100.0):
    spent = 0.0
    while spent < ms:
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(16):
            run(lib, torch, s, plan, ws, i)
        e1.record()
        e1.synchronize()
        spent += e0.elapsed_time(e1)


def same_plan(a: Plan, b: Plan) -> bool:
    # a two-part plan (the planner's bulk + edge) is never the same as a one-launch candidate
    return (a.kernel, a.tile_cfg if a.kernel == KERNEL_TILED else -1, a.split_k, a.edge_dim, a.edge_at) == \
           (b.kernel, b.tile_cfg if b.kernel == KERNEL_TILED else -1, b.split_k, b.edge_dim, b.edge_at)


def tune_shape(lib, torch, M, N, K, first: bool):
    s = Shape(torch, M, N, K, seed=M * 7 + N * 3 + K)
    base = Plan()
    if lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(base)) != 0:
        raise RuntimeError(lib.wmma_last_error().decode())
    cands = candidate_plans(lib, M, N, K)
    wsize = max([p.workspace_bytes for p in cands] + [base.workspace_bytes])
    ws = torch.empty(wsize, dtype=torch.uint8, device="cuda") if wsize else None
    ref = run(lib, torch, s, base, ws, 0, out=torch.empty(M, N, device="cuda")).clone()
    scale = ref.abs().max().item() or 1.0
    settle(lib, torch, s, base, ws, ms=100.0 if first else 30.0)
    if not any(same_plan(p, base) for p in cands):
        cands.append(base)
    results = []
    for p in cands:
        out = run(lib, torch, s, p, ws, 0, out=torch.empty(M, N, device="cuda"))
        err = (out - ref).abs().max().item() / scale
        if not err <= 1e-3:
            raise RuntimeError(f"{M}x{N}x{K} {describe(p)}: max rel err {err:.3e} vs the planner")
        results.append((time_plan(lib, torch, s, p, ws), p))
    t_base = min(t for t, p in results if same_plan(p, base))
    results.sort(key=lambda r: r[0])
    best_t, best = results[0]
    del s, ws
    return {"M": M, "N": N, "K": K, "planner": describe(base), "planner_us": round(t_base, 2),
            "differs": not same_plan(best, base),
            "best": describe(best), "best_us": round(best_t, 2),
            "kernel": best.kernel, "tile_cfg": best.tile_cfg, "split": best.split_k,
            "candidates": [[describe(p), round(t, 2)] for t, p in results]}


def table_shapes(path=TABLE_PATH):
    """(M, N, K) of the entries of the table compiled into the planner now."""
    import re
    if not os.path.exists(path):
        return set()
    out = set()
    for m in re.finditer(r"^\s*\{(\d+), (\d+), (\d+), WMMA_KERNEL_", open(path).read(), re.M):
        out.add(tuple(int(x) for x in m.groups()))
    return out


def emit_table(entries, path=TABLE_PATH):
    lines = ["// Autotuned dispatch table -- generated by wmma_ops_amd/autotune.py; do not edit by hand.",
             "// Each entry is the fastest measured plan for one exact GEMM shape on a 256-CU MI355X",
             "// (kernel WMMA_KERNEL_*, tile WMMA_TILE_*, K split); shapes not listed use the planner's",
             "// heuristics.",
             "constexpr TunedPlan kTunedPlans[] = {"]
    for e in entries:
        kern = "WMMA_KERNEL_SKINNY" if e["kernel"] == KERNEL_SKINNY else "WMMA_KERNEL_TILED"
        lines.append(f"    {{{e['M']}, {e['N']}, {e['K']}, {kern}, {e['tile_cfg']}, {e['split']}}},"
                     f"  // {e['best']}: {e['best_us']} us (heuristic {e['planner']}: {e['planner_us']} us)")
    lines.append("    {-1, -1, -1, WMMA_KERNEL_TILED, 0, 1},  // sentinel (no shape matches)")
    lines.append("};")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--shapes", nargs="*", default=["baseline"],
                    help="'baseline' (BASELINE configs[0..2]) and/or M,N,K triples")
    ap.add_argument("--emit", default=None, help="write the C++ table here (e.g. %s)" % TABLE_PATH)
    ap.add_argument("--report", default=None, help="write one JSON line per shape here")
    ap.add_argument("--min-gain", type=float, default=0.03,
                    help="a shape enters the table when its best plan is this much faster")
    args = ap.parse_args(argv)
    import torch

    if not torch.cuda.is_available():
        sys.exit("autotune needs a GPU")
    shapes = []
    for s in args.shapes:
        if s == "baseline":
            shapes += baseline_shapes()
        else:
            shapes.append(tuple(int(x) for x in s.split(",")))
    lib = load_lib()
    tabled = table_shapes()
    report = open(args.report, "w") if args.report else None
    entries = []
    for idx, (M, N, K) in enumerate(shapes):
        r = tune_shape(lib, torch, M, N, K, first=idx == 0)
        line = json.dumps(r)
        print(f"{M}x{N}x{K}: planner {r['planner']} {r['planner_us']} us, best {r['best']} "
              f"{r['best_us']} us", flush=True)
        if report:
            report.write(line + "\n")
            report.flush()
        # a shape the compiled table already holds is planned from it, so the sweep sees
        # the table's plan as the planner's: keep its entry (now the fastest plan measured)
        if (r["differs"] and r["best_us"] < r["planner_us"] * (1.0 - args.min_gain)) or \
                (M, N, K) in tabled:
            entries.append(r)
    if args.emit:
        emit_table(entries, args.emit)
        print(f"{len(entries)} table entries -> {args.emit}", flush=True)


if __name__ == "__main__":
    main()
