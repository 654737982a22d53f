"""The allocation-free GEMM entry point, wmma_gemm_f16f32_noalloc, against wmma_gemm_f16f32.

On aligned shapes both run the same plan and kernels (on ragged ones see
test_noalloc_ragged_shapes); the only difference is where the split-K partial sums
live (the library's own device array instead of a caller workspace), so every output must
be bit-identical, and within the oracle's 1e-3 max-relative bound.  Each case makes two
calls in a row, the second on a smaller shape, so the second call runs on a scratch array
still holding the first call's partial sums.
"""
import ctypes
import os

import pytest
import torch

from oracle import gemm as og
from tests.conftest import report

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _lib():
    lib = ctypes.CDLL(os.path.join(ROOT, "wmma_ops_amd", "libwmma_ops_amd.so"))
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_last_error.restype = ctypes.c_char_p
    lib.wmma_gemm_workspace_size.restype = sz
    lib.wmma_gemm_workspace_size.argtypes = [i32, i32, i32, i32]
    lib.wmma_gemm_noalloc_scratch_bytes.restype = sz
    lib.wmma_gemm_f16f32.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32,
                                     f32, f32, i32, vp, sz, vp]
    lib.wmma_gemm_f16f32_noalloc.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32,
                                             f32, f32, i32, vp]
    return lib


# (first, second): the second call is smaller.  Plans: tiled 128x128 split 2 (14 MiB of
# partial sums) then skinny split 8; the tuned tiled split 8 (16 MiB) then skinny split 8;
# tiled 64x64 split 4 then a skinny split whose last part is shorter (K = 4104); shapes
# without a split (no scratch); a two-part plan whose edge is a skinny split 8 then a tiled
# split 4; tiled 64x64 split 8 on a narrow N.
PAIRS = [((128, 14336, 4096), (16, 4096, 4096)),
         ((128, 4096, 14336), (1, 4096, 4096)),
         ((64, 4096, 4096), (3, 1024, 4104)),
         ((1024, 1024, 1024), (300, 264, 640)),
         ((4100, 4096, 4096), (64, 4096, 4096)),
         ((300, 264, 4096), (40, 512, 2048))]


@pytest.mark.parametrize("first,second", PAIRS)
def test_noalloc_matches_workspace_entry_point(first, second):
    lib = _lib()
    cap = lib.wmma_gemm_noalloc_scratch_bytes()
    stream = torch.cuda.current_stream().cuda_stream
    for (M, N, K) in (first, second):
        report("noalloc", M=M, N=N, K=K)
        need = lib.wmma_gemm_workspace_size(M, N, K, -1)
        assert need <= cap
        g = torch.Generator().manual_seed(M + N + K)
        A = torch.randn(M, K, generator=g).half()
        B = (torch.randn(K, N, generator=g) * 0.05).half()
        C0 = torch.randn(M, N, generator=g)
        Ad, Bd = A.cuda(), B.cuda()
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        for alpha, beta, in_place in [(1.0, 0.0, False), (2.0, 0.5, False), (2.0, 0.5, True)]:
            Cref = C0.cuda()
            Cna = C0.cuda()
            out_ref = Cref if in_place else torch.empty(M, N, device="cuda")
            out_na = Cna if in_place else torch.empty(M, N, device="cuda")
            rc = lib.wmma_gemm_f16f32(Ad.data_ptr(), K, Bd.data_ptr(), N, Cref.data_ptr(), N,
                                      out_ref.data_ptr(), N, M, N, K, alpha, beta, -1,
                                      ws.data_ptr() if need else None, need, stream)
            assert rc == 0, lib.wmma_last_error()
            rc = lib.wmma_gemm_f16f32_noalloc(Ad.data_ptr(), K, Bd.data_ptr(), N, Cna.data_ptr(), N,
                                              out_na.data_ptr(), N, M, N, K, alpha, beta, -1, stream)
            assert rc == 0, lib.wmma_last_error()
            torch.cuda.synchronize()
            assert torch.equal(out_na, out_ref), (M, N, K, alpha, beta, in_place)
            ref = og.gemm_ref(A, B, alpha, beta, C0 if beta != 0.0 else None)
            assert og.max_rel_err(out_na, ref) <= 1e-3


def test_noalloc_scratch_covers_baseline_shapes():
    # every configs[1]/configs[2] GEMM shape fits the scratch array
    lib = _lib()
    cap = lib.wmma_gemm_noalloc_scratch_bytes()
    shapes = [(m, n, 4096) for m in (1, 16, 64, 128) for n in (4096, 11008, 14336)] + \
             [(m, 4096, 14336) for m in (1, 16, 64, 128)] + \
             [(s, s, s) for s in (512, 1024, 2048, 4096)] + [(4096, 4096, 2048)]
    for (M, N, K) in shapes:
        assert lib.wmma_gemm_workspace_size(M, N, K, -1) <= cap, (M, N, K)


# Ragged shapes (N or K off a multiple of 8): the allocation-free entry point makes no
# padded copies, so its operands go to the element-wise kernels (split-K partials in the
# scratch array) or, on the skinny kernel (1 x 4101 x 4096), its in-place B modes, while
# wmma_gemm_f16f32 with its full workspace repacks them for the vector kernels.  Both are
# held to the oracle's 1e-3 bar and to each other (products bit-equal: the same MFMA
# inputs in the same order; the alpha/beta epilogue to rounding).  Two calls in a row, the
# second smaller.
RAGGED_PAIRS = [((128, 4100, 4096), (7, 1027, 300)),
                ((300, 1000, 1004), (1, 4101, 4096))]


@pytest.mark.parametrize("first,second", RAGGED_PAIRS)
def test_noalloc_ragged_shapes(first, second):
    lib = _lib()
    stream = torch.cuda.current_stream().cuda_stream
    for (M, N, K) in (first, second):
        report("noalloc_ragged", M=M, N=N, K=K)
        need = lib.wmma_gemm_workspace_size(M, N, K, -1)
        g = torch.Generator().manual_seed(M * 3 + N + K)
        A = torch.randn(M, K, generator=g).half()
        B = (torch.randn(K, N, generator=g) * 0.05).half()
        C0 = torch.randn(M, N, generator=g)
        Ad, Bd = A.cuda(), B.cuda()
        ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
        prods = []
        for alpha, beta in [(1.0, 0.0), (2.0, 0.5)]:
            Cref, Cna = C0.cuda(), C0.cuda()
            out_ref, out_na = torch.empty(M, N, device="cuda"), torch.empty(M, N, device="cuda")
            rc = lib.wmma_gemm_f16f32(Ad.data_ptr(), K, Bd.data_ptr(), N, Cref.data_ptr(), N,
                                      out_ref.data_ptr(), N, M, N, K, alpha, beta, -1,
                                      ws.data_ptr(), need, stream)
            assert rc == 0, lib.wmma_last_error()
            rc = lib.wmma_gemm_f16f32_noalloc(Ad.data_ptr(), K, Bd.data_ptr(), N, Cna.data_ptr(), N,
                                              out_na.data_ptr(), N, M, N, K, alpha, beta, -1, stream)
            assert rc == 0, lib.wmma_last_error()
            torch.cuda.synchronize()
            ref = og.gemm_ref(A, B, alpha, beta, C0 if beta != 0.0 else None)
            assert og.max_rel_err(out_ref, ref) <= 1e-3
            assert og.max_rel_err(out_na, ref) <= 1e-3
            if beta == 0.0:
                assert torch.equal(out_na, out_ref), (M, N, K)
            else:
                assert og.max_rel_err(out_na, out_ref) <= 1e-6


class Plan(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int), ("tile_cfg", ctypes.c_int), ("tile_m", ctypes.c_int),
                ("tile_n", ctypes.c_int), ("split_k", ctypes.c_int), ("k_per_split", ctypes.c_int),
                ("grid", ctypes.c_int), ("workspace_bytes", ctypes.c_size_t),
                ("edge_dim", ctypes.c_int), ("edge_at", ctypes.c_int)]


# A shape whose planner plan needs more partial-sum space than the scratch array holds
# (512 x 4096 x 14336: 256x256 split 8, 64 MiB): the allocation-free entry point runs
# wmma_gemm_plan_make_within's plan for its array instead (128x128 split 2, 16 MiB),
# bit-equal to wmma_gemm_f16f32_plan with that plan and within the oracle's bar; then a
# smaller call, whose plan fits and is the planner's own.
def test_noalloc_plans_within_scratch():
    lib = _lib()
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_gemm_plan_make.argtypes = [i32] * 5 + [ctypes.POINTER(Plan)]
    lib.wmma_gemm_plan_make_within.argtypes = [i32] * 5 + [sz, ctypes.POINTER(Plan)]
    lib.wmma_gemm_f16f32_plan.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32,
                                          f32, f32, ctypes.POINTER(Plan), vp, sz, vp]
    cap = lib.wmma_gemm_noalloc_scratch_bytes()
    st = torch.cuda.current_stream().cuda_stream
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for i, (M, N, K) in enumerate([(512, 4096, 14336), (64, 4096, 4096)]):
        report("noalloc_within", M=M, N=N, K=K)
        full, within = Plan(), Plan()
        assert lib.wmma_gemm_plan_make(M, N, K, -1, cus, ctypes.byref(full)) == 0
        assert lib.wmma_gemm_plan_make_within(M, N, K, -1, cus, cap, ctypes.byref(within)) == 0
        assert 0 < within.workspace_bytes <= cap
        if i == 0 and cus == 256:
            assert full.workspace_bytes > cap
        A, B, C = _inputs(M, N, K, 21 + i)
        out_na = torch.empty(M, N, device="cuda")
        out_p = torch.empty(M, N, device="cuda")
        assert _noalloc(lib, A, B, C, out_na, M, N, K, 1.0, 0.0, st) == 0, lib.wmma_last_error()
        ws = torch.empty(within.workspace_bytes, dtype=torch.uint8, device="cuda")
        rc = lib.wmma_gemm_f16f32_plan(A.data_ptr(), K, B.data_ptr(), N, None, 0, out_p.data_ptr(), N,
                                       M, N, K, 1.0, 0.0, ctypes.byref(within), ws.data_ptr(),
                                       within.workspace_bytes, st)
        assert rc == 0, lib.wmma_last_error()
        torch.cuda.synchronize()
        assert torch.equal(out_na, out_p), (M, N, K)
        assert og.max_rel_err(out_na, og.gemm_ref(A.cpu(), B.cpu(), 1.0, 0.0, None)) <= 1e-3


def _noalloc(lib, A, B, C, out, M, N, K, alpha, beta, stream):
    return lib.wmma_gemm_f16f32_noalloc(A.data_ptr(), K, B.data_ptr(), N,
                                        C.data_ptr() if C is not None else None, N,
                                        out.data_ptr(), N, M, N, K, alpha, beta, -1, stream)


def _workspace_ref(lib, A, B, C, M, N, K, alpha, beta):
    need = lib.wmma_gemm_workspace_size(M, N, K, -1)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    out = torch.empty(M, N, device="cuda")
    rc = lib.wmma_gemm_f16f32(A.data_ptr(), K, B.data_ptr(), N,
                              C.data_ptr() if C is not None else None, N, out.data_ptr(), N, M, N, K,
                              alpha, beta, -1, ws.data_ptr(), need,
                              torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.wmma_last_error()
    torch.cuda.synchronize()
    return out


def _inputs(M, N, K, seed):
    g = torch.Generator().manual_seed(seed)
    return ((torch.randn(M, K, generator=g)).half().cuda(),
            (torch.randn(K, N, generator=g) * 0.05).half().cuda(),
            torch.randn(M, N, generator=g).cuda())


# Calls on two streams with no host synchronisation between them: the library orders them
# (the second stream waits for the event recorded after the first call), so each output is
# bit-identical to the workspace entry point's.  Several rounds alternate the streams and
# the shapes (both split-K plans, the second smaller).
def test_noalloc_two_streams_ordered():
    lib = _lib()
    shapes = [(128, 14336, 4096), (16, 4096, 4096), (64, 4096, 4096), (1, 4096, 4096)]
    ins = [_inputs(M, N, K, 7 + i) for i, (M, N, K) in enumerate(shapes)]
    refs = [_workspace_ref(lib, A, B, C, M, N, K, 2.0, 0.5) for (A, B, C), (M, N, K) in zip(ins, shapes)]
    s1, s2 = torch.cuda.Stream(), torch.cuda.Stream()
    torch.cuda.synchronize()
    for rnd in range(3):
        outs = []
        for i, ((A, B, C), (M, N, K)) in enumerate(zip(ins, shapes)):
            st = s1 if (i + rnd) % 2 == 0 else s2
            out = torch.empty(M, N, device="cuda")
            report("noalloc_streams", round=rnd, M=M, N=N, K=K)
            assert _noalloc(lib, A, B, C, out, M, N, K, 2.0, 0.5, st.cuda_stream) == 0, lib.wmma_last_error()
            outs.append(out)
        torch.cuda.synchronize()
        for out, ref in zip(outs, refs):
            assert torch.equal(out, ref)


# Free device memory is the same before and after a warmed-up call: the call allocates
# nothing (hipMemGetInfo through torch.cuda.mem_get_info).
def test_noalloc_allocates_nothing():
    lib = _lib()
    M, N, K = 128, 14336, 4096
    A, B, C = _inputs(M, N, K, 11)
    out = torch.empty(M, N, device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    assert _noalloc(lib, A, B, C, out, M, N, K, 1.0, 0.0, st) == 0
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    for _ in range(3):
        assert _noalloc(lib, A, B, C, out, M, N, K, 1.0, 0.0, st) == 0
    torch.cuda.synchronize()
    assert torch.cuda.mem_get_info()[0] == free0


_CAPTURE_SCRIPT = r"""
import ctypes, os, sys
import torch
sys.path.insert(0, {root!r})
from tests.test_zz_no_alloc import _lib, _inputs, _workspace_ref, _noalloc
lib = _lib()
M, N, K = 128, 4096, 14336          # tiled split-K: partial sums in the scratch array
A, B, C = _inputs(M, N, K, 5)
out = torch.empty(M, N, device="cuda")
torch.cuda.synchronize()
g = torch.cuda.CUDAGraph()
with torch.cuda.graph(g):            # the process's first noalloc call happens under capture
    rc = _noalloc(lib, A, B, C, out, M, N, K, 2.0, 0.5, torch.cuda.current_stream().cuda_stream)
assert rc == 0, lib.wmma_last_error()
ref = _workspace_ref(lib, A, B, C, M, N, K, 2.0, 0.5)
M2, N2, K2 = 16, 4096, 4096         # eager noalloc work between replays (skinny split-K)
A2, B2, C2 = _inputs(M2, N2, K2, 6)
ref2 = _workspace_ref(lib, A2, B2, C2, M2, N2, K2, 1.0, 0.0)
for rep in range(4):
    out.zero_()
    g.replay()
    torch.cuda.synchronize()
    assert torch.equal(out, ref), rep
    o2 = torch.empty(M2, N2, device="cuda")
    assert _noalloc(lib, A2, B2, C2, o2, M2, N2, K2, 1.0, 0.0, torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    assert torch.equal(o2, ref2), rep
print("CAPTURE_OK", flush=True)
"""


# A split-K noalloc GEMM captured into a graph, in a fresh process whose first noalloc call
# is the captured one (the scratch address is looked up under capture), replayed four times
# with eager noalloc calls in between; every replay equals the workspace entry point.
def test_noalloc_first_call_under_graph_capture():
    import subprocess
    import sys

    report("noalloc_capture", M=128, N=4096, K=14336)
    r = subprocess.run([sys.executable, "-c", _CAPTURE_SCRIPT.format(root=ROOT)], cwd=ROOT,
                       stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True, timeout=110)
    assert r.returncode == 0 and "CAPTURE_OK" in r.stdout, r.stdout[-3000:]
