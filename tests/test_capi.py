"""C-ABI boundary tests that need no GPU.

* the library loads and exports every function include/wmma_ops_amd.h declares;
* argument validation returns the documented status codes (nothing reaches the GPU:
  every case below fails validation before a launch);
* the host planner's decisions for the BASELINE shapes;
* the torch extension imports and reproduces the reference's argument errors
  (wmma_gemm.hip:1433-1446, 1522-1523).
"""
import ctypes
import os
import re

import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "wmma_ops_amd.h")
# WMMA_OPS_AMD_LIBRARY: another build of the same library (the host-sanitized one of
# `python -m wmma_ops_amd.build --sanitize`)
LIB = os.environ.get("WMMA_OPS_AMD_LIBRARY") or os.path.join(ROOT, "wmma_ops_amd", "libwmma_ops_amd.so")

OK, INVALID, UNSUPPORTED, MISALIGNED, WORKSPACE = 0, 1, 2, 3, 4


class Plan(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int), ("tile_cfg", ctypes.c_int), ("tile_m", ctypes.c_int),
                ("tile_n", ctypes.c_int), ("split_k", ctypes.c_int), ("k_per_split", ctypes.c_int),
                ("grid", ctypes.c_int), ("workspace_bytes", ctypes.c_size_t),
                ("edge_dim", ctypes.c_int), ("edge_at", ctypes.c_int)]


@pytest.fixture(scope="module")
def lib():
    L = ctypes.CDLL(LIB)
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    L.wmma_last_error.restype = ctypes.c_char_p
    L.wmma_gemm_f16f32.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, f32, f32, i32,
                                   vp, sz, vp]
    L.wmma_gemm_plan_make.argtypes = [i32, i32, i32, i32, i32, ctypes.POINTER(Plan)]
    L.wmma_gemm_workspace_size.restype = sz
    L.wmma_w4a16_workspace_size.restype = sz
    L.wmma_int4_prepack.argtypes = [vp, i32, i32, vp, vp]
    L.wmma_int4_unpack.argtypes = [vp, i32, i32, vp, vp]
    L.wmma_int4_prepack_params.argtypes = [vp, vp, i32, i32, i32, i32, vp, vp, vp]
    L.wmma_gemm_plan_custom.argtypes = [i32, i32, i32, i32, i32, i32, ctypes.POINTER(Plan)]
    L.wmma_int4_from_awq.argtypes = [vp, vp, i32, i32, i32, vp, vp, vp]
    L.wmma_int4_from_gptq_zeros.argtypes = [vp, i32, i32, i32, i32, vp, vp, vp]
    L.wmma_int4_permute_rows.argtypes = [vp, vp, i32, i32, vp, vp]
    L.wmma_w4a16_gemm_f16out.argtypes = [vp, i64, vp, vp, vp, i32, i32, i32, i32, i32, vp, i64, vp, sz, vp]
    L.wmma_gemm_f16f32_plan.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, f32, f32,
                                        ctypes.POINTER(Plan), vp, sz, vp]
    L.wmma_w4a16_gemm.argtypes = [vp, i64, vp, vp, vp, i32, i32, i32, i32, i32, vp, i64, vp, sz, vp]
    L.wmma_flash_attn_fwd.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, f32, i32, vp]
    L.wmma_flash_attn_fwd_gqa.argtypes = [vp, vp, vp, vp, i32, i32, i32, i32, i32, i32, f32, i32, vp]
    L.wmma_flash_attn_varlen_fwd.argtypes = [vp, vp, vp, vp, vp, vp] + [i32] * 8 + [f32, i32, vp]
    L.wmma_flash_attn_fwd_lse.argtypes = [vp, vp, vp, vp, vp] + [i32] * 6 + [f32, i32, vp]
    L.wmma_flash_attn_varlen_fwd_lse.argtypes = [vp] * 7 + [i32] * 8 + [f32, i32, vp]
    L.wmma_flash_attn_bwd_workspace_size.argtypes = [i32, i32, i32]
    L.wmma_flash_attn_bwd_workspace_size.restype = sz
    L.wmma_flash_attn_bwd.argtypes = [vp] * 10 + [sz] + [i32] * 6 + [f32, i32, vp]
    L.wmma_flash_attn_varlen_bwd.argtypes = [vp] * 12 + [sz] + [i32] * 8 + [f32, i32, vp]
    return L


def declared_functions(header=HEADER):
    text = open(header).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*(wmma_[A-Za-z0-9_]+)\s*\(",
                       text, flags=re.M)
    return sorted(set(names))


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for must in ["wmma_gemm_f16f32", "wmma_gemm_workspace_size", "wmma_int4_prepack",
                 "wmma_int4_unpack", "wmma_w4a16_gemm", "wmma_flash_attn_fwd", "wmma_last_error"]:
        assert must in names, names


def test_library_exports_every_declared_symbol(lib):
    missing = [n for n in declared_functions() if not hasattr(lib, n)]
    assert not missing, missing
    assert lib.wmma_abi_version() == 2
    assert ctypes.sizeof(Plan) == 48   # the C struct: 7 ints, size_t, 2 ints


def test_calibration_library_exports_its_header():
    # bench.py's measuring instruments (include/wmma_calib.h, libwmma_calib.so)
    calib = ctypes.CDLL(os.path.join(ROOT, "wmma_ops_amd", "libwmma_calib.so"))
    names = declared_functions(os.path.join(ROOT, "include", "wmma_calib.h"))
    assert names == ["wmma_calib_l2_stage", "wmma_calib_l2_stage_bytes",
                     "wmma_calib_lds_read", "wmma_calib_lds_read_bytes",
                     "wmma_calib_mfma_ceiling", "wmma_calib_mfma_ceiling_flops",
                     "wmma_calib_read_stream", "wmma_calib_read_stream_shape"], names
    assert not [n for n in names if not hasattr(calib, n)]
    calib.wmma_calib_l2_stage_bytes.restype = ctypes.c_double
    assert calib.wmma_calib_l2_stage_bytes(224, 64) == 224 * 64 * 8192.0
    calib.wmma_calib_mfma_ceiling_flops.restype = ctypes.c_double
    assert calib.wmma_calib_mfma_ceiling_flops(512, 1000) == 512 * 4 * 8 * 1000 * 2.0 * 32 * 32 * 16
    # argument checks return before any launch
    calib.wmma_calib_read_stream.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                             ctypes.c_void_p, ctypes.c_void_p]
    assert calib.wmma_calib_read_stream(None, 1024, 4, 0x10000, None) == 1
    assert calib.wmma_calib_read_stream(0x10000, 1024, 3, 0x10000, None) == 2
    calib.wmma_calib_read_stream_shape.argtypes = [ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int,
                                                   ctypes.c_int, ctypes.c_void_p, ctypes.c_void_p]
    assert calib.wmma_calib_read_stream_shape(0x10000, 1024, 128, 8, 0x10000, None) == 2
    assert calib.wmma_calib_read_stream_shape(0x10002, 1024, 256, 2, 0x10000, None) == 1
    calib.wmma_calib_lds_read.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                          ctypes.c_void_p]
    assert calib.wmma_calib_lds_read(3, 256, 10, 0x10000, None) == 2
    sz = ctypes.c_size_t
    calib.wmma_calib_l2_stage.argtypes = [ctypes.c_int] * 3 + [ctypes.c_void_p, sz, sz] + \
        [ctypes.c_int] * 2 + [ctypes.c_void_p] * 2
    assert calib.wmma_calib_l2_stage(4, 4, 1, 0x10000, 1 << 20, 100, 224, 64, 0x10000, None) == 1
    assert calib.wmma_calib_l2_stage(4, 4, 1, 0x10000, 1 << 19, 8192, 224, 64, 0x10000, None) == 1
    assert calib.wmma_calib_l2_stage(2, 4, 1, 0x10000, 1 << 20, 8192, 224, 64, 0x10000, None) == 2
    assert calib.wmma_calib_lds_read(0, 0, 10, 0x10000, None) == 1
    calib.wmma_calib_lds_read_bytes.restype = ctypes.c_double
    assert calib.wmma_calib_lds_read_bytes(2, 3) == 2 * 8 * 3 * 8192
    calib.wmma_calib_mfma_ceiling.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_void_p,
                                              ctypes.c_void_p, ctypes.c_void_p]
    assert calib.wmma_calib_mfma_ceiling(512, 3, None, 0x10000, None) == 1    # odd iters
    assert calib.wmma_calib_mfma_ceiling(512, 4, 0x10002, 0x10000, None) == 1  # misaligned


# ---------------------------------------------------------------- GEMM validation --
def gemm(lib, A=None, lda=64, B=None, ldb=64, Cin=None, ldcin=64, Cout=None, ldc=64, M=64, N=64,
         K=64, alpha=1.0, beta=0.0, cfg=-1, ws=None, wsb=0):
    return lib.wmma_gemm_f16f32(A, lda, B, ldb, Cin, ldcin, Cout, ldc, M, N, K, alpha, beta, cfg,
                                ws, wsb, None)


FAKE = 0x10000  # never dereferenced: every call below fails validation first


def test_gemm_validation_codes(lib):
    assert gemm(lib, M=-1) == INVALID
    assert b"negative" in lib.wmma_last_error()
    assert gemm(lib, cfg=6) == INVALID
    assert b"Invalid tile_config" in lib.wmma_last_error()
    assert gemm(lib, A=FAKE, B=FAKE, Cout=None) == INVALID          # NULL output
    assert gemm(lib, A=None, B=FAKE, Cout=FAKE) == INVALID          # NULL A with K > 0
    assert gemm(lib, A=FAKE, B=FAKE, Cout=FAKE, lda=32) == INVALID  # lda < K
    assert gemm(lib, A=FAKE, B=FAKE, Cout=FAKE, ldb=32) == INVALID  # ldb < N
    assert gemm(lib, A=FAKE, B=FAKE, Cout=FAKE, ldc=32) == INVALID  # ldc < N
    assert gemm(lib, A=FAKE, B=FAKE, Cout=FAKE, Cin=FAKE, beta=1.0, ldcin=8) == INVALID
    # split-K shape without workspace
    assert gemm(lib, A=FAKE, B=FAKE, Cout=FAKE, M=1, N=4096, K=4096, lda=4096, ldb=4096, ldc=4096) == WORKSPACE
    assert b"workspace" in lib.wmma_last_error()
    need = lib.wmma_gemm_workspace_size(1, 4096, 4096, -1)
    assert need > 0
    assert gemm(lib, A=FAKE, B=FAKE, Cout=FAKE, M=1, N=4096, K=4096, lda=4096, ldb=4096, ldc=4096,
                ws=FAKE, wsb=need - 4) == WORKSPACE
    # empty output is a no-op success, no pointers needed
    assert gemm(lib, M=0) == OK
    assert gemm(lib, N=0) == OK


def test_plan_make(lib):
    p = Plan()
    assert lib.wmma_gemm_plan_make(4096, 4096, 4096, -1, 256, ctypes.byref(p)) == OK
    assert (p.kernel, p.tile_m, p.tile_n, p.split_k, p.grid, p.workspace_bytes) == (0, 256, 256, 1, 256, 0)
    assert lib.wmma_gemm_plan_make(1, 14336, 4096, -1, 256, ctypes.byref(p)) == OK
    assert p.kernel == 1 and p.split_k >= 2 and p.k_per_split % 64 == 0
    assert p.workspace_bytes == p.split_k * 1 * 14336 * 4
    for cfg, (bm, bn) in {0: (64, 64), 1: (128, 64), 2: (256, 64), 3: (128, 128), 4: (256, 128), 5: (256, 256)}.items():
        assert lib.wmma_gemm_plan_make(1000, 1000, 1000, cfg, 256, ctypes.byref(p)) == OK
        assert (p.tile_m, p.tile_n, p.split_k) == (bm, bn, 1)
    assert lib.wmma_gemm_plan_make(10, 10, 10, 9, 256, ctypes.byref(p)) == INVALID
    assert lib.wmma_gemm_plan_make(10, 10, 10, -1, 256, None) == INVALID
    # M <= 16 with K > 1024: the streaming kernel with its own split rule
    for (M, N, K), split in {(1, 4096, 4096): 8, (16, 4096, 4096): 8, (16, 14336, 4096): 2,
                             (16, 4096, 14336): 8}.items():
        assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
        assert (p.kernel, p.tile_m, p.tile_n, p.split_k) == (1, 16, 128, split), (M, N, K)
    # every other M <= 768: the fitted launch model's choice (kernel, tile, split), each the
    # fastest plan measured at that shape in the sweep the model was fitted on, with the
    # previous heuristics' time beside it: K <= 1024 never splits; few rows and long K split
    # deep; the streaming kernel where it still wins
    MODEL = {(8, 4096, 1024): (0, 0, 1),        # 9.1 us (skinny split 4: 10.7)
             (24, 14336, 1024): (0, 0, 1),      # 10.5 (skinny split 2: 14.0)
             (32, 4096, 4096): (0, 0, 4),       # 14.6 (skinny split 8: 15.0)
             (32, 14336, 4096): (1, -1, 2),     # 29.1, unchanged
             (64, 1024, 1024): (0, 0, 1), (128, 4096, 512): (0, 0, 1),
             (48, 1024, 14336): (0, 0, 16),     # 14.4 (64x64 split 4: 27.2)
             (128, 1024, 14336): (0, 1, 16),    # 17.7 (64x64 split 4: 27.2)
             (96, 4096, 14336): (0, 3, 8),      # 37.2 (64x64 split 2: 49.0)
             (256, 4096, 14336): (0, 3, 4),     # 53.8 (64x64 split 1: 83.5)
             (768, 14336, 1024): (0, 5, 1)}     # 33.2 (128x128 split 1: 46.2)
    for (M, N, K), want in MODEL.items():
        assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
        assert (p.kernel, p.tile_cfg, p.split_k) == want, (M, N, K)
        assert p.edge_dim == 0
    # a split only from K = 2048 on, at least 256 of K per part, within one wave of the CUs
    for M in (1, 8, 24, 40, 96, 200, 768):
        for N in (512, 4096, 14336):
            for K in (512, 1024, 2048, 8192):
                assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
                if p.split_k > 1:
                    assert K >= 2048 and K // p.split_k >= 192 and p.grid <= 3 * 256, (M, N, K)


def test_plan_make_within(lib):
    # the planner's choice among plans whose partial sums fit a budget: the same plan when it
    # fits, else another that does; a budget of 0 leaves only unsplit plans
    lib.wmma_gemm_plan_make_within.argtypes = [ctypes.c_int] * 5 + [ctypes.c_size_t,
                                                                    ctypes.POINTER(Plan)]
    p, q = Plan(), Plan()
    for (M, N, K) in [(512, 4096, 14336), (256, 4096, 14336), (64, 4096, 4096), (1, 4096, 4096),
                      (4100, 4096, 4096), (128, 4096, 14336), (16, 14336, 4096), (2048, 1024, 8192)]:
        assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
        for cap in (0, 1 << 20, 16 << 20, 32 << 20, 1 << 40):
            assert lib.wmma_gemm_plan_make_within(M, N, K, -1, 256, cap, ctypes.byref(q)) == OK
            assert q.workspace_bytes <= cap, (M, N, K, cap)
            if p.workspace_bytes <= cap:
                assert (q.kernel, q.tile_cfg, q.split_k, q.edge_dim, q.edge_at) == \
                    (p.kernel, p.tile_cfg, p.split_k, p.edge_dim, p.edge_at), (M, N, K, cap)
    assert lib.wmma_gemm_plan_make_within(512, 4096, 14336, -1, 256, 0, ctypes.byref(q)) == OK
    assert q.split_k == 1 and q.workspace_bytes == 0
    assert lib.wmma_gemm_plan_make_within(10, 10, 10, -1, 256, 0, None) == INVALID
    assert lib.wmma_gemm_plan_make_within(-1, 10, 10, -1, 256, 0, ctypes.byref(q)) == INVALID


class W4Plan(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_int), ("split_k", ctypes.c_int), ("k_per_split", ctypes.c_int),
                ("workspace_bytes", ctypes.c_size_t)]


def test_gemm_workspace_size_covers_repacked_operands(lib):
    # Contiguous operands: K or N off a multiple of 8 adds a zero-padded copy of A [M][K8]
    # and/or B [K][N8] (256-byte rounded, plus 256 bytes of alignment slack) to the split-K
    # partial sums -- except B under the skinny kernel (M <= 32), which reads it in place;
    # aligned shapes need only the partial sums.
    r256 = lambda x: (x + 255) // 256 * 256
    p = Plan()
    for M, N, K in [(4096, 4100, 4096), (4096, 4096, 4100), (4095, 4101, 4099), (1, 4100, 4096),
                    (13, 1027, 300), (1, 1, 1), (4096, 4096, 4096), (1, 4096, 4096),
                    (17, 4100, 4096)]:
        assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
        K8, N8 = (K + 7) // 8 * 8, (N + 7) // 8 * 8
        extra = 0
        b_copy = N % 8 != 0 and p.kernel != 1
        if K % 8 or b_copy:
            extra = 256 + (r256(M * K8 * 2) if K % 8 else 0) + (r256(K * N8 * 2) if b_copy else 0)
        assert lib.wmma_gemm_workspace_size(M, N, K, -1) == p.workspace_bytes + extra, (M, N, K)
    assert lib.wmma_gemm_workspace_size(0, 4100, 4096, -1) == 0
    assert lib.wmma_gemm_workspace_size(16, 4100, 0, -1) == 0


# Bulk + edge plans, pinned to decisions measured on MI355X (each two-part plan below ran
# 7-31% faster than the planner's previous one-launch plan; the one-launch shapes either
# fill whole waves or gained nothing from a split).
TWO_PART = {(4100, 4096, 4096): (1, 4096), (4352, 4096, 4096): (1, 4096),
            (5000, 4096, 4096): (1, 4096), (6000, 4096, 4096): (1, 4096),
            (4096, 4104, 4096): (2, 4096), (4096, 5000, 4096): (2, 4096),
            (9192, 4096, 4096): (1, 8192), (2560, 14336, 4096): (1, 2304),
            (4096, 14336, 4096): (2, 12288), (4100, 4096, 1024): (1, 4096)}
ONE_LAUNCH = [(7000, 4096, 4096), (3000, 4096, 4096), (2100, 4096, 4096), (4100, 14336, 4096),
              (512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
              (4096, 4096, 2048), (8192, 8192, 4096), (1, 4100, 4096), (128, 4100, 4096)]


def test_plan_two_part_decisions(lib):
    p, e = Plan(), Plan()
    for (M, N, K), (dim, at) in TWO_PART.items():
        assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
        assert (p.edge_dim, p.edge_at) == (dim, at), (M, N, K)
        # the bulk: 256x256 tiles, no split, the whole tile rows (columns) that fit in the
        # whole waves of the 256 CUs
        assert (p.kernel, p.tile_cfg, p.split_k) == (0, 5, 1)
        tm, tn = -(-M // 256), -(-N // 256)
        whole = tm * tn // 256 * 256
        across = tn if dim == 1 else tm
        assert at % 256 == 0 and p.grid == (at // 256) * across
        assert whole - across < p.grid <= whole
        # the edge: the planner's own one-launch plan for the rest
        em, en = (M - at, N) if dim == 1 else (M, N - at)
        assert lib.wmma_gemm_plan_make(em, en, K, -1, 256, ctypes.byref(e)) == OK
        assert e.edge_dim == 0 and p.workspace_bytes == e.workspace_bytes
        # an explicit tile never splits in two
        assert lib.wmma_gemm_plan_make(M, N, K, 3, 256, ctypes.byref(p)) == OK and p.edge_dim == 0
    for (M, N, K) in ONE_LAUNCH:
        assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
        assert (p.edge_dim, p.edge_at) == (0, 0), (M, N, K)


def test_w4a16_plan_make(lib):
    lib.wmma_w4a16_plan_make.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(W4Plan)]
    p = W4Plan()

    def plan(M, N, K, G=128):
        assert lib.wmma_w4a16_plan_make(M, N, K, G, 256, ctypes.byref(p)) == OK
        return (p.kernel, p.split_k, p.k_per_split, p.workspace_bytes)

    assert plan(1, 14336, 4096)[:2] == (0, 1)          # decode on the matrix pipe
    assert plan(4, 4096, 4096)[:2] == (0, 1)
    assert plan(3, 4096, 14336)[:2] == (0, 1)          # ... also past one round (49.9 KB LDS)
    assert plan(4, 4096, 8192)[:2] == (0, 1)           # (66.6 KB)
    assert plan(1, 1024, 4096)[:2] == (0, 1)           # ... at narrow N (64 slices) too
    assert plan(4, 256, 4096)[:2] == (0, 1)
    assert plan(4, 1536, 14336)[:2] == (0, 1)
    assert plan(2, 1024, 14336)[:2] == (0, 1)
    assert plan(2, 256, 8192)[:2] == (0, 1)
    assert plan(1, 256, 14336)[:2] == (0, 1)
    assert plan(3, 256, 8192)[0] == 4                  # narrow N, long K: skinny, K split
    assert plan(2, 512, 11008)[0] == 4
    assert plan(4, 1024, 14336)[0] == 4
    assert plan(3, 1024, 11008)[0] == 4
    assert plan(4, 1024, 8192)[:2] == (0, 1)           # (K under 10240 at N = 1024)
    assert plan(3, 512, 6144)[:2] == (0, 1)
    assert plan(16, 14336, 4096) == (4, 1, 4096, 0)    # skinny, 448 tiles: no split
    assert plan(16, 4096, 4096) == (4, 1, 4096, 0)     # skinny, 256 16-column workgroups
    assert plan(16, 2048, 4096) == (4, 1, 4096, 0)     # 128 of them: half the CUs, no split
    assert plan(16, 1024, 4096) == (4, 1, 4096, 0)     # 64 of them: still no split
    assert plan(5, 256, 2048) == (4, 1, 2048, 0)       # K <= 2048: never a split
    assert plan(16, 4096, 14336) == (4, 7, 2048, 7 * 16 * 4096 * 4)   # long K: split
    assert plan(32, 4096, 14336) == (4, 7, 2048, 7 * 32 * 4096 * 4)
    assert plan(32, 1024, 2048) == (6, 1, 2048, 0)     # the rows kernel beats it at short K
    assert plan(17, 14336, 8192) == (6, 1, 8192, 0)    # ... and at wide N
    assert plan(128, 14336, 4096)[:2] == (5, 1)        # 224 tiles of 64x128: no split
    assert plan(256, 4096, 4096)[:2] == (5, 2)         # 128 tiles: 2 ways
    assert plan(48, 4096, 8192)[:2] == (5, 8)          # 32 tiles: 8 ways (the cap)
    assert plan(64, 11008, 4096)[:2] == (5, 2)         # 86 tiles: 2 ways
    assert plan(1024, 1024, 1024)[:2] == (5, 1)        # K <= 1024: never a split
    # the rows kernel: short K, few columns, no split
    assert plan(128, 4096, 4096) == (6, 1, 4096, 0)
    assert plan(64, 4096, 4096) == (6, 1, 4096, 0)
    assert plan(128, 4096, 1024) == (6, 1, 1024, 0)
    assert plan(512, 1024, 2048) == (6, 1, 2048, 0)
    assert plan(33, 1024, 4096) == (6, 1, 4096, 0)
    assert plan(64, 1024, 4096, 512) == (6, 1, 4096, 0)
    assert plan(64, 1024, 4096, 64)[0] == 5            # ... for G = 128 * 2^j only
    assert plan(128, 4096, 8192)[:2] == (5, 4)         # longer K: LDS-DMA tiles again
    assert plan(2048, 1024, 1024)[:2] == (5, 1)        # M > 1024: the tile rules
    # skinny with 64-column workgroups (128 of them) and a 4-way K split
    assert plan(16, 8192, 8192) == (4, 4, 2048, 4 * 16 * 8192 * 4)
    assert plan(2048, 4096, 4096)[:2] == (5, 1)        # 512 tiles of 128x128, no split
    assert plan(1024, 14336, 4096)[:2] == (5, 1)       # 448 tiles of 128x256
    assert plan(32, 14336, 2048)[0] == 4
    assert plan(33, 14336, 4096)[0] == 5               # LDS-DMA GEMM beyond 32 rows ...
    assert plan(64, 4096, 4608, 384)[0] == 3           # ... for group sizes 2^j only
    assert plan(2048, 14336, 4096)[:2] == (5, 1)
    assert plan(16, 14336, 4096, 64)[0] == 3           # G not 128 * 2^j: older tiled kernel
    assert plan(16, 14336, 4608, 384)[0] == 3
    for M, N, K, G in [(5, 1024, 4224, 128), (17, 352, 1536, 256), (2048, 14336, 4096, 128)]:
        k, s, kps, ws = plan(M, N, K, G)
        assert kps * (s - 1) < K <= kps * s
        assert ws == (s * M * N * 4 if s > 1 else 0)
    assert lib.wmma_w4a16_plan_make(16, 100, 4096, 128, 256, ctypes.byref(p)) == INVALID
    assert lib.wmma_w4a16_plan_make(16, 4096, 4096, 128, 256, None) == INVALID


@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (16, 11008, 4096), (64, 14336, 4096),
                                   (128, 4096, 14336), (512, 512, 512), (1024, 1024, 1024),
                                   (2048, 2048, 2048), (4096, 4096, 2048), (300, 70, 5000)])
def test_plan_split_covers_k(lib, M, N, K):
    p = Plan()
    assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
    assert p.k_per_split * (p.split_k - 1) < K <= p.k_per_split * p.split_k
    if p.split_k > 1:
        assert p.k_per_split % 64 == 0
        assert p.workspace_bytes == p.split_k * M * N * 4
    else:
        assert p.workspace_bytes == 0


# ---------------------------------------------------------------- INT4 / flash validation --
def test_int4_validation_codes(lib):
    assert lib.wmma_int4_prepack(FAKE, 100, 64, FAKE, None) == UNSUPPORTED   # K % 64
    assert lib.wmma_int4_prepack(FAKE, 128, 48, FAKE, None) == UNSUPPORTED   # N % 32
    assert lib.wmma_int4_prepack(None, 128, 64, FAKE, None) == INVALID
    assert lib.wmma_int4_prepack(FAKE, 128, 64, FAKE + 4, None) == MISALIGNED
    assert lib.wmma_int4_unpack(FAKE, 12, 64, FAKE, None) == INVALID
    w = lambda **kw: lib.wmma_w4a16_gemm(kw.get("A", FAKE), kw.get("lda", 4096), FAKE, FAKE, FAKE,
                                         kw.get("zf", 0), kw.get("M", 1), 4096, 4096, kw.get("G", 128),
                                         FAKE, 4096, kw.get("ws", None), kw.get("wsb", 0), None)
    assert w(G=48) == UNSUPPORTED
    assert w(G=0) == UNSUPPORTED
    assert w(zf=7) == INVALID
    assert w(A=FAKE + 2) == MISALIGNED
    assert w(lda=100) == INVALID
    assert w(M=0) == OK


TUNED = os.path.join(ROOT, "wmma_ops_amd", "csrc", "tuned_table.inc")


def tuned_entries():
    pat = re.compile(r"\{(-?\d+), (-?\d+), (-?\d+), WMMA_KERNEL_(TILED|SKINNY), (-?\d+), (\d+)\}")
    out = []
    for m in pat.finditer(open(TUNED).read()):
        M, N, K = int(m.group(1)), int(m.group(2)), int(m.group(3))
        if M >= 0:
            out.append((M, N, K, 1 if m.group(4) == "SKINNY" else 0, int(m.group(5)), int(m.group(6))))
    return out


def test_tuned_table_drives_the_planner(lib):
    # every autotuned shape gets exactly its measured plan on a 256-CU device, and the
    # heuristics elsewhere (another CU count, or an explicit tile)
    entries = tuned_entries()
    assert entries, "the autotuned table is empty"
    for M, N, K, kernel, tile, split in entries:
        p = Plan()
        assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == OK
        assert (p.kernel, p.split_k) == (kernel, split)
        if kernel == 0:
            assert p.tile_cfg == tile
        q = Plan()
        assert lib.wmma_gemm_plan_custom(M, N, K, kernel, tile, split, ctypes.byref(q)) == OK
        assert (q.k_per_split, q.grid, q.workspace_bytes) == (p.k_per_split, p.grid, p.workspace_bytes)


def test_plan_custom_validation(lib):
    p = Plan()
    assert lib.wmma_gemm_plan_custom(64, 64, 4096, 0, 3, 4, ctypes.byref(p)) == OK
    assert (p.kernel, p.tile_cfg, p.split_k, p.k_per_split) == (0, 3, 4, 1024)
    assert p.workspace_bytes == 4 * 64 * 64 * 4
    assert lib.wmma_gemm_plan_custom(64, 64, 4096, 0, 6, 1, ctypes.byref(p)) == INVALID   # no such tile
    assert lib.wmma_gemm_plan_custom(65, 64, 4096, 1, -1, 2, ctypes.byref(p)) == INVALID  # skinny: M <= 64
    assert lib.wmma_gemm_plan_custom(16, 64, 128, 1, -1, 4, ctypes.byref(p)) == INVALID   # K < 64 per split
    assert lib.wmma_gemm_plan_custom(16, 64, 4096, 2, 0, 1, ctypes.byref(p)) == INVALID   # no such kernel
    assert lib.wmma_gemm_plan_custom(16, 64, 4096, 0, 0, 33, ctypes.byref(p)) == INVALID  # split > 32
    # a plan made for another shape is rejected before anything is launched
    assert lib.wmma_gemm_plan_custom(64, 64, 4096, 0, 0, 2, ctypes.byref(p)) == OK
    assert lib.wmma_gemm_f16f32_plan(FAKE, 2048, FAKE, 64, None, 64, FAKE, 64, 64, 64, 2048, 1.0, 0.0,
                                     ctypes.byref(p), FAKE, 1 << 20, None) == INVALID
    assert b"plan does not describe this shape" in lib.wmma_last_error()


def test_awq_and_f16out_validation_codes(lib):
    a = lambda **kw: lib.wmma_int4_from_awq(kw.get("q", FAKE), FAKE, kw.get("K", 256), kw.get("N", 64),
                                            kw.get("G", 64), FAKE, FAKE, None)
    assert a(K=100) == INVALID             # K % 8
    assert a(G=96) == INVALID              # group size must divide K
    assert a(q=None) == INVALID
    assert a(q=FAKE + 2) == MISALIGNED
    w = lambda Y: lib.wmma_w4a16_gemm_f16out(FAKE, 256, FAKE, FAKE, FAKE, 0, 1, 64, 256, 64, Y, 64,
                                             None, 0, None)
    assert w(FAKE + 1) == MISALIGNED       # fp16 Y must be 2-byte aligned


def test_prepack_params_validation_codes(lib):
    f = lambda **kw: lib.wmma_int4_prepack_params(kw.get("s", FAKE), FAKE, kw.get("zf", 0), kw.get("K", 256),
                                                  kw.get("N", 64), kw.get("G", 64), FAKE, kw.get("zo", FAKE), None)
    assert f(N=48) == UNSUPPORTED          # N % 32
    assert f(G=96) == INVALID              # group size must divide K
    assert f(zf=2) == INVALID              # already sliced
    assert f(s=None) == INVALID
    assert f(s=FAKE + 1) == MISALIGNED
    assert f(zo=FAKE + 2) == MISALIGNED


def test_flash_validation_codes(lib):
    f = lambda **kw: lib.wmma_flash_attn_fwd(FAKE, FAKE, FAKE, kw.get("O", FAKE), 1, 1, kw.get("S", 128),
                                             kw.get("S", 128), kw.get("D", 128), kw.get("scale", 0.1), 0, None)
    # head dims: multiples of 8 from 8 to 256 (the torch layer pads other sizes)
    for D in (0, 4, 100, 264, 512):
        assert f(D=D) == UNSUPPORTED, D
    assert b"multiples of 8 from 8 to 256" in lib.wmma_last_error()
    assert f(scale=0.0) == INVALID
    assert f(scale=float("nan")) == INVALID
    assert f(O=None) == INVALID
    assert f(O=FAKE + 8) == MISALIGNED
    assert f(S=0) == OK
    g = lambda H, Hkv: lib.wmma_flash_attn_fwd_gqa(FAKE, FAKE, FAKE, FAKE, 1, H, Hkv, 128, 128, 128,
                                                    0.1, 0, None)
    assert g(8, 3) == INVALID                      # key/value heads must divide query heads
    assert b"must divide" in lib.wmma_last_error()
    assert g(8, 0) == INVALID
    assert g(0, 0) == OK                           # no heads: nothing to do
    v = lambda **kw: lib.wmma_flash_attn_varlen_fwd(FAKE, FAKE, FAKE, FAKE, kw.get("cu", FAKE), FAKE, 2,
                                                    8, kw.get("Hkv", 2), 100, 100, 64, 64, 128, 0.1, 0, None)
    assert v(Hkv=3) == INVALID
    assert v(cu=None) == INVALID
    assert v(cu=FAKE + 2) == MISALIGNED


def test_flash_split_workspace(lib):
    # the decoding split: 0 bytes for the BASELINE prefill shape (its query blocks fill the
    # CUs); for one query against 4096 keys on 32 heads, 8 chunks of 512 keys, each holding
    # fp32 O (D values) plus the running max and row sum per query row
    ws = lib.wmma_flash_attn_fwd_workspace_size
    ws.restype = ctypes.c_size_t
    ws.argtypes = [ctypes.c_int] * 7
    assert ws(4, 32, 32, 4096, 4096, 128, 0) == 0
    assert ws(1, 32, 32, 1, 4096, 128, 0) == 8 * 32 * 1 * (128 + 2) * 4
    assert ws(1, 32, 32, 1, 600, 128, 0) == 2 * 32 * (128 + 2) * 4    # chunks of >= 4 tiles
    assert ws(1, 32, 32, 1024, 1024, 128, 0) == 0                    # partial sums too large
    assert ws(1, 32, 32, 1, 4096, 100, 0) == 0 and ws(0, 32, 32, 1, 4096, 128, 0) == 0
    # grouped-query heads without a causal mask run as one sequence per K/V head: 8 rows of
    # 4 queries, 32 chunks of 256 keys; with the mask, 32 heads of one query, 8 chunks
    assert ws(1, 32, 8, 1, 8192, 128, 0) == 32 * (8 * 4) * (128 + 2) * 4
    assert ws(1, 32, 8, 1, 8192, 128, 1) == 8 * 32 * (128 + 2) * 4
    f = lib.wmma_flash_attn_fwd_ws
    f.argtypes = [ctypes.c_void_p] * 5 + [ctypes.c_int] * 6 + [ctypes.c_float, ctypes.c_int,
                                                                ctypes.c_void_p, ctypes.c_size_t, ctypes.c_void_p]
    # a misaligned workspace large enough to be used is rejected before any launch
    assert f(FAKE, FAKE, FAKE, FAKE, None, 1, 32, 32, 1, 4096, 128, 0.1, 0, FAKE + 4, 1 << 20, None) == MISALIGNED
    assert f(None, FAKE, FAKE, FAKE, None, 1, 32, 32, 1, 4096, 128, 0.1, 0, FAKE, 1 << 20, None) == INVALID


def test_flash_bwd_split_workspace(lib):
    # grouped-query backward with few K/V heads: the row statistics (256-byte rounded) plus
    # fp32 partial dK and dV per part; unchanged where the dK/dV workgroups fill the CUs
    lib.wmma_flash_attn_bwd_workspace_size.restype = ctypes.c_size_t
    f = lib.wmma_flash_attn_bwd_split_workspace_size
    f.restype = ctypes.c_size_t
    f.argtypes = [ctypes.c_int] * 7
    stats = lambda B, H, S: 2 * 4 * B * H * S
    part = lambda gs, B, Hkv, S, D: 2 * gs * B * Hkv * S * D * 4
    # 8 K/V heads x 16 key blocks = 128 workgroups: 2 parts of 2 query heads each
    assert f(1, 32, 8, 2048, 2048, 128, 0) == stats(1, 32, 2048) + part(2, 1, 8, 2048, 128)
    assert f(1, 32, 8, 2048, 2048, 128, 1) == stats(1, 32, 2048) + part(2, 1, 8, 2048, 128)
    # 2 x 4 K/V heads x 8 key blocks = 64 workgroups: 4 parts
    assert f(2, 32, 4, 1024, 1024, 128, 1) == stats(2, 32, 1024) + part(4, 2, 4, 1024, 128)
    assert f(4, 32, 32, 4096, 4096, 128, 1) == stats(4, 32, 4096)     # no group
    # 256 workgroups fill one wave: unsplit without a mask, 2 parts with one
    assert f(1, 32, 8, 4096, 4096, 128, 0) == stats(1, 32, 4096)
    assert f(1, 32, 8, 4096, 4096, 128, 1) == stats(1, 32, 4096) + part(2, 1, 8, 4096, 128)
    assert f(1, 32, 8, 8192, 8192, 128, 1) == stats(1, 32, 8192)      # two waves already
    # D = 64 (256 keys per workgroup): 4 workgroups, one part per query head
    assert f(1, 32, 1, 1024, 1024, 64, 0) == stats(1, 32, 1024) + part(32, 1, 1, 1024, 64)
    assert f(1, 8, 2, 0, 100, 64, 0) == 0


def test_flash_training_validation_codes(lib):
    # forward with log-sum-exp
    f = lambda **kw: lib.wmma_flash_attn_fwd_lse(FAKE, FAKE, FAKE, FAKE, kw.get("lse", FAKE), 1, 4, 2,
                                                 128, 128, kw.get("D", 128), 0.1, 0, None)
    for D in (4, 100, 264):
        assert f(D=D) == UNSUPPORTED, D
    assert f(lse=FAKE + 2) == MISALIGNED
    # workspace: two fp32 statistics per query row
    assert lib.wmma_flash_attn_bwd_workspace_size(4, 32, 4096) == 2 * 4 * 4 * 32 * 4096
    assert lib.wmma_flash_attn_bwd_workspace_size(0, 32, 4096) == 0
    need = lib.wmma_flash_attn_bwd_workspace_size(1, 4, 128)

    def bwd(**kw):
        ptr = lambda k: kw.get(k, FAKE)
        return lib.wmma_flash_attn_bwd(ptr("dO"), FAKE, FAKE, FAKE, ptr("O"), ptr("lse"), ptr("dQ"), FAKE,
                                       FAKE, ptr("ws"), kw.get("wsb", need), 1, 4, kw.get("Hkv", 2),
                                       kw.get("Sq", 128), kw.get("Sk", 128), kw.get("D", 128),
                                       kw.get("scale", 0.1), 0, None)
    assert bwd(D=36) == UNSUPPORTED
    assert bwd(D=264) == UNSUPPORTED
    assert b"from 8 to 256" in lib.wmma_last_error()
    assert bwd(Hkv=3) == INVALID
    assert bwd(scale=-1.0) == INVALID
    assert bwd(dO=None) == INVALID
    assert bwd(lse=None) == INVALID
    assert bwd(dQ=FAKE + 8) == MISALIGNED
    assert bwd(lse=FAKE + 1) == MISALIGNED
    assert bwd(ws=None) == WORKSPACE
    assert bwd(wsb=need - 4) == WORKSPACE
    assert b"needed" in lib.wmma_last_error()
    assert bwd(Sk=0) == INVALID                   # queries without keys
    assert bwd(Sq=0, Sk=0) == OK                  # nothing to do
    # variable length
    vb = lambda **kw: lib.wmma_flash_attn_varlen_bwd(
        FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, kw.get("cu", FAKE), FAKE, FAKE,
        kw.get("wsb", 2 * 4 * 8 * 100), 2, 8, kw.get("Hkv", 2), 100, 100, 64, 64, 128, 0.1, 0, None)
    assert vb(Hkv=3) == INVALID
    assert vb(cu=None) == INVALID
    assert vb(cu=FAKE + 2) == MISALIGNED
    assert vb(wsb=16) == WORKSPACE


# ---------------------------------------------------------------- torch layer on CPU --
def test_torch_extension_reference_errors(wo):
    A = torch.zeros(4, 8, dtype=torch.float16)
    B = torch.zeros(8, 4, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="Inputs must be CUDA tensors"):
        wo.matmul(A, B)
    with pytest.raises(RuntimeError, match="Inputs must be CUDA tensors"):
        wo.matmul_tiled(A, B, 1)
    with pytest.raises(RuntimeError, match="Inputs must be CUDA tensors"):
        wo.gemm(A, B, alpha=2.0, beta=0.5, C=None)
    with pytest.raises(RuntimeError, match="Inputs must be CUDA tensors"):
        wo.flash_attention(torch.zeros(1, 1, 4, 64, dtype=torch.float16),
                           torch.zeros(1, 1, 4, 64, dtype=torch.float16),
                           torch.zeros(1, 1, 4, 64, dtype=torch.float16))
    for name in ["matmul", "matmul_adaptive", "matmul_tiled", "gemm", "gemm_inplace", "gemm_adaptive",
                 "flash_attention", "flash_attention_forward", "flash_attention_backward",
                 "flash_attention_varlen_forward", "flash_attention_varlen_backward",
                 "prepack_int4", "matmul_int4", "unpack_int4",
                 "matmul_kunroll", "matmul_hilbert", "matmul_opt", "matmul_pingpong"]:
        assert callable(getattr(wo, name))


def test_torch_plan_binding(wo):
    assert wo.gemm_plan(4096, 4096, 4096) == [0, 5, 256, 256, 1, 4096, 256, 0, 0, 0]


def test_import_name_of_the_reference():
    # The reference's module is `wmma_ops` (setup.py:18-21); `import wmma_ops` gives this
    # library, the same module object as wmma_ops_amd.
    import wmma_ops
    import wmma_ops_amd
    assert wmma_ops is wmma_ops_amd
    for name in ["matmul", "matmul_adaptive", "matmul_tiled", "gemm", "gemm_inplace",
                 "gemm_adaptive", "flash_attention", "matmul_asmOpt", "matmul_xor_optimized"]:
        assert callable(getattr(wmma_ops, name))
    with pytest.raises(RuntimeError, match="Inputs must be CUDA tensors"):
        wmma_ops.matmul_adaptive(torch.zeros(4, 8, dtype=torch.float16),
                                 torch.zeros(8, 4, dtype=torch.float16))


def test_gptq_entry_points_validate(lib):
    FAKE = 1 << 20
    # zeros: bad format, N not a multiple of 8, group size not dividing K, misalignment
    assert lib.wmma_int4_from_gptq_zeros(FAKE, 256, 64, 64, 3, FAKE, None, None) == INVALID
    assert lib.wmma_int4_from_gptq_zeros(FAKE, 256, 60, 64, 1, FAKE, None, None) == INVALID
    assert lib.wmma_int4_from_gptq_zeros(FAKE, 256, 64, 96, 1, FAKE, None, None) == INVALID
    assert lib.wmma_int4_from_gptq_zeros(FAKE + 2, 256, 64, 64, 2, FAKE, None, None) == MISALIGNED
    assert lib.wmma_int4_from_gptq_zeros(None, 256, 64, 64, 1, FAKE, None, None) == INVALID
    # row permutation: K not a multiple of 8, in place, NULL perm
    assert lib.wmma_int4_permute_rows(FAKE, FAKE * 2, 100, 64, FAKE * 3, None) == INVALID
    assert lib.wmma_int4_permute_rows(FAKE, FAKE * 2, 128, 64, FAKE, None) == INVALID
    assert lib.wmma_int4_permute_rows(FAKE, None, 128, 64, FAKE * 3, None) == INVALID


def test_w4a16_offset_limits(lib):
    # 32-bit buffer offsets: the whole-A bound applies per 256-row tile, so a long prefill is
    # accepted up to the launch (nothing here reaches the GPU: the pointers below are
    # checked for NULL only after the shape checks, and this call fails on the K bound);
    # K so large that one workgroup's weight columns pass 2^31 bytes is rejected.
    FAKE = 1 << 20
    K = 1 << 24
    rc = lib.wmma_w4a16_gemm(FAKE, K, FAKE, FAKE, FAKE, 0, 4, 64, K, 128, FAKE, 64, None, 0, None)
    assert rc == UNSUPPORTED
    assert b"weight offsets" in lib.wmma_last_error()


# --------------------------------------------------- fused decode layout validation --
def test_fused_layout_validation_codes(lib):
    """wmma_int4_fused_bytes against the oracle's layout arithmetic, and every argument
    check of the fused prepack / unprepack / W4A16 entry points (none reaches the GPU)."""
    from oracle import int4 as oi
    vp, i32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
    lib.wmma_int4_fused_bytes.argtypes = [i32, i32]
    lib.wmma_int4_fused_bytes.restype = sz
    for K, N in ((4096, 4096), (4096, 14336), (640, 32), (128, 64), (1152, 96)):
        assert lib.wmma_int4_fused_bytes(K, N) == (N // 16) * oi.fused_slice_bytes(K), (K, N)
    for K, N in ((192, 64), (4096, 48), (0, 64), (4096, -32)):
        assert lib.wmma_int4_fused_bytes(K, N) == 0, (K, N)
    lib.wmma_int4_prepack_fused.argtypes = [vp, vp, vp, i32, i32, i32, i32, vp, vp]
    pf = lambda q=FAKE, s=FAKE, z=FAKE, zf=0, K=4096, N=4096, G=128, out=FAKE: \
        lib.wmma_int4_prepack_fused(q, s, z, zf, K, N, G, out, None)
    assert pf(K=192) == UNSUPPORTED            # K % 128
    assert pf(N=48) == UNSUPPORTED             # N % 32
    assert pf(K=0) == INVALID
    for G in (64, 384, 96, 8192):              # not 128 * 2^j dividing K
        assert pf(G=G) == UNSUPPORTED, G
    assert pf(zf=2) == INVALID                 # slice-major parameters cannot be fused
    assert pf(zf=7) == INVALID
    assert pf(q=None) == INVALID and pf(s=None) == INVALID and pf(z=None) == INVALID
    assert pf(out=None) == INVALID
    assert pf(out=FAKE + 4) == MISALIGNED
    assert pf(q=FAKE + 2) == MISALIGNED
    assert pf(s=FAKE + 1) == MISALIGNED
    assert pf(z=FAKE + 2) == MISALIGNED        # packed zeros: 4-byte aligned
    lib.wmma_int4_unprepack_fused.argtypes = [vp, i32, i32, i32, vp, vp, vp, vp]
    uf = lambda f=FAKE, K=4096, N=4096, G=128, q=FAKE, s=FAKE, z=FAKE: \
        lib.wmma_int4_unprepack_fused(f, K, N, G, q, s, z, None)
    assert uf(K=192) == UNSUPPORTED and uf(G=64) == UNSUPPORTED and uf(N=16) == UNSUPPORTED
    assert uf(f=None) == INVALID and uf(q=None) == INVALID
    assert uf(f=FAKE + 8) == MISALIGNED and uf(z=FAKE + 2) == MISALIGNED and uf(s=FAKE + 1) == MISALIGNED
    # the W4A16 entry point with the fused layout: decode shapes only, G = 128 * 2^j
    w = lambda M=1, K=4096, G=128, A=FAKE: lib.wmma_w4a16_gemm(A, K, FAKE, None, None, 3, M, 4096, K,
                                                              G, FAKE, 4096, None, 0, None)
    assert w(M=5) == UNSUPPORTED
    assert b"decode kernel only" in lib.wmma_last_error()
    assert w(M=4, K=14336, A=None) == INVALID  # M = 4 past one round is in the domain (NULL A)
    assert w(G=64) == UNSUPPORTED
    assert w(K=4160, G=64) == UNSUPPORTED      # K % 128 != 0
    assert w(M=0) == OK                        # empty output: scales and zeros are not read
    assert w(A=FAKE + 2) == MISALIGNED
    assert w(A=None) == INVALID


# ------------------------------------------------- allocation-free GEMM validation --
def test_noalloc_validation_codes(lib):
    """wmma_gemm_f16f32_noalloc rejects bad arguments exactly like wmma_gemm_f16f32 (before
    touching a device: the scratch address is looked up only after these checks), and every
    plan it makes fits its scratch array: it plans with wmma_gemm_plan_make_within(scratch
    size), which over a sweep of shapes and every tile choice stays within the 32 MiB where
    the unconstrained planner's plan would not (the entry point's WMMA_ERR_WORKSPACE
    rejection is a guard that no such plan reaches)."""
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_gemm_f16f32_noalloc.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32,
                                             f32, f32, i32, vp]
    lib.wmma_gemm_noalloc_scratch_bytes.restype = sz
    cap = lib.wmma_gemm_noalloc_scratch_bytes()
    assert cap == 32 << 20
    na = lambda M=64, N=64, K=64, lda=64, ldb=64, ldc=64, C=FAKE, A=FAKE, cfg=-1: \
        lib.wmma_gemm_f16f32_noalloc(A, lda, FAKE, ldb, None, 0, C, ldc, M, N, K, 1.0, 0.0, cfg, None)
    assert na(M=-1) == INVALID
    assert na(cfg=9) == INVALID
    assert na(C=None) == INVALID
    assert na(ldc=32) == INVALID
    assert na(lda=32) == INVALID
    assert na(A=None) == INVALID
    assert na(M=0) == OK and na(N=0) == OK     # empty output
    p = Plan()
    lib.wmma_gemm_plan_make_within.argtypes = [ctypes.c_int] * 5 + [ctypes.c_size_t,
                                                                    ctypes.POINTER(Plan)]
    largest = over = 0
    for cfg in range(-1, 6):
        for M in (1, 16, 32, 64, 128, 256, 512, 1024, 4100):
            for N in (520, 4096, 16384, 65536):
                for K in (520, 4096, 14336, 65536, 262144):
                    assert lib.wmma_gemm_plan_make(M, N, K, cfg, 256, ctypes.byref(p)) == OK
                    over += p.workspace_bytes > cap
                    assert lib.wmma_gemm_plan_make_within(M, N, K, cfg, 256, cap,
                                                          ctypes.byref(p)) == OK
                    largest = max(largest, p.workspace_bytes)
    assert over > 0 and largest <= cap
