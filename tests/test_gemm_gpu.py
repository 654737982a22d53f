"""GPU parity of the FP16 GEMM family against the CPU oracle (fp32 torch).

Bar: max|Y - Y_ref| / max|Y_ref| <= 1e-3 (the reference's metric and the task's bound,
test_rocwmma_patch.py:66-74, test_fragment_loading.py:116-120), exact where the data
makes every partial sum exact.  Inputs are seeded on the CPU (seed 42 + config index)
and copied to the device, so both sides see identical values.
"""
import pytest
import torch

from oracle import gemm as og
from tests.conftest import report

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _inputs(M, N, K, seed, bstd=1.0):
    g = torch.Generator().manual_seed(seed)
    A = torch.randn(M, K, generator=g).half()
    B = (torch.randn(K, N, generator=g) * bstd).half()
    return A, B


def _check(Y, ref, tol=TOL):
    assert Y.dtype == torch.float32 and tuple(Y.shape) == tuple(ref.shape)
    assert torch.isfinite(Y).all()
    err = og.max_rel_err(Y, ref)
    assert err <= tol, f"max rel err {err:.3e} > {tol}"
    return err


def test_known_answer_fragment(wo):
    A, B, C = og.kat_fragment()
    report("kat", M=64, N=64, K=16)
    for fn in (wo.matmul, wo.matmul_adaptive, wo.matmul_asmOpt):
        assert torch.equal(fn(A.cuda(), B.cuda()).cpu(), C)
    for cfg in range(6):
        assert torch.equal(wo.matmul_tiled(A.cuda(), B.cuda(), cfg).cpu(), C)


# The reference's own correctness cases: the seven seeded shapes of its fragment-loading
# test (test_fragment_loading.py:67-75, seed 42, fp32 torch.matmul reference) and the
# small-K shapes of its patch test (test_rocwmma_patch.py:58-106), through every entry
# point: matmul, matmul_adaptive, the asmOpt alias it calls, and every matmul_tiled tile.
@pytest.mark.parametrize("M,N,K", [(512, 512, 64), (512, 512, 128), (1024, 1024, 256),
                                   (2048, 2048, 512), (4096, 4096, 1024), (2048, 1024, 512),
                                   (1024, 2048, 512), (2048, 2048, 128)])
def test_reference_test_shapes(wo, M, N, K):
    report("reference_shapes", M=M, N=N, K=K, plan=wo.gemm_plan(M, N, K))
    A, B = _inputs(M, N, K, 42)
    ref = og.gemm_ref(A, B)
    Ad, Bd = A.cuda(), B.cuda()
    for fn in (wo.matmul, wo.matmul_adaptive, wo.matmul_asmOpt):
        _check(fn(Ad, Bd), ref)
    for cfg in range(6):
        _check(wo.matmul_tiled(Ad, Bd, cfg), ref)


# configs[0] and configs[1] of the task: square and rectangular shapes
@pytest.mark.parametrize("M,N,K", [(512, 512, 512), (1024, 1024, 1024), (2048, 2048, 2048),
                                   (4096, 4096, 4096), (4096, 4096, 2048)])
def test_matmul_baseline_shapes(wo, M, N, K):
    report("matmul", M=M, N=N, K=K, plan=wo.gemm_plan(M, N, K))
    A, B = _inputs(M, N, K, 42 + 1)
    ref = og.gemm_ref(A, B)
    Ad, Bd = A.cuda(), B.cuda()
    _check(wo.matmul(Ad, Bd), ref)
    _check(wo.matmul_adaptive(Ad, Bd), ref)


@pytest.mark.parametrize("M,N,K", [(1024, 1024, 1024), (2048, 2048, 2048), (4096, 4096, 4096),
                                   (4096, 4096, 2048)])
def test_gemm_epilogue_out_of_place_and_in_place(wo, M, N, K):
    # C = 2.0*A*B + 0.5*C with C fp32 N(0,1), out-of-place and in-place.
    report("gemm_epilogue", M=M, N=N, K=K)
    A, B = _inputs(M, N, K, 42 + 1)
    C = torch.randn(M, N, generator=torch.Generator().manual_seed(7))
    ref = og.gemm_ref(A, B, 2.0, 0.5, C)
    Ad, Bd, Cd = A.cuda(), B.cuda(), C.cuda()
    out = wo.gemm(Ad, Bd, alpha=2.0, beta=0.5, C=Cd)
    _check(out, ref)
    assert torch.equal(Cd.cpu(), C)                       # out-of-place leaves C alone
    out2 = wo.gemm_adaptive(Ad, Bd, 2.0, 0.5, Cd)
    assert torch.equal(out, out2)
    Ci = Cd.clone()
    assert wo.gemm_inplace(Ad, Bd, Ci, 2.0, 0.5) is None
    assert torch.equal(Ci, out)                           # in-place == out-of-place bitwise


def test_gemm_beta_rules(wo):
    A, B = _inputs(256, 192, 320, 5)
    Ad, Bd = A.cuda(), B.cuda()
    nan_c = torch.full((256, 192), float("nan"), device="cuda")
    out = wo.gemm(Ad, Bd, alpha=1.5, beta=0.0, C=nan_c)   # beta == 0 never reads C
    assert torch.isfinite(out).all()
    _check(out, og.gemm_ref(A, B, 1.5))
    out = wo.gemm(Ad, Bd, alpha=1.0, beta=3.0, C=None)    # beta without C is ignored
    _check(out, og.gemm_ref(A, B))
    Ci = nan_c.clone()
    wo.gemm_inplace(Ad, Bd, Ci, 1.0, 0.0)
    assert torch.isfinite(Ci).all()
    with pytest.raises(RuntimeError, match="C dimensions must match output"):
        wo.gemm(Ad, Bd, 1.0, 1.0, torch.zeros(3, 3, device="cuda"))
    with pytest.raises(RuntimeError, match="C must be float32"):
        wo.gemm(Ad, Bd, 1.0, 1.0, torch.zeros(256, 192, device="cuda", dtype=torch.float16))


# skinny shapes that take the split-K / streaming paths
SKINNY = [(m, n, 4096) for m in (1, 16, 64, 128) for n in (4096, 11008, 14336)] + \
         [(m, 4096, 14336) for m in (1, 16, 64, 128)] + \
         [(m, n, 4096) for m in (17, 32, 48) for n in (4096, 11008)] + [(32, 4096, 14336)]


@pytest.mark.parametrize("M,N,K", SKINNY)
def test_skinny_split_k(wo, M, N, K):
    report("skinny", M=M, N=N, K=K, plan=wo.gemm_plan(M, N, K))
    A, B = _inputs(M, N, K, 42 + 2, bstd=0.02)
    ref = og.gemm_ref(A, B)
    _check(wo.matmul(A.cuda(), B.cuda()), ref)


def _capi():
    import ctypes
    import os
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                   "wmma_ops_amd", "libwmma_ops_amd.so"))
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_gemm_workspace_size.restype = sz
    lib.wmma_gemm_workspace_size.argtypes = [i32, i32, i32, i32]
    lib.wmma_gemm_f16f32.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32,
                                     f32, f32, i32, vp, sz, vp]
    return lib



# Row strides of C_in and C_out larger than N and different from each other: the epilogue
# reads C_in at its own stride, writes only the N columns of each output row, and leaves
# the padding of both buffers alone (512x512 takes full 256x256 tiles, 300x264 ragged ones).
@pytest.mark.parametrize("M,N,K,tile", [(512, 512, 1024, 5), (300, 264, 640, -1)])
def test_gemm_strided_c(wo, M, N, K, tile):
    report("gemm_strided_c", M=M, N=N, K=K, tile=tile)
    lib = _capi()
    A, B = _inputs(M, N, K, 31 + M)
    ldcin, ldc = N + 40, N + 72
    g = torch.Generator().manual_seed(32)
    Cin = torch.randn(M, ldcin, generator=g)
    Cout = torch.full((M, ldc), 7.0)
    Ad, Bd, Cid, Cod = A.cuda(), B.cuda(), Cin.cuda(), Cout.cuda()
    nws = lib.wmma_gemm_workspace_size(M, N, K, tile)
    ws = torch.empty(max(nws, 1), dtype=torch.uint8, device="cuda")
    rc = lib.wmma_gemm_f16f32(Ad.data_ptr(), K, Bd.data_ptr(), N, Cid.data_ptr(), ldcin,
                              Cod.data_ptr(), ldc, M, N, K, 2.0, 0.5, tile, ws.data_ptr(), nws,
                              torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    out = Cod.cpu()
    _check(out[:, :N].contiguous(), og.gemm_ref(A, B, 2.0, 0.5, Cin[:, :N].contiguous()))
    assert torch.equal(out[:, N:], Cout[:, N:])
    assert torch.equal(Cid.cpu(), Cin)

# Split-K partials go through a caller workspace whose contents are arbitrary: a workspace
# of random bytes, the same workspace again and re-randomised must all give the same bits
# (fixed summation order), within tolerance of the oracle, and so must the in-place
# epilogue through the same workspace.
@pytest.mark.parametrize("M,N,K", [(1, 4096, 4096), (16, 14336, 4096), (5, 1024, 14336),
                                   (3, 4096, 2056)])
def test_skinny_split_k_any_workspace(wo, M, N, K):
    report("skinny_ws", M=M, N=N, K=K, plan=wo.gemm_plan(M, N, K))
    lib = _capi()
    A, B = _inputs(M, N, K, 77 + M, bstd=0.02)
    ref = og.gemm_ref(A, B)
    Ad, Bd = A.cuda(), B.cuda()
    need = lib.wmma_gemm_workspace_size(M, N, K, -1)
    assert need > 0 and wo.gemm_plan(M, N, K)[4] > 1
    g = torch.Generator(device="cuda").manual_seed(M + N)
    ws = torch.randint(0, 256, (need,), dtype=torch.uint8, device="cuda", generator=g)
    stream = torch.cuda.current_stream().cuda_stream
    outs = []
    for rnd in range(3):
        if rnd == 2:
            ws.random_(0, 256, generator=g)
        C = torch.full((M, N), float("nan"), device="cuda")
        rc = lib.wmma_gemm_f16f32(Ad.data_ptr(), K, Bd.data_ptr(), N, None, N, C.data_ptr(), N,
                                  M, N, K, 1.0, 0.0, -1, ws.data_ptr(), need, stream)
        assert rc == 0
        outs.append(C)
    torch.cuda.synchronize()
    _check(outs[0], ref)
    assert torch.equal(outs[0], outs[1]) and torch.equal(outs[0], outs[2])
    Cin = torch.randn(M, N, generator=torch.Generator().manual_seed(3))
    Ci = Cin.cuda()
    rc = lib.wmma_gemm_f16f32(Ad.data_ptr(), K, Bd.data_ptr(), N, Ci.data_ptr(), N, Ci.data_ptr(), N,
                              M, N, K, 2.0, 0.5, -1, ws.data_ptr(), need, stream)
    assert rc == 0
    _check(Ci, og.gemm_ref(A, B, 2.0, 0.5, Cin))


# Explicit plans (the autotuner's entry point): every kernel, tile and split gives the
# oracle's result within tolerance, including the epilogue.
@pytest.mark.parametrize("kernel,tile,split", [(0, t, s) for t in range(6) for s in (1, 3, 8)] +
                         [(1, -1, s) for s in (1, 5, 32)] + [(1, -2, s) for s in (1, 3)] +
                         [(1, -4, s) for s in (1, 6)])
def test_gemm_explicit_plans(wo, kernel, tile, split):
    import ctypes
    from tests.test_capi import Plan
    report("gemm_plan", kernel=kernel, tile=tile, split=split)
    lib = _capi()
    lib.wmma_gemm_plan_custom.argtypes = [ctypes.c_int] * 6 + [ctypes.POINTER(Plan)]
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_gemm_f16f32_plan.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, f32, f32,
                                          ctypes.POINTER(Plan), vp, sz, vp]
    # skinny plans: tile -1 / -2 / -4 picks one, two or four 16-row blocks of A (M = 13,
    # 29, 61: the last block partly past M)
    M, N, K = ({-1: 13, -2: 29, -4: 61}[tile], 200, 4096) if kernel == 1 else (300, 264, 2560)
    A, B = _inputs(M, N, K, 5 + tile + split)
    Cin = torch.randn(M, N, generator=torch.Generator().manual_seed(6))
    p = Plan()
    assert lib.wmma_gemm_plan_custom(M, N, K, kernel, -1 if kernel == 1 else tile, split,
                                     ctypes.byref(p)) == 0
    assert p.tile_m == (16 * -tile if kernel == 1 else p.tile_m)
    ws = torch.empty(max(p.workspace_bytes, 1), dtype=torch.uint8, device="cuda")
    Ad, Bd, C = A.cuda(), B.cuda(), Cin.cuda()
    rc = lib.wmma_gemm_f16f32_plan(Ad.data_ptr(), K, Bd.data_ptr(), N, C.data_ptr(), N, C.data_ptr(), N,
                                   M, N, K, 2.0, 0.5, ctypes.byref(p), ws.data_ptr(), p.workspace_bytes,
                                   torch.cuda.current_stream().cuda_stream)
    assert rc == 0
    _check(C, og.gemm_ref(A, B, 2.0, 0.5, Cin))


@pytest.mark.parametrize("M", [16, 32])
def test_skinny_epilogue_in_place(wo, M):
    A, B = _inputs(M, 4096, 4096, 11, bstd=0.02)
    C = torch.randn(M, 4096, generator=torch.Generator().manual_seed(12))
    ref = og.gemm_ref(A, B, 2.0, 0.5, C)
    Ci = C.cuda()
    wo.gemm_inplace(A.cuda(), B.cuda(), Ci, 2.0, 0.5)
    _check(Ci, ref)


@pytest.mark.parametrize("cfg", range(6))
# (129, 97, 203): N and K not multiples of 8, so every tile runs the element-wise-load kernel
@pytest.mark.parametrize("M,N,K", [(512, 384, 320), (300, 264, 136), (1, 8, 64), (257, 520, 1000),
                                   (129, 97, 203)])
def test_matmul_tiled_every_config(wo, cfg, M, N, K):
    report("tiled", cfg=cfg, M=M, N=N, K=K)
    A, B = _inputs(M, N, K, 100 + cfg)
    _check(wo.matmul_tiled(A.cuda(), B.cuda(), cfg), og.gemm_ref(A, B))


def test_matmul_tiled_invalid_config(wo):
    A = torch.zeros(64, 64, dtype=torch.float16, device="cuda")
    with pytest.raises(RuntimeError, match="Invalid tile_config"):
        wo.matmul_tiled(A, A, 7)


@pytest.mark.parametrize("M,N,K", [(33, 40, 24), (130, 72, 200), (17, 19, 23), (5, 3, 7),
                                   (1, 1, 1), (70, 129, 513), (3, 4096, 520), (640, 8, 8)])
def test_ragged_shapes(wo, M, N, K):
    # N or K not multiples of 8: the operand is repacked into a zero-padded copy.
    report("ragged", M=M, N=N, K=K)
    A, B = _inputs(M, N, K, M * 1000 + N + K)
    ref = og.gemm_ref(A, B)
    _check(wo.matmul(A.cuda(), B.cuda()), ref)
    C = torch.randn(M, N)
    _check(wo.gemm(A.cuda(), B.cuda(), 0.5, -2.0, C.cuda()), og.gemm_ref(A, B, 0.5, -2.0, C))


def _repack_bytes(M, N, K, a, b):
    r256 = lambda x: (x + 255) // 256 * 256
    if not (a or b):
        return 0
    return 256 + (r256(M * ((K + 7) // 8 * 8) * 2) if a else 0) + (r256(K * ((N + 7) // 8 * 8) * 2) if b else 0)


# Operands whose rows break 16-byte vectors, through the C-ABI two ways: with the workspace
# wmma_gemm_workspace_size reports (or, for strided / misaligned operands, the partial sums
# plus room for the padded copies) the operand is repacked and the vector kernels run; with
# only the partial-sum workspace the element-wise kernels read it in place.  Both match the
# oracle; the products (alpha = 1, beta = 0) match each other bit for bit (same MFMA inputs
# in the same K order), the alpha/beta epilogue to rounding (the two kernels' epilogues
# contract alpha*acc + beta*c into different fused multiply-adds); no byte of the workspace
# past the reported size is written.
@pytest.mark.parametrize("M,N,K,case", [
    (300, 4100, 520, "contig"), (640, 1000, 1004, "contig"), (70, 129, 513, "contig"),
    (33, 4100, 4096, "contig"), (257, 3001, 64, "contig"),
    (96, 256, 320, "a_off"), (200, 136, 256, "b_ld"), (40, 640, 1024, "both")])
def test_ragged_repack_matches_inplace(wo, M, N, K, case):
    report("ragged_repack", M=M, N=N, K=K, case=case, plan=wo.gemm_plan(M, N, K))
    lib = _capi()
    A, B = _inputs(M, N, K, 5 * M + N + K, bstd=0.05)
    Cin = torch.randn(M, N, generator=torch.Generator().manual_seed(M + K))
    ref = og.gemm_ref(A, B, 1.5, -0.5, Cin)
    plan_ws = wo.gemm_plan(M, N, K)[7]
    if case in ("a_off", "both"):   # A one element off 16-byte alignment, lda = K + 3
        Abuf = torch.zeros(M * (K + 3) + 1, dtype=torch.half)
        Abuf[1:].view(M, K + 3)[:, :K] = A
        Ad, a_ptr, lda = Abuf.cuda(), None, K + 3
        a_ptr = Ad.data_ptr() + 2
    else:
        Ad = A.cuda()
        a_ptr, lda = Ad.data_ptr(), K
    if case in ("b_ld", "both"):    # B rows at an odd stride
        Bbuf = torch.zeros(K, N + 5, dtype=torch.half)
        Bbuf[:, :N] = B
        Bd, ldb = Bbuf.cuda(), N + 5
    else:
        Bd, ldb = B.cuda(), N
    a_bad = K % 8 != 0 or lda % 8 != 0 or case in ("a_off", "both")
    b_bad = N % 8 != 0 or ldb % 8 != 0
    need = plan_ws + _repack_bytes(M, N, K, a_bad, b_bad)
    assert need > plan_ws
    if case == "contig":
        assert lib.wmma_gemm_workspace_size(M, N, K, -1) == need
    stream = torch.cuda.current_stream().cuda_stream
    prods, outs = [], []
    for wsb in (need, plan_ws):
        ws = torch.full((need + 4096,), 0xA5, dtype=torch.uint8, device="cuda")
        wsp = ws.data_ptr() if wsb else None
        P = torch.full((M, N), float("nan"), device="cuda")
        rc = lib.wmma_gemm_f16f32(a_ptr, lda, Bd.data_ptr(), ldb, None, N, P.data_ptr(), N,
                                  M, N, K, 1.0, 0.0, -1, wsp, wsb, stream)
        assert rc == 0
        Ci = Cin.cuda()
        rc = lib.wmma_gemm_f16f32(a_ptr, lda, Bd.data_ptr(), ldb, Ci.data_ptr(), N, Ci.data_ptr(), N,
                                  M, N, K, 1.5, -0.5, -1, wsp, wsb, stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.all(ws[need:] == 0xA5), "workspace written past the reported size"
        _check(P.cpu(), og.gemm_ref(A, B))
        _check(Ci.cpu(), ref)
        prods.append(P.cpu())
        outs.append(Ci.cpu())
    assert torch.equal(prods[0], prods[1])
    assert og.max_rel_err(outs[0], outs[1]) <= 1e-6


# The skinny kernel (M <= 32) reads a B whose rows break 16-byte vectors in place: with B
# 4-byte aligned, rows are fetched by dword-aligned 16-byte loads (ldb even), or every other
# row by a load from 2 bytes earlier plus one dword, realigned (ldb odd); the chunk that
# straddles column N element-wise.  A with K off a multiple of 8 is repacked.  The same
# operands with B moved 2 bytes off a dword and only the split-K workspace take the
# element-wise kernel: the products match it bit for bit and the oracle to the 1e-3 bar.
@pytest.mark.parametrize("M,N,K,ldb_pad", [
    (1, 4100, 4096, 0), (16, 4100, 4096, 0), (1, 4101, 4096, 0), (7, 1027, 1100, 0),
    (3, 4096, 1096, 3), (16, 32001, 1280, 0), (1, 9, 1088, 0), (2, 5, 1040, 0), (9, 130, 1064, 1),
    (17, 4100, 4096, 0), (32, 4101, 4100, 1), (25, 4101, 2056, 3)])
def test_skinny_unaligned_b_in_place(wo, M, N, K, ldb_pad):
    plan = wo.gemm_plan(M, N, K)
    report("skinny_unaligned_b", M=M, N=N, K=K, ldb=N + ldb_pad, plan=plan)
    assert plan[0] == 1
    lib = _capi()
    A, B = _inputs(M, N, K, 3 * M + N + K, bstd=0.05)
    Cin = torch.randn(M, N, generator=torch.Generator().manual_seed(N))
    ldb = N + ldb_pad
    Bbuf = torch.zeros(K * ldb + 8, dtype=torch.half)
    Bbuf[:K * ldb].view(K, ldb)[:, :N] = B
    Bbuf1 = torch.zeros(K * ldb + 8, dtype=torch.half)   # the same rows, 2 bytes later
    Bbuf1[1:1 + K * ldb].view(K, ldb)[:, :N] = B
    Ad, Bd, Bd1 = A.cuda(), Bbuf.cuda(), Bbuf1.cuda()
    plan_ws = plan[7]
    need = plan_ws + _repack_bytes(M, N, K, K % 8 != 0, False)
    if ldb_pad == 0:
        assert lib.wmma_gemm_workspace_size(M, N, K, -1) == need
    stream = torch.cuda.current_stream().cuda_stream
    prods = []
    for b_ptr, wsb in ((Bd.data_ptr(), need), (Bd1.data_ptr() + 2, plan_ws)):
        ws = torch.full((need + 4096,), 0xA5, dtype=torch.uint8, device="cuda")
        wsp = ws.data_ptr() if wsb else None
        P = torch.full((M, N), float("nan"), device="cuda")
        rc = lib.wmma_gemm_f16f32(Ad.data_ptr(), K, b_ptr, ldb, None, N, P.data_ptr(), N,
                                  M, N, K, 1.0, 0.0, -1, wsp, wsb, stream)
        assert rc == 0
        Ci = Cin.cuda()
        rc = lib.wmma_gemm_f16f32(Ad.data_ptr(), K, b_ptr, ldb, Ci.data_ptr(), N, Ci.data_ptr(), N,
                                  M, N, K, 1.5, -0.5, -1, wsp, wsb, stream)
        assert rc == 0
        torch.cuda.synchronize()
        assert torch.all(ws[need:] == 0xA5), "workspace written past the reported size"
        _check(P.cpu(), og.gemm_ref(A, B))
        _check(Ci.cpu(), og.gemm_ref(A, B, 1.5, -0.5, Cin))
        prods.append(P.cpu())
    assert torch.equal(prods[0], prods[1])


# Two-part plans (a bulk on whole waves of 256x256 tiles, then the edge rows or columns as
# a GEMM of their own): the edge as a split-K skinny GEMM, a one-launch tile and a column
# strip; with B repacked (N off a multiple of 8); through matmul, gemm out of place and in
# place (bitwise equal), the C-ABI with row strides of C_in / C_out above N (padding left
# alone) and wmma_gemm_f16f32_plan with the planner's own two-part plan (bitwise equal).
@pytest.mark.parametrize("M,N,K,dim", [(4100, 4096, 2048, 1), (4103, 4096, 520, 1),
                                       (4352, 4096, 256, 1), (8200, 2048, 512, 1),
                                       (4100, 4100, 1000, 1), (4096, 4101, 1024, 2),
                                       (4096, 4200, 1024, 2)])
def test_two_part_plans(wo, M, N, K, dim):
    import ctypes
    from wmma_ops_amd.autotune import Plan
    plan = wo.gemm_plan(M, N, K)
    report("two_part", M=M, N=N, K=K, plan=plan)
    assert plan[8] == dim
    A, B = _inputs(M, N, K, M + N + K, bstd=0.05)
    Cin = torch.randn(M, N, generator=torch.Generator().manual_seed(11))
    Ad, Bd, Cd = A.cuda(), B.cuda(), Cin.cuda()
    Y = wo.matmul(Ad, Bd)
    _check(Y.cpu(), og.gemm_ref(A, B))
    ref = og.gemm_ref(A, B, 1.5, -0.5, Cin)
    out = wo.gemm(Ad, Bd, 1.5, -0.5, Cd)
    _check(out.cpu(), ref)
    Ci = Cd.clone()
    wo.gemm_inplace(Ad, Bd, Ci, 1.5, -0.5)
    assert torch.equal(Ci, out)
    lib = _capi()
    stream = torch.cuda.current_stream().cuda_stream
    need = lib.wmma_gemm_workspace_size(M, N, K, -1)
    ws = torch.empty(max(need, 1), dtype=torch.uint8, device="cuda")
    ldcin, ldc = N + 40, N + 72
    Cs = torch.full((M, ldcin), 3.0, device="cuda")
    Cs[:, :N] = Cd
    Co = torch.full((M, ldc), 7.0, device="cuda")
    rc = lib.wmma_gemm_f16f32(Ad.data_ptr(), K, Bd.data_ptr(), N, Cs.data_ptr(), ldcin, Co.data_ptr(), ldc,
                              M, N, K, 1.5, -0.5, -1, ws.data_ptr(), need, stream)
    assert rc == 0
    assert torch.equal(Co[:, :N], out)
    assert torch.all(Co[:, N:] == 7.0) and torch.all(Cs[:, N:] == 3.0)
    p = Plan()
    lib.wmma_gemm_plan_make.argtypes = [ctypes.c_int] * 5 + [ctypes.POINTER(Plan)]
    assert lib.wmma_gemm_plan_make(M, N, K, -1, 256, ctypes.byref(p)) == 0 and p.edge_dim == dim
    vp, i64, i32, f32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_gemm_f16f32_plan.argtypes = [vp, i64, vp, i64, vp, i64, vp, i64, i32, i32, i32, f32, f32,
                                          ctypes.POINTER(Plan), vp, sz, vp]
    Yp = torch.empty(M, N, device="cuda")
    rc = lib.wmma_gemm_f16f32_plan(Ad.data_ptr(), K, Bd.data_ptr(), N, None, N, Yp.data_ptr(), N, M, N, K,
                                   1.0, 0.0, ctypes.byref(p), ws.data_ptr(), need, stream)
    assert rc == 0
    assert torch.equal(Yp, Y)
    p.edge_at += 256   # an edited two-part plan is rejected, not launched
    assert lib.wmma_gemm_f16f32_plan(Ad.data_ptr(), K, Bd.data_ptr(), N, None, N, Yp.data_ptr(), N, M, N, K,
                                     1.0, 0.0, ctypes.byref(p), ws.data_ptr(), need, stream) == 1


def test_empty_and_zero_k(wo):
    out = wo.matmul(torch.zeros(0, 16, dtype=torch.half, device="cuda"),
                    torch.zeros(16, 8, dtype=torch.half, device="cuda"))
    assert out.shape == (0, 8)
    out = wo.matmul(torch.zeros(4, 0, dtype=torch.half, device="cuda"),
                    torch.zeros(0, 8, dtype=torch.half, device="cuda"))
    assert out.shape == (4, 8) and torch.count_nonzero(out) == 0
    C = torch.randn(4, 8, device="cuda")
    out = wo.gemm(torch.zeros(4, 0, dtype=torch.half, device="cuda"),
                  torch.zeros(0, 8, dtype=torch.half, device="cuda"), 1.0, 2.0, C)
    assert torch.allclose(out, 2.0 * C)


def test_noncontiguous_inputs(wo):
    A, B = _inputs(96, 80, 128, 3)
    At = A.t().contiguous().cuda().t()   # non-contiguous view of A
    Bt = B.t().contiguous().cuda().t()
    assert not At.is_contiguous()
    _check(wo.matmul(At, Bt), og.gemm_ref(A, B))


def test_identity_and_linearity(wo):
    A, _ = _inputs(256, 256, 256, 9)
    eye = torch.eye(256, dtype=torch.half)
    assert torch.equal(wo.matmul(A.cuda(), eye.cuda()).cpu(), A.float())
    _, B = _inputs(256, 256, 256, 10)
    y1 = wo.gemm(A.cuda(), B.cuda(), alpha=4.0)
    y2 = wo.matmul(A.cuda(), B.cuda())
    assert torch.equal(y1, 4.0 * y2)


def test_integer_data_exact(wo):
    # small integers: every partial sum is exact in fp32, so any tiling or split is exact
    g = torch.Generator().manual_seed(21)
    for M, N, K in [(1, 4096, 4096), (16, 4096, 4096), (256, 512, 4096), (2048, 2048, 2048)]:
        A = torch.randint(-2, 3, (M, K), generator=g).half()
        B = torch.randint(-2, 3, (K, N), generator=g).half()
        assert torch.equal(wo.matmul(A.cuda(), B.cuda()).cpu(), og.gemm_ref(A, B)), (M, N, K)


def test_reference_alignment_texts(wo):
    # The reference's texts (wmma_gemm.hip:1443-1446, 1483-1486 say "... for vectorized
    # loads"; matmul_adaptive, gemm and gemm_adaptive, :1207-1210 and :1920-1923, do not),
    # reached through the reference's own module name.
    import wmma_ops
    buf = torch.zeros(64 * 64 + 8, dtype=torch.half, device="cuda")
    A = buf[1:1 + 64 * 64].view(64, 64)   # contiguous, 2 bytes past a 16-byte boundary
    B = torch.zeros(64, 64, dtype=torch.half, device="cuda")
    assert A.is_contiguous() and A.data_ptr() % 16 == 2
    for fn in (wmma_ops.matmul, lambda a, b: wmma_ops.matmul_tiled(a, b, 0)):
        with pytest.raises(RuntimeError, match="A must be 16-byte aligned for vectorized loads"):
            fn(A, B)
    for fn in (wmma_ops.matmul_adaptive, wmma_ops.gemm, wmma_ops.gemm_adaptive):
        with pytest.raises(RuntimeError) as e:
            fn(A, B)
        assert "A must be 16-byte aligned" in str(e.value) and "vectorized" not in str(e.value)
    # and the reference's module name runs the HIP GEMM
    Ah, Bh = _inputs(256, 128, 192, 4)
    _check(wmma_ops.matmul(Ah.cuda(), Bh.cuda()), og.gemm_ref(Ah, Bh))
