"""GPU parity of the INT4 prepack/unpack kernels (bit-exact) and W4A16 dequant-GEMM
(max rel err <= 1e-3 against the fp32 CPU oracle)."""
import os

import numpy as np
import pytest
import torch

from oracle import gemm as og
from oracle import int4 as oi
from tests.conftest import report

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "int4_k256_n64_g64.npz")


def test_golden_fixture_bit_exact(wo):
    d = np.load(GOLDEN)
    qw = torch.from_numpy(d["qweight"]).cuda()
    K, N = d["q"].shape
    packed = d["packed"]
    assert packed.shape == (N // 16, K // 64, 32, 4)
    assert np.array_equal(wo.prepack_int4(qw).cpu().numpy(), packed)
    assert np.array_equal(wo.unpack_int4(qw).cpu().numpy(), d["q"])
    assert np.array_equal(wo.unprepack_int4(torch.from_numpy(packed).cuda()).cpu().numpy(),
                          d["qweight"])
    A = torch.from_numpy(d["A"])
    Y = wo.matmul_int4(A.cuda(), torch.from_numpy(packed).cuda(),
                       torch.from_numpy(d["scales"]).cuda(), torch.from_numpy(d["zeros_packed"]).cuda(), 64)
    assert og.max_rel_err(Y, torch.from_numpy(d["Y"])) <= 1e-3


@pytest.mark.parametrize("K,N", [(4096, 4096), (4096, 14336), (64, 32), (192, 96)])
def test_prepack_unpack_bit_exact(wo, K, N):
    report("prepack", K=K, N=N)
    q = np.random.default_rng(K + N).integers(0, 16, (K, N), dtype=np.uint8)
    qw = oi.pack_gptq(q)
    qd = torch.from_numpy(qw).cuda()
    pk = wo.prepack_int4(qd)
    assert np.array_equal(pk.cpu().numpy(), oi.prepack(qw))
    assert np.array_equal(wo.unpack_int4(qd).cpu().numpy(), q)
    assert torch.equal(wo.unprepack_int4(pk), qd)


# M in {1,16,128,2048}, K=4096, N in {4096, 14336}, G=128, seed 42 + 3; also in
# the layout bench.py times there (M <= 4: the fused decode layout; otherwise the
# slice-major parameters, bit-identical to the standard ones)
@pytest.mark.parametrize("N", [4096, 14336])
@pytest.mark.parametrize("M", [1, 16, 128, 2048])
def test_w4a16_baseline(wo, M, N):
    K, G = 4096, 128
    report("w4a16", M=M, N=N, K=K, G=G, plan=wo.w4a16_plan(M, N, K, G))
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=42 + 3)
    ref = oi.w4a16_ref(A, q, s, z, G)
    qd = torch.from_numpy(oi.pack_gptq(q)).cuda()
    pk = wo.prepack_int4(qd)
    sd, zd, Ad = torch.from_numpy(s).cuda(), torch.from_numpy(oi.pack_zeros(z)).cuda(), A.cuda()
    Y = wo.matmul_int4(Ad, pk, sd, zd, G)
    assert torch.isfinite(Y).all()
    err = og.max_rel_err(Y, ref)
    assert err <= 1e-3, err
    if M <= 4:
        Yb = wo.matmul_int4_fused(Ad, wo.prepack_int4_fused(qd, sd, zd, G), G)
        assert torch.isfinite(Yb).all()
        assert og.max_rel_err(Yb, ref) <= 1e-3
    else:
        Yb = wo.matmul_int4(Ad, pk, *wo.prepack_int4_params(sd, zd), G)
        assert torch.equal(Yb, Y)


@pytest.mark.parametrize("M,K,N,G", [(1, 256, 64, 32), (3, 512, 96, 64), (5, 1024, 128, 256),
                                     (40, 512, 160, 128), (300, 1024, 96, 1024), (2, 64, 32, 64),
                                     (40, 384, 96, 96), (129, 1152, 64, 384)])
def test_w4a16_group_sizes_and_u8_zeros(wo, M, K, N, G):
    report("w4a16_g", M=M, K=K, N=N, G=G)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=M + K + N + G)
    ref = oi.w4a16_ref(A, q, s, z, G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    Ad, sd = A.cuda(), torch.from_numpy(s).cuda()
    Yp = wo.matmul_int4(Ad, pk, sd, torch.from_numpy(oi.pack_zeros(z)).cuda(), G)
    Yu = wo.matmul_int4(Ad, pk, sd, torch.from_numpy(z).cuda(), G)
    assert og.max_rel_err(Yp, ref) <= 1e-3
    assert torch.equal(Yp, Yu)


# The 4 < M <= 32 matrix-pipe kernel: one and two 16-row blocks, K split over workgroups
# (N=1024; N=4096 and N=352 for M > 16; N=8192), a ragged last split (K=4224: 33
# pair-steps), G=256, a tile count that is not a multiple of the XCD count (N=352), lda > K,
# both zero formats.  N=8192 (4-way K split) and N=12288 take 64-column workgroups on a
# 256-CU device.
@pytest.mark.parametrize("M", [5, 8, 16, 17, 31, 32])
@pytest.mark.parametrize("K,N,G", [(4096, 4096, 128), (4224, 1024, 128), (1536, 352, 256),
                                   (8192, 8192, 128), (4096, 12288, 256)])
def test_w4a16_skinny(wo, M, K, N, G):
    plan = wo.w4a16_plan(M, N, K, G)
    report("w4a16_skinny", M=M, K=K, N=N, G=G, plan=plan)
    assert plan[0] in (4, 6)  # the skinny kernel, or the rows kernel where the model prefers it
    if N == 8192 and M <= 16 and plan[0] == 4:
        assert plan[1] == 4
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=7 * M + K + N)
    ref = oi.w4a16_ref(A, q, s, z, G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    sd = torch.from_numpy(s).cuda()
    Abig = torch.zeros(M, K + 64, dtype=torch.half)
    Abig[:, :K] = A
    Ad = Abig.cuda()[:, :K]  # lda = K + 64
    Yp = wo.matmul_int4(Ad, pk, sd, torch.from_numpy(oi.pack_zeros(z)).cuda(), G)
    Yu = wo.matmul_int4(Ad, pk, sd, torch.from_numpy(z).cuda(), G)
    assert torch.isfinite(Yp).all()
    assert og.max_rel_err(Yp, ref) <= 1e-3
    assert torch.equal(Yp, Yu)


# The LDS-DMA W4A16 GEMM with a K split, called repeatedly through the C-ABI on a workspace
# filled with NaN each time: every call bit-identical and within the oracle's bar.  (Its
# ring once let a stage's DMA overwrite LDS rows another wave was still reading, which
# showed as wrong 8-row groups in a few calls out of several.)
@pytest.mark.parametrize("M,N,K", [(48, 4096, 8192), (256, 4096, 4096), (33, 14336, 4096),
                                   (192, 4096, 8192), (128, 11008, 14336)])
def test_w4a16_gemm_split_repeatable(wo, M, N, K):
    import ctypes
    G = 128
    plan = wo.w4a16_plan(M, N, K, G)
    report("w4a16_gemm_repeat", M=M, N=N, K=K, plan=plan)
    assert plan[0] == 5 and plan[1] > 1
    lib = ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                   "wmma_ops_amd", "libwmma_ops_amd.so"))
    vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
    lib.wmma_w4a16_gemm.argtypes = [vp, i64, vp, vp, vp, i32, i32, i32, i32, i32, vp, i64, vp, sz, vp]
    lib.wmma_last_error.restype = ctypes.c_char_p
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=M + N + K)
    ref = oi.w4a16_ref(A, q, s, z, G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    sd, zd = torch.from_numpy(s).cuda(), torch.from_numpy(oi.pack_zeros(z)).cuda()
    Ad = A.cuda()
    st = torch.cuda.current_stream().cuda_stream
    outs = []
    for rep in range(8):
        ws = torch.full((plan[3] // 4,), float("nan"), device="cuda")
        Y = torch.full((M, N), float("nan"), device="cuda")
        rc = lib.wmma_w4a16_gemm(Ad.data_ptr(), K, pk.data_ptr(), sd.data_ptr(), zd.data_ptr(), 0,
                                 M, N, K, G, Y.data_ptr(), N, ws.data_ptr(), plan[3], st)
        assert rc == 0, lib.wmma_last_error()
        outs.append(Y)
    torch.cuda.synchronize()
    assert og.max_rel_err(outs[0], ref) <= 1e-3
    for Y in outs[1:]:
        assert torch.equal(Y, outs[0])


# The skinny kernel's other workgroup shapes on a 256-CU device (16-column slices per
# workgroup NH x pair-steps per wave U, one or two 16-row blocks): 1x1 unsplit (K = 1024) and
# with an 8-way split, 2x2 unsplit and with a 7-way split, 2x4, 4x1 unsplit and split, 4x2
# unsplit and 2x1 for two blocks, 2x2 split for two blocks.  Within the oracle's bar.
@pytest.mark.parametrize("M,K,N", [(5, 1024, 256), (5, 8192, 256), (12, 2048, 8192),
                                   (16, 14336, 1024), (8, 4096, 8192), (9, 1024, 11008),
                                   (12, 6144, 2048), (24, 2048, 11008), (28, 1024, 4096),
                                   (20, 6144, 2048), (32, 14336, 1024)])
def test_w4a16_skinny_shapes(wo, M, K, N):
    G = 128
    plan = wo.w4a16_plan(M, N, K, G)
    report("w4a16_skinny_shapes", M=M, K=K, N=N, plan=plan)
    assert plan[0] == 4
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=11 * M + K + N)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    Y = wo.matmul_int4(A.cuda(), pk, torch.from_numpy(s).cuda(),
                       torch.from_numpy(oi.pack_zeros(z)).cuda(), G)
    assert torch.isfinite(Y).all()
    assert og.max_rel_err(Y, oi.w4a16_ref(A, q, s, z, G)) <= 1e-3


# The M > 32 LDS-DMA kernel: the three tile configurations (64x128 up to 128 rows, 128x256
# for grids of many such tiles -- M=4000, N=4128: 544, partial in M and N -- else 128x128),
# partial M and N tiles, K shorter than the stage ring (K=192), K split (M=64, N=1024: few
# tiles; M=33, N=14336), G=32 (the two K halves of a chunk in different groups), lda > K,
# both zero formats.
@pytest.mark.parametrize("M,K,N,G", [(33, 4096, 14336, 128), (64, 2048, 1024, 64), (200, 192, 288, 32),
                                     (512, 1024, 2048, 128), (1100, 512, 288, 256),
                                     (1030, 2048, 1056, 128), (100, 768, 4128, 64),
                                     (4000, 512, 4128, 128)])
def test_w4a16_gemm_tiles(wo, M, K, N, G):
    plan = wo.w4a16_plan(M, N, K, G)
    report("w4a16_gemm", M=M, K=K, N=N, G=G, plan=plan)
    assert plan[0] == 5
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=3 * M + K + N + G)
    ref = oi.w4a16_ref(A, q, s, z, G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    sd = torch.from_numpy(s).cuda()
    Abig = torch.zeros(M, K + 32, dtype=torch.half)
    Abig[:, :K] = A
    Ad = Abig.cuda()[:, :K]  # lda = K + 32
    Yp = wo.matmul_int4(Ad, pk, sd, torch.from_numpy(oi.pack_zeros(z)).cuda(), G)
    Yu = wo.matmul_int4(Ad, pk, sd, torch.from_numpy(z).cuda(), G)
    assert torch.isfinite(Yp).all()
    assert og.max_rel_err(Yp, ref) <= 1e-3
    assert torch.equal(Yp, Yu)


def _w4a16_capi(lib, Ad, lda, pk, S, Z, zfmt, M, N, K, G, Y, half=False):
    import ctypes
    vp, i64, i32, sz = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int, ctypes.c_size_t
    fn = lib.wmma_w4a16_gemm_f16out if half else lib.wmma_w4a16_gemm
    fn.argtypes = [vp, i64, vp, vp, vp, i32, i32, i32, i32, i32, vp, i64, vp, sz, vp]
    lib.wmma_last_error.restype = ctypes.c_char_p
    rc = fn(Ad.data_ptr(), lda, pk.data_ptr(), S.data_ptr(), Z.data_ptr(), zfmt, M, N, K, G,
            Y.data_ptr(), N, None, 0, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, lib.wmma_last_error()
    return Y


def _capi_lib():
    import ctypes
    return ctypes.CDLL(os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))),
                                    "wmma_ops_amd", "libwmma_ops_amd.so"))


# The rows kernel through the C-ABI: each of its workgroup shapes -- 16 rows x 32 columns
# (M=40, 77, 50, 600; M=17), 16 x 64 (M=37; M=17), 32 x 64 (M=200, 333; M=17) above and
# below 33 rows, and 16 x 16 (M=5, below 33 rows only) -- with the last row group partial,
# N a multiple of 32 but not 64 (N=288), G = 128, 256, 512 (a pair-step's group found by a
# shift), lda > K, packed and byte zeros and the slice-major parameters (identical bits),
# fp16 output (the fp32 result rounded once), and repeated calls bit-identical.
@pytest.mark.parametrize("M,K,N,G", [(40, 1024, 512, 128), (77, 2048, 1024, 128), (37, 2048, 4096, 128),
                                     (200, 2048, 2048, 256), (333, 1024, 1024, 128),
                                     (50, 4096, 2048, 512), (600, 512, 288, 256),
                                     (5, 3072, 256, 128), (17, 3072, 4096, 128), (17, 3072, 8192, 128),
                                     (17, 3072, 14336, 128)])
def test_w4a16_rows(wo, M, K, N, G):
    plan = wo.w4a16_plan(M, N, K, G)
    report("w4a16_rows", M=M, K=K, N=N, G=G, plan=plan)
    assert plan[0] == 6 and plan[1] == 1 and plan[3] == 0
    lib = _capi_lib()
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=5 * M + K + N + G)
    ref = oi.w4a16_ref(A, q, s, z, G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    sd = torch.from_numpy(s).cuda()
    zp = torch.from_numpy(oi.pack_zeros(z)).cuda()
    zu = torch.from_numpy(z).cuda()
    ss, zs = wo.prepack_int4_params(sd, zp)
    lda = K + 64
    Abig = torch.zeros(M, lda, dtype=torch.half)
    Abig[:, :K] = A
    Ad = Abig.cuda()
    outs = [_w4a16_capi(lib, Ad, lda, pk, S, Z, f, M, N, K, G, torch.full((M, N), float("nan"), device="cuda"))
            for S, Z, f in ((sd, zp, 0), (sd, zu, 1), (ss, zs, 2), (sd, zp, 0))]
    Yh = _w4a16_capi(lib, Ad, lda, pk, sd, zp, 0, M, N, K, G,
                     torch.full((M, N), float("nan"), dtype=torch.half, device="cuda"), half=True)
    torch.cuda.synchronize()
    assert torch.isfinite(outs[0]).all()
    assert og.max_rel_err(outs[0], ref) <= 1e-3
    for Y in outs[1:]:
        assert torch.equal(Y, outs[0])
    assert torch.equal(Yh, outs[0].half())
    assert torch.equal(wo.matmul_int4(A.cuda(), pk, sd, zp, G), outs[0])


# The M <= 2 decode kernel applies s and z to each 128-deep partial sum: the MFMA sees the
# nibbles offset by 1024 and the offset is subtracted through fp32 sums of the activations.
# Activations with a large common mean or outlier channels make that offset term large
# against the result, which is where a cancellation mistake would show.
@pytest.mark.parametrize("M", [1, 2])
@pytest.mark.parametrize("kind", ["mean4", "outliers"])
def test_w4a16_decode_offset_cancellation(wo, M, kind):
    K, N, G = 4096, 512, 128
    report("w4a16_offset", M=M, kind=kind)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=7 + M)
    if kind == "mean4":
        A = (4.0 + 0.5 * A.float()).half()
    else:
        A = A.clone()
        A[:, ::512] *= 64.0
    ref = oi.w4a16_ref(A, q, s, z, G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    for zeros in (oi.pack_zeros(z), z):
        Y = wo.matmul_int4(A.cuda(), pk, torch.from_numpy(s).cuda(), torch.from_numpy(zeros).cuda(), G)
        err = og.max_rel_err(Y, ref)
        assert err <= 1e-3, err


@pytest.mark.parametrize("M", [1, 2])
def test_w4a16_decode_q_equals_z_cancels(wo, M):
    # q == z everywhere: the result is a difference of two fp32 sums of the same terms,
    # zero up to their rounding (far below the offset term 1024 s sum|a|).
    K, N, G = 4096, 256, 128
    q = np.random.default_rng(3).integers(0, 16, (K // G, N), dtype=np.uint8)
    zq = np.repeat(q, G, axis=0)
    s = np.full((K // G, N), 0.01, dtype=np.float16)
    A = torch.randn(M, K, generator=torch.Generator().manual_seed(5)).half()
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(zq)).cuda())
    Y = wo.matmul_int4(A.cuda(), pk, torch.from_numpy(s).cuda(), torch.from_numpy(q).cuda(), G)
    offset = 1024 * 0.01 * A.float().abs().sum(dim=1, keepdim=True)
    assert (Y.cpu().abs() <= 1e-5 * offset).all(), float((Y.cpu().abs() / offset).max())


# Slice-major group parameters (prepack_int4_params): a bit-exact layout conversion, and
# every kernel reads them to the same bits as the standard [K/G, N] layout.
def test_prepack_params_bit_exact(wo):
    d = np.load(GOLDEN)
    for zeros in (d["zeros_packed"], d["zeros_u8"]):
        s_sl, z_sl = wo.prepack_int4_params(torch.from_numpy(d["scales"]).cuda(),
                                            torch.from_numpy(zeros).cuda())
        ws, wz = oi.slice_params(d["scales"], d["zeros_u8"])
        assert np.array_equal(s_sl.cpu().numpy().view(np.uint16), ws.view(np.uint16))
        assert np.array_equal(z_sl.cpu().numpy(), wz)


@pytest.mark.parametrize("M", [1, 2, 3, 4, 5, 16, 17, 32, 33, 128, 300])
@pytest.mark.parametrize("K,N,G", [(4096, 1024, 128), (1024, 352, 64), (2048, 160, 256), (512, 96, 32),
                                   (2048, 12288, 128)])
def test_w4a16_sliced_params_same_bits(wo, M, K, N, G):
    report("w4a16_sliced", M=M, K=K, N=N, G=G)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=M * 7 + N + G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    Ad, sd, zd = A.cuda(), torch.from_numpy(s).cuda(), torch.from_numpy(oi.pack_zeros(z)).cuda()
    Y = wo.matmul_int4(Ad, pk, sd, zd, G)
    s_sl, z_sl = wo.prepack_int4_params(sd, zd)
    Ys = wo.matmul_int4(Ad, pk, s_sl, z_sl, G)
    assert torch.equal(Y, Ys)
    assert og.max_rel_err(Ys, oi.w4a16_ref(A, q, s, z, G)) <= 1e-3


# Fused decode layout (prepack_int4_fused): bit-exact against the oracle and round-tripped,
# including a partial last record (K = 640, 4224) and G > 128 (parameters repeated per step).
@pytest.mark.parametrize("K,N,G", [(4096, 4096, 128), (4096, 14336, 128), (640, 64, 128),
                                   (4224, 96, 128), (2048, 160, 256), (8192, 64, 1024)])
def test_prepack_fused_bit_exact(wo, K, N, G):
    report("prepack_fused", K=K, N=N, G=G)
    A, q, s, z = oi.make_inputs(1, K, N, G, seed=K + N + G)
    qw = oi.pack_gptq(q)
    ref = oi.prepack_fused(qw, s, z, G)
    qd, sd = torch.from_numpy(qw).cuda(), torch.from_numpy(s).cuda()
    for zeros in (oi.pack_zeros(z), z):
        f = wo.prepack_int4_fused(qd, sd, torch.from_numpy(zeros).cuda(), G)
        assert np.array_equal(f.cpu().numpy(), ref)
    q2, s2, z2 = wo.unprepack_int4_fused(f, G)
    assert torch.equal(q2, qd)
    assert np.array_equal(s2.cpu().numpy().view(np.uint16), s.view(np.uint16))
    assert np.array_equal(z2.cpu().numpy(), oi.pack_zeros(z))


# configs[3] decode rows (M = 1, K = 4096, N in {4096, 14336}, G = 128, seed 42 + 3) in the
# fused layout the headline times, plus M = 2..4, K past one round (8192, ragged 4224) and
# G > 128: within the oracle's bar, and bit-equal to the standard layout wherever the planner
# gives that layout the same decode kernel (the same arithmetic on values read from other
# addresses; narrow N, where the standard layout takes a split kernel, only the bar).
@pytest.mark.parametrize("M,K,N,G", [(1, 4096, 4096, 128), (1, 4096, 14336, 128),
                                     (2, 4096, 4096, 128), (3, 4096, 1024, 128),
                                     (4, 4096, 14336, 128), (1, 8192, 1024, 128),
                                     (2, 4224, 2048, 128), (1, 2048, 4096, 256), (4, 640, 4096, 128),
                                     (3, 8192, 1024, 128), (4, 14336, 2048, 128)])
def test_w4a16_fused_decode(wo, M, K, N, G):
    report("w4a16_fused", M=M, K=K, N=N, G=G)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=42 + 3 if K == 4096 and G == 128 else M + K + N)
    qd, sd = torch.from_numpy(oi.pack_gptq(q)).cuda(), torch.from_numpy(s).cuda()
    zd = torch.from_numpy(oi.pack_zeros(z)).cuda()
    f = wo.prepack_int4_fused(qd, sd, zd, G)
    Ad = A.cuda()
    Y = wo.matmul_int4_fused(Ad, f, G)
    assert og.max_rel_err(Y, oi.w4a16_ref(A, q, s, z, G)) <= 1e-3
    if wo.w4a16_plan(M, N, K, G)[0] == 0:  # the standard layout also takes the decode kernel
        Ys = wo.matmul_int4(Ad, wo.prepack_int4(qd), sd, zd, G)
        assert torch.equal(Y, Ys)
    Yh = wo.matmul_int4_fused(Ad, f, G, out_dtype=torch.float16)
    assert torch.equal(Yh, Y.half())


# Decode shapes past one round (K > 4096) at every M <= 4: the matrix-pipe decode kernel in
# both layouts (M = 3, 4 stage up to 66.6 KB of activations in LDS), within the oracle's bar
# and bit-equal between the layouts (the same kernel on the same values).
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N", [(8192, 4096), (14336, 4096)])
def test_w4a16_decode_long_k(wo, M, K, N):
    G = 128
    report("w4a16_decode_long_k", M=M, K=K, N=N, plan=wo.w4a16_plan(M, N, K, G))
    assert wo.w4a16_plan(M, N, K, G)[0] == 0
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=M + K)
    qd, sd = torch.from_numpy(oi.pack_gptq(q)).cuda(), torch.from_numpy(s).cuda()
    zd = torch.from_numpy(oi.pack_zeros(z)).cuda()
    Ad = A.cuda()
    Y = wo.matmul_int4(Ad, wo.prepack_int4(qd), sd, zd, G)
    assert og.max_rel_err(Y, oi.w4a16_ref(A, q, s, z, G)) <= 1e-3
    assert torch.equal(wo.matmul_int4_fused(Ad, wo.prepack_int4_fused(qd, sd, zd, G), G), Y)


# Narrow N at M <= 4 (under half a 16-column slice per CU): the planner's matrix-pipe decode,
# or, at long K with enough rows, the skinny kernel with a K split (K = 14336, N = 512:
# M >= 2; K = 11008, N = 1024: M >= 3; K = 8192, N = 256: M >= 3).  Within the oracle's bar;
# where the decode runs, bit-equal to the fused layout (same kernel, same values).
@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("K,N", [(4096, 256), (1024, 1536), (8192, 256), (11008, 1024),
                                 (14336, 512)])
def test_w4a16_narrow_n(wo, M, K, N):
    G = 128
    plan = wo.w4a16_plan(M, N, K, G)
    report("w4a16_narrow_n", M=M, K=K, N=N, plan=plan)
    skinny = (K, N) == (14336, 512) and M >= 2 or K in (8192, 11008) and M >= 3 and N <= 1024
    assert plan[0] == (4 if skinny else 0)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=5 * M + K + N)
    qd, sd = torch.from_numpy(oi.pack_gptq(q)).cuda(), torch.from_numpy(s).cuda()
    zd = torch.from_numpy(oi.pack_zeros(z)).cuda()
    Ad = A.cuda()
    Y = wo.matmul_int4(Ad, wo.prepack_int4(qd), sd, zd, G)
    assert torch.isfinite(Y).all()
    assert og.max_rel_err(Y, oi.w4a16_ref(A, q, s, z, G)) <= 1e-3
    Yf = wo.matmul_int4_fused(Ad, wo.prepack_int4_fused(qd, sd, zd, G), G)
    if skinny:
        assert og.max_rel_err(Yf, oi.w4a16_ref(A, q, s, z, G)) <= 1e-3
    else:
        assert torch.equal(Yf, Y)


def test_w4a16_fused_errors(wo):
    A, q, s, z = oi.make_inputs(5, 512, 64, 128, seed=3)
    qd, sd = torch.from_numpy(oi.pack_gptq(q)).cuda(), torch.from_numpy(s).cuda()
    f = wo.prepack_int4_fused(qd, sd, torch.from_numpy(z).cuda(), 128)
    with pytest.raises(RuntimeError, match="decode kernel only"):
        wo.matmul_int4_fused(A.cuda(), f, 128)  # M = 5
    with pytest.raises(RuntimeError, match="Inner dimensions"):
        wo.matmul_int4_fused(A[:1, :384].contiguous().cuda(), f, 128)
    with pytest.raises(RuntimeError, match="fused must be"):
        wo.matmul_int4_fused(A[:1].cuda(), wo.prepack_int4(qd), 128)
    with pytest.raises(RuntimeError, match="128"):
        wo.prepack_int4_fused(qd, torch.from_numpy(oi.make_inputs(1, 512, 64, 64, seed=1)[2]).cuda(),
                              torch.from_numpy(oi.make_inputs(1, 512, 64, 64, seed=1)[3]).cuda(), 64)


# AutoAWQ import: bit-exact conversion to the GPTQ layout and packed zeros, and the same
# product as the GPTQ-layout path.
@pytest.mark.parametrize("K,N,G", [(256, 64, 64), (4096, 1024, 128)])
def test_int4_from_awq_bit_exact(wo, K, N, G):
    rng = np.random.default_rng(K + N)
    q = rng.integers(0, 16, (K, N), dtype=np.uint8)
    z = rng.integers(0, 16, (K // G, N), dtype=np.uint8)
    qw, qz = wo.int4_from_awq(torch.from_numpy(oi.pack_awq(q)).cuda(), torch.from_numpy(oi.pack_awq(z)).cuda())
    assert np.array_equal(qw.cpu().numpy(), oi.pack_gptq(q))
    assert np.array_equal(qz.cpu().numpy(), oi.pack_zeros(z))


# fp16 output: every kernel (decode, skinny, GEMM; with and without a K split) rounds its
# fp32 result once, so the fp16 output equals the fp32 output converted.
@pytest.mark.parametrize("M", [1, 2, 3, 5, 16, 33, 300])
@pytest.mark.parametrize("K,N,G", [(4096, 1024, 128), (1024, 352, 64)])
def test_w4a16_fp16_output(wo, M, K, N, G):
    report("w4a16_f16out", M=M, K=K, N=N, G=G)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=M + K + N)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    args = (A.cuda(), pk, torch.from_numpy(s).cuda(), torch.from_numpy(oi.pack_zeros(z)).cuda(), G)
    Y32 = wo.matmul_int4(*args)
    Y16 = wo.matmul_int4(*args, out_dtype=torch.float16)
    assert Y16.dtype == torch.float16 and Y16.shape == Y32.shape
    assert torch.equal(Y16, Y32.half())
    assert torch.equal(wo.matmul_int4(*args, out_dtype=torch.float32), Y32)


def test_w4a16_zero_when_q_equals_z(wo):
    K, N, G = 256, 64, 128
    q = np.full((K, N), 9, dtype=np.uint8)
    z = np.full((K // G, N), 9, dtype=np.uint8)
    s = np.full((K // G, N), 0.01, dtype=np.float16)
    A = torch.randn(4, K).half()
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    Y = wo.matmul_int4(A.cuda(), pk, torch.from_numpy(s).cuda(), torch.from_numpy(z).cuda(), G)
    assert torch.count_nonzero(Y) == 0


def test_w4a16_integer_weights_exact(wo):
    # s = 1, z = 0 and small integer activations: every sum exact
    K, N, G = 512, 64, 128
    q = np.random.default_rng(1).integers(0, 16, (K, N), dtype=np.uint8)
    A = torch.randint(-2, 3, (16, K)).half()
    s = np.ones((K // G, N), dtype=np.float16)
    z = np.zeros((K // G, N), dtype=np.uint8)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    for m in (1, 4, 16):
        Y = wo.matmul_int4(A[:m].cuda(), pk, torch.from_numpy(s).cuda(), torch.from_numpy(z).cuda(), G)
        assert torch.equal(Y.cpu(), A[:m].float() @ torch.from_numpy(q.astype(np.float32)))


def test_w4a16_errors(wo):
    pk = torch.zeros(4, 1, 32, 4, dtype=torch.int32, device="cuda")  # prepacked K=64, N=64
    A = torch.zeros(1, 64, dtype=torch.half, device="cuda")
    s = torch.zeros(1, 64, dtype=torch.half, device="cuda")
    z = torch.zeros(1, 8, dtype=torch.int32, device="cuda")
    with pytest.raises(RuntimeError, match="scales must be float16"):
        wo.matmul_int4(A, pk, s.float(), z, 64)
    with pytest.raises(RuntimeError, match="Inner dimensions must match"):
        wo.matmul_int4(torch.zeros(1, 32, dtype=torch.half, device="cuda"), pk, s, z, 64)
    s3 = torch.zeros(4, 1, 16, dtype=torch.half, device="cuda")
    with pytest.raises(RuntimeError, match="sliced zeros must be int32"):
        wo.matmul_int4(A, pk, s3, z, 64)
    with pytest.raises(RuntimeError, match="must be a multiple of 64"):
        wo.prepack_int4(torch.zeros(3, 64, dtype=torch.int32, device="cuda"))
    # a GPTQ qweight [K/8, N] where prepacked weights belong is rejected, not read as garbage
    with pytest.raises(RuntimeError, match="output of prepack_int4"):
        wo.matmul_int4(A, torch.zeros(8, 64, dtype=torch.int32, device="cuda"), s, z, 64)
    with pytest.raises(RuntimeError, match="output of prepack_int4"):
        wo.unprepack_int4(torch.zeros(8, 64, dtype=torch.int32, device="cuda"))


# Tiny-magnitude activations: the decode kernel pre-scales a quarter of the activations by
# 1/16 in fp16, which is inexact for fp16-subnormal |a| < 2^-10; the error stays far inside
# the bound (a relative error against max|Y|).
@pytest.mark.parametrize("M", [1, 2, 16])
def test_w4a16_tiny_activations(wo, M):
    K, N, G = 4096, 4096, 128
    report("w4a16_tiny", M=M)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=31 + M)
    A = (A.float() * 1e-4).half()
    ref = oi.w4a16_ref(A, q, s, z, G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    Y = wo.matmul_int4(A.cuda(), pk, torch.from_numpy(s).cuda(), torch.from_numpy(oi.pack_zeros(z)).cuda(), G)
    assert og.max_rel_err(Y, ref) <= 1e-3


# GPTQ checkpoints (int4_from_gptq).  v1 stores z - 1: the adapter's zeros equal the packed
# true zeros bit for bit, and v2 passes them through.
@pytest.mark.parametrize("K,N,G", [(256, 64, 64), (4096, 1024, 128)])
def test_int4_from_gptq_zeros_bit_exact(wo, K, N, G):
    rng = np.random.default_rng(K + 3 * N)
    q = rng.integers(0, 16, (K, N), dtype=np.uint8)
    z = rng.integers(1, 16, (K // G, N), dtype=np.uint8)
    qw = torch.from_numpy(oi.pack_gptq(q)).cuda()
    qw1, zo1, perm1 = wo.int4_from_gptq(qw, torch.from_numpy(oi.pack_gptq_v1_zeros(z)).cuda())
    assert perm1 is None and torch.equal(qw1, qw)
    assert np.array_equal(zo1.cpu().numpy(), oi.pack_zeros(z))
    z2 = rng.integers(0, 16, (K // G, N), dtype=np.uint8)
    _, zo2, _ = wo.int4_from_gptq(qw, torch.from_numpy(oi.pack_zeros(z2)).cuda(), zero_format="v2")
    assert np.array_equal(zo2.cpu().numpy(), oi.pack_zeros(z2))


def test_int4_from_gptq_v1_q_equals_z_is_zero(wo):
    # q == z in every group: with v1 zeros stored as z - 1 every product term is exactly 0
    K, N, G = 1024, 256, 128
    rng = np.random.default_rng(9)
    z = rng.integers(1, 16, (K // G, N), dtype=np.uint8)
    q = np.repeat(z, G, axis=0)
    s = rng.uniform(0.001, 0.02, (K // G, N)).astype(np.float16)
    qw, zo, _ = wo.int4_from_gptq(torch.from_numpy(oi.pack_gptq(q)).cuda(),
                                  torch.from_numpy(oi.pack_gptq_v1_zeros(z)).cuda())
    pk = wo.prepack_int4(qw)
    # the same zeros read as v2 (no +1): every column is off by s * sum(a) per group
    qw2, zo2, _ = wo.int4_from_gptq(torch.from_numpy(oi.pack_gptq(q)).cuda(),
                                    torch.from_numpy(oi.pack_gptq_v1_zeros(z)).cuda(),
                                    zero_format="v2")
    for M in (1, 5, 40):
        A = torch.randn(M, K, generator=torch.Generator().manual_seed(M)).half().cuda()
        Y = wo.matmul_int4(A, pk, torch.from_numpy(s).cuda(), zo, G)
        if M <= 2 and wo.w4a16_plan(M, N, K, G)[0] == 0:
            # the M <= 2 decode subtracts the zero point through fp32 sums of the activations:
            # a difference of two sums of the same terms, zero up to their rounding (a few
            # fp32 ulps of the offset term 1024 s sum|a| per group)
            bound = 1e-6 * 1024 * float(s.max()) * A.float().abs().sum(dim=1, keepdim=True)
            assert (Y.abs() <= bound).all()
            Yw = wo.matmul_int4(A, wo.prepack_int4(qw2), torch.from_numpy(s).cuda(), zo2, G)
            assert (Yw.abs() > 10 * bound).any()
        else:
            assert torch.count_nonzero(Y) == 0


@pytest.mark.parametrize("M", [1, 16, 128])
def test_int4_from_gptq_g_idx(wo, M):
    K, N, G = 4096, 1024, 128
    report("gptq_g_idx", M=M, K=K, N=N, G=G)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=40 + M)
    z = np.maximum(z, 1)  # v1 zero points are 1..16
    qw = torch.from_numpy(oi.pack_gptq(q)).cuda()
    qz = torch.from_numpy(oi.pack_gptq_v1_zeros(z)).cuda()
    sd = torch.from_numpy(s).cuda()
    # a plain g_idx (k // G) is the plain layout: no permutation, the same bits
    plain = torch.arange(K, dtype=torch.int32, device="cuda") // G
    qw0, zo0, perm0 = wo.int4_from_gptq(qw, qz)
    qwp, zop, permp = wo.int4_from_gptq(qw, qz, plain)
    assert perm0 is None and permp is None and torch.equal(qw0, qwp) and torch.equal(zo0, zop)
    Y0 = wo.matmul_int4(A.cuda(), wo.prepack_int4(qw0), sd, zo0, G)
    assert og.max_rel_err(Y0, oi.gptq_w4a16_ref(A, oi.pack_gptq(q), oi.pack_gptq_v1_zeros(z), s, None)) <= 1e-3
    # act order: rows regrouped by a stable sort, A's columns gathered by perm
    g_idx = oi.act_order_g_idx(K, G, seed=M)
    qwa, zoa, perma = wo.int4_from_gptq(qw, qz, torch.from_numpy(g_idx).cuda())
    assert perma is not None and perma.dtype == torch.int64
    assert np.array_equal(perma.cpu().numpy(), np.argsort(g_idx, kind="stable"))
    assert np.array_equal(wo.unpack_int4(qwa).cpu().numpy(), q[perma.cpu().numpy()])
    Ya = wo.matmul_int4(A.cuda(), wo.prepack_int4(qwa), sd, zoa, G, perm=perma)
    ref = oi.gptq_w4a16_ref(A, oi.pack_gptq(q), oi.pack_gptq_v1_zeros(z), s, g_idx)
    assert og.max_rel_err(Ya, ref) <= 1e-3


def test_int4_from_gptq_errors(wo):
    K, N, G = 256, 64, 64
    qw = torch.zeros(K // 8, N, dtype=torch.int32, device="cuda")
    bad = torch.from_numpy(oi.pack_zeros(np.full((K // G, N), 15, dtype=np.uint8))).cuda()
    with pytest.raises(RuntimeError, match="zero point 16"):
        wo.int4_from_gptq(qw, bad)                     # v1 nibble 15 = zero point 16
    wo.int4_from_gptq(qw, bad, zero_format="v2")       # as stored in v2: fine
    qz = torch.zeros(K // G, N // 8, dtype=torch.int32, device="cuda")
    uneven = torch.zeros(K, dtype=torch.int32, device="cuda")  # every row in group 0
    with pytest.raises(RuntimeError, match="exactly group_size rows"):
        wo.int4_from_gptq(qw, qz, uneven)
    with pytest.raises(RuntimeError, match="zero_format"):
        wo.int4_from_gptq(qw, qz, zero_format="v3")
