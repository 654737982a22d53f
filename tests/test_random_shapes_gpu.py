"""Randomised shape sweep: GEMM, W4A16 (both layouts) and flash attention (forward and backward) on shapes
drawn from a fixed seed, each against the fp32 CPU oracle.

The hand-picked cases of the other GPU test files pin the boundaries the kernels were
written for; this sweep covers what lies between them -- ragged M, N, K (multiples of 8 or
not), every planner branch a shape can fall into (skinny, tiled, split-K, the W4A16 decode,
skinny and GEMM kernels), group sizes, zero-point formats, output dtypes, grouped-query
heads and head dims up to 256.  The case list is drawn once from numpy's PCG64 with seed
20261202, so every run checks the same shapes and a failing case is reproducible from its
id.

Bars: GEMM max rel err <= 1e-4 (fp32 accumulation of exact fp16 products; the documented
bar is 1e-3); W4A16, flash forward and each flash gradient 1e-3, the documented bar.
Every path is deterministic, so each case also repeats its call (with other work and fresh
allocations in between) and requires bit-identical results: a race that corrupts a call
now and then shows there, not only as an error above the bar.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import gemm as og
from oracle import int4 as oi
from tests.conftest import report

pytestmark = pytest.mark.gpu

_RNG = np.random.Generator(np.random.PCG64(20261202))


def _dim(lo, hi, p_mult8=0.6):
    """A size in [lo, hi], a multiple of 8 with probability p_mult8 (when one exists)."""
    v = int(_RNG.integers(lo, hi + 1))
    if _RNG.random() < p_mult8 and hi >= 8:
        v = max(8, (v // 8) * 8)
    return v


def _m():
    r = _RNG.random()
    if r < 0.35:
        return int(_RNG.integers(1, 17))      # skinny kernel / W4A16 decode and skinny
    if r < 0.75:
        return int(_RNG.integers(17, 301))    # split-K tiles / W4A16 GEMM at small M
    return int(_RNG.integers(301, 1101))      # full tiles


def _gemm_cases(n):
    out = []
    for _ in range(n):
        M, N, K = _m(), _dim(1, 1200), _dim(1, 1200)
        alpha = 1.0 if _RNG.random() < 0.4 else float(np.round(_RNG.uniform(-2, 2), 3))
        beta = 0.0 if _RNG.random() < 0.4 else float(np.round(_RNG.uniform(-2, 2), 3))
        out.append((M, N, K, alpha, beta))
    return out


def _w4_cases(n):
    out = []
    for _ in range(n):
        G = int(_RNG.choice([32, 64, 128, 256]))
        step = int(np.lcm(G, 64))
        K = step * int(_RNG.integers(1, max(2, 4096 // step) + 1))
        N = 32 * int(_RNG.integers(1, 80))
        zf = str(_RNG.choice(["packed", "u8", "sliced"]))
        f16out = bool(_RNG.random() < 0.3)
        out.append((_m(), N, K, G, zf, f16out))
    return out


def _flash_cases(n, dmax=256):
    out = []
    for _ in range(n):
        B = int(_RNG.integers(1, 3))
        Hkv = int(_RNG.choice([1, 2, 4]))
        H = Hkv * int(_RNG.choice([1, 2, 4]))
        Sq, Sk = int(_RNG.integers(1, 600)), int(_RNG.integers(1, 600))
        D = int(_RNG.integers(1, dmax + 1))
        if _RNG.random() < 0.6:
            D = max(8, (D // 8) * 8)
        causal = bool(_RNG.random() < 0.5)
        out.append((B, H, Hkv, Sq, Sk, D, causal))
    return out


GEMM_CASES = _gemm_cases(40)
W4_CASES = _w4_cases(30)
FLASH_CASES = _flash_cases(24)
FLASH_BWD_CASES = _flash_cases(12)


@pytest.mark.parametrize("case", range(len(GEMM_CASES)))
def test_random_gemm(wo, case):
    M, N, K, alpha, beta = GEMM_CASES[case]
    report("random_gemm", case=case, M=M, N=N, K=K, alpha=alpha, beta=beta,
           plan=wo.gemm_plan(M, N, K))
    g = torch.Generator().manual_seed(1000 + case)
    A = torch.randn(M, K, generator=g).half()
    B = torch.randn(K, N, generator=g).half()
    C = torch.randn(M, N, generator=g)
    Y = wo.gemm(A.cuda(), B.cuda(), alpha, beta, C.cuda() if beta != 0.0 else None)
    ref = og.gemm_ref(A, B, alpha, beta, C)
    assert torch.isfinite(Y).all()
    err = og.max_rel_err(Y, ref)
    assert err <= 1e-4, f"max rel err {err:.3e}"
    P = wo.matmul(A.cuda(), B.cuda())
    assert og.max_rel_err(P, og.gemm_ref(A, B)) <= 1e-4
    for _ in range(2):
        assert torch.equal(wo.gemm(A.cuda(), B.cuda(), alpha, beta, C.cuda() if beta != 0.0 else None), Y)
        assert torch.equal(wo.matmul(A.cuda(), B.cuda()), P)


@pytest.mark.parametrize("case", range(len(W4_CASES)))
def test_random_w4a16(wo, case):
    M, N, K, G, zf, f16out = W4_CASES[case]
    report("random_w4a16", case=case, M=M, N=N, K=K, G=G, zeros=zf, f16out=f16out,
           plan=wo.w4a16_plan(M, N, K, G))
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=2000 + case)
    ref = oi.w4a16_ref(A, q, s, z, G)
    pk = wo.prepack_int4(torch.from_numpy(oi.pack_gptq(q)).cuda())
    sd = torch.from_numpy(s).cuda()
    zp = torch.from_numpy(oi.pack_zeros(z)).cuda()
    if zf == "packed":
        args = (sd, zp)
    elif zf == "u8":
        args = (sd, torch.from_numpy(z).cuda())
    else:
        args = wo.prepack_int4_params(sd, zp)
    kw = {"out_dtype": torch.float16} if f16out else {}
    Y = wo.matmul_int4(A.cuda(), pk, *args, G, **kw)
    assert Y.dtype == (torch.float16 if f16out else torch.float32)
    assert torch.isfinite(Y).all()
    err = og.max_rel_err(Y.float(), ref)
    assert err <= 1e-3, f"max rel err {err:.3e}"
    for _ in range(3):
        assert torch.equal(wo.matmul_int4(A.cuda(), pk, *args, G, **kw), Y)


@pytest.mark.parametrize("case", range(len(FLASH_CASES)))
def test_random_flash_forward(wo, case):
    B, H, Hkv, Sq, Sk, D, causal = FLASH_CASES[case]
    report("random_flash", case=case, B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=3000 + case, Sk=Sk, Hkv=Hkv)
    O = wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal)
    ref = oatt.sdpa_ref(Q, K, V, causal)
    assert O.dtype == torch.float16 and tuple(O.shape) == tuple(ref.shape)
    assert torch.isfinite(O).all()
    err = og.max_rel_err(O.float(), ref)
    assert err <= 1e-3, f"max rel err {err:.3e}"
    for _ in range(2):
        assert torch.equal(wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal=causal), O)


@pytest.mark.parametrize("case", range(len(FLASH_BWD_CASES)))
def test_random_flash_backward(wo, case):
    B, H, Hkv, Sq, Sk, D, causal = FLASH_BWD_CASES[case]
    report("random_flash_bwd", case=case, B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=4000 + case, Sk=Sk, Hkv=Hkv)
    dO = torch.randn(B, H, Sq, D, generator=torch.Generator().manual_seed(5000 + case)).half()
    Qd, Kd, Vd = (t.cuda().requires_grad_(True) for t in (Q, K, V))
    O = wo.flash_attention(Qd, Kd, Vd, causal=causal)
    O.backward(dO.cuda())
    # fp32 autograd of the CPU oracle on the same fp16 values
    Qr, Kr, Vr = (t.float().requires_grad_(True) for t in (Q, K, V))
    sc = oatt.resolve_scale(D, -1.0)
    Kx, Vx = oatt.expand_kv(Kr, H), oatt.expand_kv(Vr, H)
    Or = torch.nn.functional.scaled_dot_product_attention(Qr, Kx, Vx, is_causal=causal, scale=sc)
    Or.backward(dO.float())
    for name, got, want in (("dQ", Qd.grad, Qr.grad), ("dK", Kd.grad, Kr.grad), ("dV", Vd.grad, Vr.grad)):
        assert got.shape == want.shape
        assert torch.isfinite(got).all(), name
        err = og.max_rel_err(got.float(), want)
        assert err <= 1e-3, f"{name}: max rel err {err:.3e}"
    Q2, K2, V2 = (t.cuda().requires_grad_(True) for t in (Q, K, V))
    wo.flash_attention(Q2, K2, V2, causal=causal).backward(dO.cuda())
    for got, again in ((Qd.grad, Q2.grad), (Kd.grad, K2.grad), (Vd.grad, V2.grad)):
        assert torch.equal(got, again)


# The fused decode layout on its own seeded draw (so the cases above keep their shapes):
# M = 1..4, K a multiple of 128 up to 8192 (single-round and multi-round decode), N a
# multiple of 32, G = 128 * 2^j dividing K, fp32 or fp16 output.  Each case also checks the
# layout's exact inverse.
_FRNG = np.random.Generator(np.random.PCG64(20261203))


def _fused_cases(n):
    out = []
    for _ in range(n):
        G = int(_FRNG.choice([128, 256, 512]))
        K = G * int(_FRNG.integers(1, 8192 // G + 1))
        out.append((int(_FRNG.integers(1, 5)), 32 * int(_FRNG.integers(1, 65)), K, G,
                    bool(_FRNG.random() < 0.3)))
    return out


FUSED_CASES = _fused_cases(16)


@pytest.mark.parametrize("case", range(len(FUSED_CASES)))
def test_random_w4a16_fused(wo, case):
    M, N, K, G, f16out = FUSED_CASES[case]
    report("random_w4a16_fused", case=case, M=M, N=N, K=K, G=G, f16out=f16out)
    A, q, s, z = oi.make_inputs(M, K, N, G, seed=5000 + case)
    qd = torch.from_numpy(oi.pack_gptq(q)).cuda()
    sd, zp = torch.from_numpy(s).cuda(), torch.from_numpy(oi.pack_zeros(z)).cuda()
    f = wo.prepack_int4_fused(qd, sd, zp, G)
    kw = {"out_dtype": torch.float16} if f16out else {}
    Y = wo.matmul_int4_fused(A.cuda(), f, G, **kw)
    assert Y.dtype == (torch.float16 if f16out else torch.float32)
    assert torch.isfinite(Y).all()
    err = og.max_rel_err(Y.float(), oi.w4a16_ref(A, q, s, z, G))
    assert err <= 1e-3, f"max rel err {err:.3e}"
    q2, s2, z2 = wo.unprepack_int4_fused(f, G)
    assert torch.equal(q2, qd) and torch.equal(s2, sd) and torch.equal(z2, zp)
