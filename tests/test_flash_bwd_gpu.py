"""GPU parity of the flash-attention training path (forward log-sum-exp, backward dQ/dK/dV)
against the CPU oracle: torch autograd of FP32 attention on the same fp16 inputs.

Tolerances.  The log-sum-exp is FP32 arithmetic on exact fp16 products: absolute 1e-4 plus
relative 1e-5.  Gradients: max |got - ref| / max |ref| <= 1e-3 per tensor, the forward's
bar; the kernels round P and dS to fp16 for the matrix cores and the outputs to fp16
(each 2^-11 relative), and Delta is formed from the fp16 O, as in every fp16 flash-attention
backward pass.
"""
import math

import numpy as np
import pytest
import torch

from oracle import attention as oatt
from oracle import gemm as og
from tests.conftest import report

pytestmark = pytest.mark.gpu
TOL = 1e-3


def _grads_close(got, want, tol=TOL):
    errs = []
    for name, g, w in zip(("dQ", "dK", "dV"), got, want):
        assert g.dtype == torch.float16 and tuple(g.shape) == tuple(w.shape), name
        g = g.float().cpu()
        assert torch.isfinite(g).all(), name
        err = og.max_rel_err(g, w)
        errs.append(err)
        assert err <= tol, f"{name}: max rel err {err:.3e}"
    return errs


def _dout(shape, seed):
    return torch.randn(*shape, generator=torch.Generator().manual_seed(seed)).half()


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D", [(2, 4, 4, 300, 300, 128), (1, 8, 2, 257, 100, 64),
                                             (1, 2, 2, 1, 1, 128)])
def test_forward_lse(wo, causal, B, H, Hkv, Sq, Sk, D):
    report("flash_lse", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=Sq + D, Sk=Sk, Hkv=Hkv)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
    assert lse.dtype == torch.float32 and tuple(lse.shape) == (B, H, Sq)
    ref = oatt.lse_ref(Q, K, causal)
    assert torch.allclose(lse.cpu(), ref, atol=1e-4, rtol=1e-5), (lse.cpu() - ref).abs().max()
    # the training forward computes the same output bits as the inference forward
    assert torch.equal(O, wo.flash_attention(Q.cuda(), K.cuda(), V.cuda(), causal))


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,Sq,Sk,D", [(2, 4, 512, 512, 128), (2, 4, 512, 512, 64),
                                         (1, 3, 77, 77, 128), (1, 2, 300, 100, 64),
                                         (1, 2, 100, 300, 128), (1, 2, 2, 3, 64),
                                         (1, 2, 129, 129, 128), (1, 2, 1000, 1000, 64)])
def test_flash_bwd_shapes(wo, causal, B, H, Sq, Sk, D):
    report("flash_bwd", B=B, H=H, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=Sq * 3 + Sk + D, Sk=Sk)
    dO = _dout((B, H, Sq, D), Sq + 1)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
    got = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O, lse, causal)
    errs = _grads_close(got, oatt.sdpa_bwd_ref(Q, K, V, dO, causal))
    print(f"[err] dQ {errs[0]:.2e} dK {errs[1]:.2e} dV {errs[2]:.2e}", flush=True)


# Head dims other than 64, 128 and 256 (see the forward's head-dim test): the dQ and dK/dV
# kernels load the missing d columns as zeros and do not store them; D = 256 splits the
# dK/dV columns over two workgroups; grouped-query heads.
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [16, 32, 48, 80, 96, 112, 33, 100, 136, 160, 200, 256, 250])
def test_flash_bwd_head_dims(wo, causal, D):
    B, H, Hkv, Sq, Sk = 1, 4, 2, 300, 200
    report("flash_bwd_head_dim", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=900 + D, Sk=Sk, Hkv=Hkv)
    dO = _dout((B, H, Sq, D), D)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
    got = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O, lse, causal)
    errs = _grads_close(got, oatt.sdpa_bwd_ref(Q, K, V, dO, causal))
    print(f"[err] D {D} dQ {errs[0]:.2e} dK {errs[1]:.2e} dV {errs[2]:.2e}", flush=True)


# D = 256 over many key and query tiles (the 2-deep rings, the dK/dV column split), ragged
# lengths, grouped-query heads.
@pytest.mark.parametrize("causal", [False, True])
def test_flash_bwd_head_dim_256_long(wo, causal):
    B, H, Hkv, Sq, Sk, D = 1, 4, 2, 1100, 900, 256
    report("flash_bwd_d256", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=2560, Sk=Sk, Hkv=Hkv)
    dO = _dout((B, H, Sq, D), 2561)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
    got = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O, lse, causal)
    errs = _grads_close(got, oatt.sdpa_bwd_ref(Q, K, V, dO, causal))
    print(f"[err] dQ {errs[0]:.2e} dK {errs[1]:.2e} dV {errs[2]:.2e}", flush=True)


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("Sq,D", [(1, 64), (77, 128)])
def test_flash_bwd_single_key(wo, causal, Sq, D):
    # One key: P = 1 for every query, so dV = sum of the dO rows, and dS = P (dP - Delta) = 0
    # gives dQ = dK = 0 (up to the FP32 rounding of dP - Delta; relative errors against a
    # zero reference say nothing, so this case is checked in closed form).
    report("flash_bwd_single_key", Sq=Sq, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(1, 2, Sq, D, seed=Sq + D, Sk=1)
    dO = _dout((1, 2, Sq, D), 3)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
    dQ, dK, dV = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O, lse, causal)
    want = dO.float().sum(dim=2, keepdim=True)
    assert og.max_rel_err(dV.float().cpu(), want) <= TOL
    assert dQ.float().abs().max().item() <= 1e-4 and dK.float().abs().max().item() <= 1e-4


@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D", [(2, 8, 2, 300, 300, 128), (1, 8, 1, 257, 257, 64),
                                             (1, 6, 3, 100, 333, 128)])
def test_flash_bwd_gqa(wo, causal, B, H, Hkv, Sq, Sk, D):
    # dK and dV of a key/value head are summed over the query heads that read it
    report("flash_bwd_gqa", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=H * 100 + Hkv + Sq, Sk=Sk, Hkv=Hkv)
    dO = _dout((B, H, Sq, D), H + Sq)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
    got = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O, lse, causal)
    _grads_close(got, oatt.sdpa_bwd_ref(Q, K, V, dO, causal))


# [4, 32, 4096, 128].  The CPU oracle runs on a sample of heads at the full
# sequence length; every head is checked against the closed forms (dV rows sum to the dO
# rows, dK rows sum to zero).
@pytest.mark.parametrize("causal", [False, True])
def test_flash_bwd_baseline_config(wo, causal):
    B, H, S, D = 4, 32, 4096, 128
    report("flash_bwd_baseline", B=B, H=H, S=S, D=D, causal=causal)
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=42 + 4)
    dO = _dout((B, H, S, D), 77)
    Qd, Kd, Vd, dOd = Q.cuda(), K.cuda(), V.cuda(), dO.cuda()
    O, lse = wo.flash_attention_forward(Qd, Kd, Vd, causal)
    dQ, dK, dV = wo.flash_attention_backward(dOd, Qd, Kd, Vd, O, lse, causal)
    for t in (dQ, dK, dV):
        assert torch.isfinite(t).all()
    sum_dv = dV.float().sum(dim=2)
    sum_do = dOd.float().sum(dim=2)
    assert og.max_rel_err(sum_dv.cpu(), sum_do.cpu()) <= 1e-3
    # sum_j dK_j = 0 up to rounding: compare with the scale of the row sums' terms
    assert dK.float().sum(dim=2).abs().max().item() <= 1e-3 * dK.float().abs().sum(dim=2).max().item()
    for b, h in [(0, 0), (3, 31)]:
        sl = lambda X: X[b:b + 1, h:h + 1]
        ref = oatt.sdpa_bwd_ref(sl(Q), sl(K), sl(V), sl(dO), causal)
        _grads_close((sl(dQ), sl(dK), sl(dV)), ref)


# Ragged packed sequences: lengths 1, 0, not multiples of the tiles, different query and
# key lengths, a sequence with no keys (dQ = 0) and one with no queries (dK = dV = 0).
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("H,Hkv,D", [(4, 4, 128), (8, 2, 64), (4, 2, 80), (4, 4, 36), (4, 2, 256)])
def test_flash_bwd_varlen(wo, causal, H, Hkv, D):
    lens_q = [300, 1, 0, 700, 64, 5]
    lens_k = [300, 1, 9, 700, 77, 0]
    report("flash_bwd_varlen", H=H, Hkv=Hkv, D=D, causal=causal)
    cu_q = torch.tensor([0] + list(np.cumsum(lens_q)), dtype=torch.int32)
    cu_k = torch.tensor([0] + list(np.cumsum(lens_k)), dtype=torch.int32)
    g = torch.Generator().manual_seed(H * 10 + D)
    q = torch.randn(int(cu_q[-1]), H, D, generator=g).half()
    k = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).half()
    v = torch.randn(int(cu_k[-1]), Hkv, D, generator=g).half()
    dO = torch.randn(int(cu_q[-1]), H, D, generator=g).half()
    args = (cu_q.cuda(), cu_k.cuda(), max(lens_q), max(lens_k))
    O, lse = wo.flash_attention_varlen_forward(q.cuda(), k.cuda(), v.cuda(), *args, causal=causal)
    ref_lse = oatt.lse_varlen_ref(q, k, cu_q, cu_k, causal)
    assert torch.equal(torch.isinf(lse.cpu()), torch.isinf(ref_lse))
    fin = torch.isfinite(ref_lse)
    assert torch.allclose(lse.cpu()[fin], ref_lse[fin], atol=1e-4, rtol=1e-5)
    got = wo.flash_attention_varlen_backward(dO.cuda(), q.cuda(), k.cuda(), v.cuda(), O, lse, *args,
                                             causal=causal)
    _grads_close(got, oatt.sdpa_varlen_bwd_ref(q, k, v, dO, cu_q, cu_k, causal))
    a, e = int(cu_q[5]), int(cu_q[6])
    assert torch.count_nonzero(got[0][a:e]) == 0          # the sequence without keys
    a, e = int(cu_k[2]), int(cu_k[3])
    assert torch.count_nonzero(got[1][a:e]) == 0 and torch.count_nonzero(got[2][a:e]) == 0


def test_flash_bwd_varlen_equals_dense(wo):
    B, H, S, D = 3, 4, 333, 128
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=13)
    dO = _dout((B, H, S, D), 14)
    pack = lambda X: X.transpose(1, 2).reshape(B * S, H, D).contiguous().cuda()
    cu = torch.arange(0, (B + 1) * S, S, dtype=torch.int32).cuda()
    for causal in (False, True):
        O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), causal)
        dense = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O, lse, causal)
        Op, lsep = wo.flash_attention_varlen_forward(pack(Q), pack(K), pack(V), cu, cu, S, S,
                                                     causal=causal)
        assert torch.equal(lsep, lse.permute(1, 0, 2).reshape(H, B * S))
        packed = wo.flash_attention_varlen_backward(pack(dO), pack(Q), pack(K), pack(V), Op, lsep,
                                                    cu, cu, S, S, causal=causal)
        for p_, d_ in zip(packed, dense):
            assert torch.equal(p_, d_.transpose(1, 2).reshape(B * S, H, D))


def test_flash_autograd(wo):
    # flash_attention is differentiable when its inputs require grad: the backward pass is
    # the fused kernels (same bits as calling them directly) and matches the oracle.
    B, H, Hkv, S, D = 2, 4, 2, 200, 64
    Q, K, V = oatt.make_inputs(B, H, S, D, seed=31, Hkv=Hkv)
    dO = _dout((B, H, S, D), 32)
    q, k, v = (X.cuda().requires_grad_() for X in (Q, K, V))
    O = wo.flash_attention(q, k, v, causal=True)
    assert O.requires_grad
    O.backward(dO.cuda())
    O2, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), True)
    direct = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O2, lse, True)
    for g, d in zip((q.grad, k.grad, v.grad), direct):
        assert torch.equal(g, d)
    _grads_close((q.grad, k.grad, v.grad), oatt.sdpa_bwd_ref(Q, K, V, dO, True))
    with torch.no_grad():
        assert not wo.flash_attention(q, k, v).requires_grad


def test_flash_bwd_deterministic(wo):
    Q, K, V = oatt.make_inputs(1, 8, 1024, 128, seed=41, Hkv=2)
    dO = _dout((1, 8, 1024, 128), 42)
    O, lse = wo.flash_attention_forward(Q.cuda(), K.cuda(), V.cuda(), True)
    a = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O, lse, True)
    b = wo.flash_attention_backward(dO.cuda(), Q.cuda(), K.cuda(), V.cuda(), O, lse, True)
    for x, y in zip(a, b):
        assert torch.equal(x, y)


def test_flash_bwd_no_queries(wo):
    # Sq = 0: dQ is empty and dK = dV = 0 (written, not left uninitialised)
    Q = torch.zeros(1, 2, 0, 64, dtype=torch.half, device="cuda")
    K = torch.randn(1, 2, 50, 64).half().cuda()
    O, lse = wo.flash_attention_forward(Q, K, K)
    dQ, dK, dV = wo.flash_attention_backward(Q, Q, K, K, O, lse)
    assert dQ.shape == Q.shape and torch.count_nonzero(dK) == 0 and torch.count_nonzero(dV) == 0


def test_flash_bwd_errors(wo):
    Qd = torch.zeros(1, 1, 8, 264, dtype=torch.half, device="cuda")
    with pytest.raises(RuntimeError, match="head_dim must be between 1 and 256"):
        wo.flash_attention_backward(Qd, Qd, Qd, Qd, Qd, torch.zeros(1, 1, 8, device="cuda"))
    Q, K, V = (X.cuda() for X in oatt.make_inputs(1, 2, 16, 64, seed=1))
    O, lse = wo.flash_attention_forward(Q, K, V)
    with pytest.raises(RuntimeError, match="lse must be float32"):
        wo.flash_attention_backward(Q, Q, K, V, O, lse[:, :, :8])
    with pytest.raises(RuntimeError, match="dO and O must have Q's shape"):
        wo.flash_attention_backward(Q[:, :, :8], Q, K, V, O, lse)
    with pytest.raises(RuntimeError, match="dO and O must be float16"):
        wo.flash_attention_backward(Q.float(), Q, K, V, O, lse)


# Grouped-query split of the dK/dV kernel (few K/V heads, short sequences): with the
# workspace wmma_flash_attn_bwd_split_workspace_size reports, the group's query heads run
# on separate workgroups whose fp32 partial dK, dV are added in part order; with only the
# row statistics, one workgroup sums the group in registers.  Both match the oracle; dQ is
# the same computation either way (bit-equal), dK and dV agree to fp32 summation order.
@pytest.mark.parametrize("B,H,Hkv,Sq,Sk,D,causal", [
    (1, 16, 4, 1024, 1024, 128, False), (1, 16, 4, 1024, 1024, 128, True),
    (2, 8, 1, 300, 500, 64, True), (1, 8, 2, 257, 257, 256, False), (1, 6, 3, 130, 130, 72, True)])
def test_flash_bwd_group_split(wo, B, H, Hkv, Sq, Sk, D, causal):
    import ctypes
    lib = ctypes.CDLL(wo.LIBRARY_PATH)
    vp, i32, f32, sz = ctypes.c_void_p, ctypes.c_int, ctypes.c_float, ctypes.c_size_t
    lib.wmma_flash_attn_bwd_workspace_size.restype = sz
    lib.wmma_flash_attn_bwd_workspace_size.argtypes = [i32] * 3
    lib.wmma_flash_attn_bwd_split_workspace_size.restype = sz
    lib.wmma_flash_attn_bwd_split_workspace_size.argtypes = [i32] * 7
    lib.wmma_flash_attn_bwd.argtypes = [vp] * 10 + [sz] + [i32] * 6 + [f32, i32, vp]
    base = lib.wmma_flash_attn_bwd_workspace_size(B, H, Sq)
    full = lib.wmma_flash_attn_bwd_split_workspace_size(B, H, Hkv, Sq, Sk, D, 1 if causal else 0)
    report("flash_bwd_group_split", B=B, H=H, Hkv=Hkv, Sq=Sq, Sk=Sk, D=D, causal=causal, ws=full)
    assert full > base, "the shape should take the split"
    Q, K, V = oatt.make_inputs(B, H, Sq, D, seed=B + H + Sq + D, Sk=Sk, Hkv=Hkv)
    dO = _dout((B, H, Sq, D), H * 3 + Sq)
    Qd, Kd, Vd, dOd = Q.cuda(), K.cuda(), V.cuda(), dO.cuda()
    O, lse = wo.flash_attention_forward(Qd, Kd, Vd, causal)
    res = []
    for wsb in (full, base):
        ws = torch.empty(wsb, dtype=torch.uint8, device="cuda")
        dQ, dK, dV = torch.empty_like(Qd), torch.empty_like(Kd), torch.empty_like(Vd)
        rc = lib.wmma_flash_attn_bwd(dOd.data_ptr(), Qd.data_ptr(), Kd.data_ptr(), Vd.data_ptr(), O.data_ptr(),
                                     lse.data_ptr(), dQ.data_ptr(), dK.data_ptr(), dV.data_ptr(), ws.data_ptr(),
                                     wsb, B, H, Hkv, Sq, Sk, D, 1.0 / math.sqrt(D), 1 if causal else 0,
                                     torch.cuda.current_stream().cuda_stream)
        assert rc == 0
        res.append((dQ, dK, dV))
    want = oatt.sdpa_bwd_ref(Q, K, V, dO, causal)
    _grads_close(res[0], want)
    _grads_close(res[1], want)
    assert torch.equal(res[0][0], res[1][0])
    for a, b in zip(res[0][1:], res[1][1:]):
        assert og.max_rel_err(a.float(), b.float()) <= 1e-3
    # the torch layer passes the split workspace: its gradients are the split ones
    got = wo.flash_attention_backward(dOd, Qd, Kd, Vd, O, lse, causal)
    for a, b in zip(got, res[0]):
        assert torch.equal(a, b)
