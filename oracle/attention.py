"""Attention oracle (CPU).  Test infrastructure only -- see oracle/__init__.py.

The reference documents flash_attention(Q, K, V, causal=False, scale=-1.0) on
[B, H, N, D] fp16 tensors, default scale 1/sqrt(D), checked against PyTorch SDPA
(README.md:221-251).  Causal masking keeps key j <= query i (torch SDPA's is_causal,
top-left aligned).
"""
from __future__ import annotations

import math

import numpy as np
import torch
import torch.nn.functional as F


def resolve_scale(D: int, scale: float) -> float:
    """scale <= 0 selects the default 1/sqrt(D) (README.md:244)."""
    return scale if scale > 0 else 1.0 / math.sqrt(D)


def expand_kv(X, heads: int):
    """Grouped-query attention: key/value head j serves query heads j*g .. j*g+g-1,
    g = heads / X.shape[1] (torch SDPA's enable_gqa mapping)."""
    hkv = X.shape[1]
    assert heads % hkv == 0
    g = heads // hkv
    if isinstance(X, np.ndarray):
        return np.repeat(X, g, axis=1)
    return X.repeat_interleave(g, dim=1)


def sdpa_ref(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, causal: bool = False,
             scale: float = -1.0) -> torch.Tensor:
    """FP32 scaled-dot-product attention on the CPU (the library routine); K/V may carry
    fewer heads than Q (grouped-query attention, expanded by expand_kv)."""
    sc = resolve_scale(Q.shape[-1], scale)
    H = Q.shape[1]
    K, V = expand_kv(K.detach().cpu().float(), H), expand_kv(V.detach().cpu().float(), H)
    return F.scaled_dot_product_attention(Q.detach().cpu().float(), K, V, is_causal=causal,
                                          scale=sc)


def attention_naive_f64(Q: np.ndarray, K: np.ndarray, V: np.ndarray, causal: bool = False,
                        scale: float = -1.0) -> np.ndarray:
    """Explicit float64 softmax(scale * Q K^T + mask) V, for tiny shapes."""
    Q = np.asarray(Q, dtype=np.float64)
    K = expand_kv(np.asarray(K, dtype=np.float64), Q.shape[1])
    V = expand_kv(np.asarray(V, dtype=np.float64), Q.shape[1])
    sc = resolve_scale(Q.shape[-1], scale)
    S = np.einsum("...qd,...kd->...qk", Q, K) * sc
    if causal:
        sq, sk = S.shape[-2], S.shape[-1]
        mask = np.tril(np.ones((sq, sk), dtype=bool))
        S = np.where(mask, S, -np.inf)
    S = S - S.max(axis=-1, keepdims=True)
    P = np.exp(S)
    P = P / P.sum(axis=-1, keepdims=True)
    return np.einsum("...qk,...kd->...qd", P, V)


def make_inputs(B: int, H: int, S: int, D: int, seed: int, Sk: int | None = None,
                Hkv: int | None = None):
    """Seeded Q [B,H,S,D], K and V [B,Hkv,Sk,D] ~ N(0, 1) in fp16 (Hkv defaults to H)."""
    g = torch.Generator().manual_seed(seed)
    Sk = S if Sk is None else Sk
    Hkv = H if Hkv is None else Hkv
    Q = torch.randn(B, H, S, D, generator=g).half()
    K = torch.randn(B, Hkv, Sk, D, generator=g).half()
    V = torch.randn(B, Hkv, Sk, D, generator=g).half()
    return Q, K, V


def sdpa_varlen_ref(q, k, v, cu_q, cu_k, causal: bool = False, scale: float = -1.0):
    """Packed variable-length batches ([total, heads, D], sequence b in rows
    cu[b] .. cu[b+1]): sdpa_ref per sequence, top-left causal alignment per sequence; a
    query of a sequence with no keys gives zeros."""
    cu_q = [int(x) for x in cu_q]
    cu_k = [int(x) for x in cu_k]
    out = torch.zeros(q.shape[0], q.shape[1], q.shape[2], dtype=torch.float32)
    for b in range(len(cu_q) - 1):
        qa, qe, ka, ke = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        if qe <= qa or ke <= ka:
            continue
        Q = q[qa:qe].transpose(0, 1).unsqueeze(0)   # [1, H, Sq, D]
        K = k[ka:ke].transpose(0, 1).unsqueeze(0)
        V = v[ka:ke].transpose(0, 1).unsqueeze(0)
        out[qa:qe] = sdpa_ref(Q, K, V, causal, scale)[0].transpose(0, 1)
    return out


# ------------------------------------------------------------------------ training path --
# No reference counterpart: the reference's flash_attention is forward-only
# (README.md:221-251).  These restate the mathematics of its training extension -- the
# log-sum-exp a backward pass needs and the gradients of sum(O * dO) -- through the library
# routines (torch.logsumexp, torch autograd of scaled_dot_product_attention); the tests pin
# them against float64 finite differences and closed forms.

def lse_ref(Q, K, causal: bool = False, scale: float = -1.0) -> torch.Tensor:
    """Natural-log log-sum-exp of each row of scale * Q K^T over its unmasked keys, fp32
    [B, H, Sq]; +inf for a row with no key (the value the kernels store there)."""
    sc = resolve_scale(Q.shape[-1], scale)
    Qf = Q.detach().cpu().float()
    Kf = expand_kv(K.detach().cpu().float(), Q.shape[1])
    S = torch.matmul(Qf, Kf.transpose(-1, -2).contiguous()) * sc
    if causal:
        sq, sk = S.shape[-2], S.shape[-1]
        S = S.masked_fill(~torch.ones(sq, sk, dtype=torch.bool).tril(), float("-inf"))
    out = torch.logsumexp(S, dim=-1)
    return torch.where(torch.isneginf(out), torch.full_like(out, float("inf")), out)


def sdpa_bwd_ref(Q, K, V, dO, causal: bool = False, scale: float = -1.0):
    """(dQ, dK, dV), fp32 on the CPU: torch autograd of sdpa_ref's FP32 attention for the
    upstream gradient dO.  With fewer K/V heads than Q heads the K/V gradients are summed
    over the query heads that share them (autograd through expand_kv)."""
    sc = resolve_scale(Q.shape[-1], scale)
    H = Q.shape[1]
    q = Q.detach().cpu().float().requires_grad_()
    k = K.detach().cpu().float().requires_grad_()
    v = V.detach().cpu().float().requires_grad_()
    with torch.enable_grad():
        out = F.scaled_dot_product_attention(q, expand_kv(k, H), expand_kv(v, H),
                                             is_causal=causal, scale=sc)
        out.backward(dO.detach().cpu().float())
    return q.grad, k.grad, v.grad


def sdpa_varlen_bwd_ref(q, k, v, dO, cu_q, cu_k, causal: bool = False, scale: float = -1.0):
    """Gradients of sdpa_varlen_ref, per sequence (zero for rows of a sequence with no keys
    or no queries, and for rows outside every sequence)."""
    cu_q = [int(x) for x in cu_q]
    cu_k = [int(x) for x in cu_k]
    dq = torch.zeros(q.shape, dtype=torch.float32)
    dk = torch.zeros(k.shape, dtype=torch.float32)
    dv = torch.zeros(v.shape, dtype=torch.float32)
    for b in range(len(cu_q) - 1):
        qa, qe, ka, ke = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        if qe <= qa or ke <= ka:
            continue
        t = lambda X, a, e: X[a:e].transpose(0, 1).unsqueeze(0)
        gq, gk, gv = sdpa_bwd_ref(t(q, qa, qe), t(k, ka, ke), t(v, ka, ke), t(dO, qa, qe),
                                  causal, scale)
        dq[qa:qe] = gq[0].transpose(0, 1)
        dk[ka:ke] = gk[0].transpose(0, 1)
        dv[ka:ke] = gv[0].transpose(0, 1)
    return dq, dk, dv


def lse_varlen_ref(q, k, cu_q, cu_k, causal: bool = False, scale: float = -1.0) -> torch.Tensor:
    """lse_ref per sequence in the packed layout [H, total_q] (+inf for a sequence with no
    keys)."""
    cu_q = [int(x) for x in cu_q]
    cu_k = [int(x) for x in cu_k]
    out = torch.full((q.shape[1], q.shape[0]), float("inf"), dtype=torch.float32)
    for b in range(len(cu_q) - 1):
        qa, qe, ka, ke = cu_q[b], cu_q[b + 1], cu_k[b], cu_k[b + 1]
        if qe <= qa or ke <= ka:
            continue
        Q = q[qa:qe].transpose(0, 1).unsqueeze(0)
        K = k[ka:ke].transpose(0, 1).unsqueeze(0)
        out[:, qa:qe] = lse_ref(Q, K, causal, scale)[0]
    return out
