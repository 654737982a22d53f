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


def sdpa_ref(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor, causal: bool = False,
             scale: float = -1.0) -> torch.Tensor:
    """FP32 scaled-dot-product attention on the CPU (the library routine)."""
    sc = resolve_scale(Q.shape[-1], scale)
    return F.scaled_dot_product_attention(Q.detach().cpu().float(), K.detach().cpu().float(),
                                          V.detach().cpu().float(), is_causal=causal, scale=sc)


def attention_naive_f64(Q: np.ndarray, K: np.ndarray, V: np.ndarray, causal: bool = False,
                        scale: float = -1.0) -> np.ndarray:
    """Explicit float64 softmax(scale * Q K^T + mask) V, for tiny shapes."""
    Q = np.asarray(Q, dtype=np.float64)
    K = np.asarray(K, dtype=np.float64)
    V = np.asarray(V, dtype=np.float64)
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


def make_inputs(B: int, H: int, S: int, D: int, seed: int, Sk: int | None = None):
    """Seeded Q, K, V ~ N(0, 1) in fp16."""
    g = torch.Generator().manual_seed(seed)
    Sk = S if Sk is None else Sk
    Q = torch.randn(B, H, S, D, generator=g).half()
    K = torch.randn(B, H, Sk, D, generator=g).half()
    V = torch.randn(B, H, Sk, D, generator=g).half()
    return Q, K, V
