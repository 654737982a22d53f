"""GEMM oracle (CPU).  Test infrastructure only -- see oracle/__init__.py.

Restates the reference's FP16 x FP16 -> FP32 GEMM path:
  * product        C = A @ B with FP32 accumulation (wmma_gemm.hip:45-233; the reference's
                   tests compare against torch.matmul(A.float(), B.float()),
                   test_fragment_loading.py:93)
  * epilogue       r = alpha*acc; if (beta != 0 && C_in) r += beta*C_in
                   (wmma_gemm.hip:636-666, 1912-1924)
  * split-K        k_per_split = ceil(K / split); partial sums reduced in split order
                   (wmma_xor_swizzle.hpp:293-353)
  * metric         max|Y - Y_ref| / max|Y_ref| (test_fragment_loading.py:116-120)
"""
from __future__ import annotations

import numpy as np
import torch


def gemm_ref(A: torch.Tensor, B: torch.Tensor, alpha: float = 1.0, beta: float = 0.0,
             C: torch.Tensor | None = None) -> torch.Tensor:
    """alpha * (A @ B) + beta * C in fp32 on the CPU; C is read only if beta != 0."""
    Y = torch.matmul(A.detach().cpu().float(), B.detach().cpu().float())
    out = Y * np.float32(alpha) if alpha != 1.0 else Y
    if beta != 0.0 and C is not None:
        out = out + np.float32(beta) * C.detach().cpu().float()
    return out


def gemm_ref_f64(A: np.ndarray, B: np.ndarray, alpha: float = 1.0, beta: float = 0.0,
                 C: np.ndarray | None = None) -> np.ndarray:
    """Brute-force triple loop in float64 (tiny shapes only)."""
    A = np.asarray(A, dtype=np.float64)
    B = np.asarray(B, dtype=np.float64)
    M, K = A.shape
    N = B.shape[1]
    Y = np.zeros((M, N), dtype=np.float64)
    for i in range(M):
        for j in range(N):
            s = 0.0
            for k in range(K):
                s += A[i, k] * B[k, j]
            Y[i, j] = s
    out = alpha * Y
    if beta != 0.0 and C is not None:
        out = out + beta * np.asarray(C, dtype=np.float64)
    return out


def splitk_partition(K: int, split: int) -> list[tuple[int, int]]:
    """K ranges of a split-K GEMM: k_per_split = ceil(K / split) (wmma_xor_swizzle.hpp:327)."""
    kps = -(-K // split)
    return [(s * kps, min(K, (s + 1) * kps)) for s in range(split) if s * kps < K]


def splitk_gemm_ref(A: torch.Tensor, B: torch.Tensor, split: int) -> torch.Tensor:
    """Sum of per-range partial products in split order (wmma_xor_swizzle.hpp:334-353)."""
    A32 = A.detach().cpu().float()
    B32 = B.detach().cpu().float()
    out = torch.zeros(A32.shape[0], B32.shape[1], dtype=torch.float32)
    for k0, k1 in splitk_partition(A32.shape[1], split):
        out += A32[:, k0:k1] @ B32[k0:k1, :]
    return out


def kat_fragment(M: int = 64, N: int = 64, K: int = 16):
    """Known-answer test of test_fragment_loading.py:237-256: A[i][j] = i % 16, B[j][k] = j,
    so C[i][k] = (i % 16) * sum_j j = (i % 16) * K(K-1)/2 (= (i%16)*120 at K=16), exact in
    fp16 inputs and fp32 accumulation."""
    A = torch.tensor([[float(i % 16)] * K for i in range(M)], dtype=torch.float16)
    B = torch.tensor([[float(j)] * N for j in range(K)], dtype=torch.float16)
    s = K * (K - 1) // 2
    C = torch.tensor([[float((i % 16) * s)] * N for i in range(M)], dtype=torch.float32)
    return A, B, C


def max_rel_err(Y: torch.Tensor, Y_ref: torch.Tensor) -> float:
    """max|Y - Y_ref| / max|Y_ref| (test_fragment_loading.py:116-120); 0 if both are 0."""
    Y = Y.detach().cpu().float()
    Y_ref = Y_ref.detach().cpu().float()
    err = (Y - Y_ref).abs().max().item() if Y.numel() else 0.0
    ref = Y_ref.abs().max().item() if Y_ref.numel() else 0.0
    if ref == 0.0:
        return 0.0 if err == 0.0 else float("inf")
    return err / ref


def rel_l2_err(Y: torch.Tensor, Y_ref: torch.Tensor) -> float:
    """||Y - Y_ref||_2 / ||Y_ref||_2 (test_fragment_loading.py:123-125)."""
    Y = Y.detach().cpu().double()
    Y_ref = Y_ref.detach().cpu().double()
    den = torch.linalg.vector_norm(Y_ref).item()
    num = torch.linalg.vector_norm(Y - Y_ref).item()
    return num / den if den > 0 else (0.0 if num == 0 else float("inf"))
