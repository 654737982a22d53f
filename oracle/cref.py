"""ctypes binding of the plain-C oracle (oracle/liboracle.so).  Test infrastructure only."""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# WMMA_ORACLE_LIBRARY: another build of the same sources (the host-sanitized one of
# `python -m wmma_ops_amd.build --sanitize`)
LIB = os.environ.get("WMMA_ORACLE_LIBRARY") or os.path.join(_HERE, "liboracle.so")
_lib = None


def build() -> str:
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return LIB


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB):
            build()
        _lib = ctypes.CDLL(LIB)
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def gemm(A16: np.ndarray, B16: np.ndarray, alpha=1.0, beta=0.0, C=None, split=1) -> np.ndarray:
    A = np.ascontiguousarray(A16, dtype=np.float16).view(np.uint16)
    B = np.ascontiguousarray(B16, dtype=np.float16).view(np.uint16)
    M, K = A.shape
    N = B.shape[1]
    out = np.empty((M, N), dtype=np.float32)
    Cin = None if C is None else np.ascontiguousarray(C, dtype=np.float32)
    lib().oracle_gemm(_p(A), _p(B), None if Cin is None else _p(Cin), _p(out), M, N, K,
                      ctypes.c_float(alpha), ctypes.c_float(beta), split)
    return out


def pack_gptq(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    K, N = q.shape
    out = np.empty((K // 8, N), dtype=np.int32)
    lib().oracle_int4_pack_gptq(_p(q), K, N, _p(out))
    return out


def prepack(qweight: np.ndarray) -> np.ndarray:
    qw = np.ascontiguousarray(qweight, dtype=np.int32)
    K, N = qw.shape[0] * 8, qw.shape[1]
    out = np.empty_like(qw)
    lib().oracle_int4_prepack(_p(qw), K, N, _p(out))
    return out


def dequant(q: np.ndarray, scales: np.ndarray, zeros_u8: np.ndarray, G: int) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.uint8)
    s = np.ascontiguousarray(scales, dtype=np.float16).view(np.uint16)
    z = np.ascontiguousarray(zeros_u8, dtype=np.uint8)
    K, N = q.shape
    out = np.empty((K, N), dtype=np.uint16)
    lib().oracle_int4_dequant(_p(q), _p(s), _p(z), K, N, G, _p(out))
    return out.view(np.float16)


def w4a16(A16: np.ndarray, W16: np.ndarray) -> np.ndarray:
    A = np.ascontiguousarray(A16, dtype=np.float16).view(np.uint16)
    W = np.ascontiguousarray(W16, dtype=np.float16).view(np.uint16)
    M, K = A.shape
    N = W.shape[1]
    out = np.empty((M, N), dtype=np.float32)
    lib().oracle_w4a16(_p(A), _p(W), M, N, K, _p(out))
    return out
