"""wmma_ops for MI355X (gfx950): hand-written MFMA kernels behind the wmma_ops API.

Drop-in for the reference module ``wmma_ops`` (pybind functions at
wmma_gemm.hip:2120-2157)::

    import wmma_ops_amd as wmma_ops
    C = wmma_ops.matmul(A, B)                        # fp16 x fp16 -> fp32
    C = wmma_ops.gemm(A, B, alpha=2.0, beta=0.5, C=C0)
    wmma_ops.gemm_inplace(A, B, C, 2.0, 0.5)
    O = wmma_ops.flash_attention(Q, K, V, causal=True)   # differentiable (fused backward)
    P = wmma_ops.prepack_int4(qweight); Y = wmma_ops.matmul_int4(A, P, scales, zeros, 128)

Every function runs the HIP kernels in ``libwmma_ops_amd.so`` through the C++ extension
``_C``; there is no fallback path.  Importing fails loudly when the extension has not been
built (``python -m wmma_ops_amd.build``).
"""
from __future__ import annotations

import os as _os

_PKG = _os.path.dirname(_os.path.abspath(__file__))
LIBRARY_PATH = _os.path.join(_PKG, "libwmma_ops_amd.so")
HEADER_PATH = _os.path.join(_os.path.dirname(_PKG), "include", "wmma_ops_amd.h")

try:
    import torch as _torch  # noqa: F401  (loads libtorch/libc10 before the extension)
    from . import _C
except ImportError as _e:  # pragma: no cover - exercised only on an unbuilt tree
    raise ImportError(
        "wmma_ops_amd: the native extension is not built; run `python -m wmma_ops_amd.build` "
        f"(original error: {_e})"
    ) from _e

matmul = _C.matmul
matmul_adaptive = _C.matmul_adaptive
matmul_tiled = _C.matmul_tiled
gemm = _C.gemm
gemm_inplace = _C.gemm_inplace
gemm_adaptive = _C.gemm_adaptive
flash_attention_forward = _C.flash_attention_forward
flash_attention_backward = _C.flash_attention_backward
flash_attention_varlen_forward = _C.flash_attention_varlen_forward
flash_attention_varlen_backward = _C.flash_attention_varlen_backward


class FlashAttentionFunction(_torch.autograd.Function):
    """Autograd node of flash_attention: the forward keeps O and the log-sum-exp, the
    backward runs the fused dQ and dK/dV kernels."""

    @staticmethod
    def forward(ctx, Q, K, V, causal=False, scale=-1.0):
        O, lse = _C.flash_attention_forward(Q, K, V, causal, scale)
        ctx.save_for_backward(Q, K, V, O, lse)
        ctx.causal, ctx.scale = causal, scale
        return O

    @staticmethod
    def backward(ctx, dO):
        Q, K, V, O, lse = ctx.saved_tensors
        dQ, dK, dV = _C.flash_attention_backward(dO, Q, K, V, O, lse, ctx.causal, ctx.scale)
        return dQ, dK, dV, None, None


class FlashAttentionVarlenFunction(_torch.autograd.Function):
    """Autograd node of flash_attention_varlen."""

    @staticmethod
    def forward(ctx, q, k, v, cu_q, cu_k, max_q, max_k, causal=False, scale=-1.0):
        O, lse = _C.flash_attention_varlen_forward(q, k, v, cu_q, cu_k, max_q, max_k, causal, scale)
        ctx.save_for_backward(q, k, v, O, lse, cu_q, cu_k)
        ctx.args = (max_q, max_k, causal, scale)
        return O

    @staticmethod
    def backward(ctx, dO):
        q, k, v, O, lse, cu_q, cu_k = ctx.saved_tensors
        max_q, max_k, causal, scale = ctx.args
        dq, dk, dv = _C.flash_attention_varlen_backward(dO, q, k, v, O, lse, cu_q, cu_k, max_q,
                                                        max_k, causal, scale)
        return dq, dk, dv, None, None, None, None, None, None


def _needs_grad(*ts) -> bool:
    return _torch.is_grad_enabled() and any(t.requires_grad for t in ts)


def flash_attention(Q, K, V, causal: bool = False, scale: float = -1.0):
    """flash_attention(Q, K, V, causal=False, scale=-1.0) (the reference's README.md:221-251):
    fp16 [B,H,Sq,D] attention output, D up to 256.  Differentiable when an input requires
    grad (the reference's op is forward-only; inference calls take the plain forward
    kernel)."""
    if _needs_grad(Q, K, V):
        return FlashAttentionFunction.apply(Q, K, V, causal, scale)
    return _C.flash_attention(Q, K, V, causal, scale)


def flash_attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q, max_seqlen_k,
                           causal: bool = False, scale: float = -1.0):
    """Packed variable-length attention ([total, heads, D] with int32 cu_seqlens [B+1]);
    differentiable in q, k, v.

    max_seqlen_q / max_seqlen_k must be at least the longest sequence in cu_seqlens_q /
    cu_seqlens_k: each sequence is processed up to that many rows only, so rows of a longer
    sequence past it are never written (the output and, for training, the log-sum-exp keep
    whatever their allocation held there) and no error is raised.  Offsets outside the
    packed tensors are clamped, so inconsistent cu_seqlens give wrong rows, never an access
    outside the tensors."""
    if _needs_grad(q, k, v):
        return FlashAttentionVarlenFunction.apply(q, k, v, cu_seqlens_q, cu_seqlens_k,
                                                  max_seqlen_q, max_seqlen_k, causal, scale)
    return _C.flash_attention_varlen(q, k, v, cu_seqlens_q, cu_seqlens_k, max_seqlen_q,
                                     max_seqlen_k, causal, scale)

prepack_int4 = _C.prepack_int4
prepack_int4_params = _C.prepack_int4_params
int4_from_awq = _C.int4_from_awq
int4_from_gptq = _C.int4_from_gptq
unprepack_int4 = _C.unprepack_int4
unpack_int4 = _C.unpack_int4
matmul_int4 = _C.matmul_int4
prepack_int4_fused = _C.prepack_int4_fused
unprepack_int4_fused = _C.unprepack_int4_fused
matmul_int4_fused = _C.matmul_int4_fused
gemm_plan = _C.gemm_plan
w4a16_plan = _C.w4a16_plan

# The reference binds 13 more matmul_* names, each a gfx1151 tuning experiment computing
# the same C = A @ B (wmma_gemm.hip:2122-2137).  They resolve to the planner-driven MFMA
# GEMM here so code written against the reference keeps importing and running.
_REFERENCE_VARIANTS = (
    "matmul_hilbert", "matmul_kunroll", "matmul_native", "matmul_zerocopy", "matmul_quad",
    "matmul_highOcc", "matmul_noPrefetch", "matmul_asmOpt", "matmul_swizzled",
    "matmul_xor_optimized", "matmul_coop", "matmul_pingpong", "matmul_opt",
)
for _name in _REFERENCE_VARIANTS:
    globals()[_name] = _C.matmul

TILE_CONFIGS = {0: (64, 64), 1: (128, 64), 2: (256, 64), 3: (128, 128), 4: (256, 128), 5: (256, 256)}

__all__ = [
    "matmul", "matmul_adaptive", "matmul_tiled", "gemm", "gemm_inplace", "gemm_adaptive",
    "flash_attention", "flash_attention_varlen", "flash_attention_forward",
    "flash_attention_backward", "flash_attention_varlen_forward", "flash_attention_varlen_backward",
    "FlashAttentionFunction", "FlashAttentionVarlenFunction", "prepack_int4", "prepack_int4_params", "int4_from_awq", "int4_from_gptq", "unprepack_int4", "unpack_int4", "matmul_int4", "prepack_int4_fused", "unprepack_int4_fused", "matmul_int4_fused",
    "gemm_plan", "w4a16_plan", "TILE_CONFIGS", "LIBRARY_PATH", "HEADER_PATH", *_REFERENCE_VARIANTS,
]
