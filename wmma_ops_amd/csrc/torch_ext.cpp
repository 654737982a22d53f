// PyTorch-ROCm extension: the reference's Python API on top of the C-ABI.
//
// Mirrors the pybind module of the reference (wmma_gemm.hip:2120-2157): the same
// function names, argument meaning, defaults and TORCH_CHECK messages
// (wmma_gemm.hip:1197-1263, 1432-1528, 1891-2078).  Tensors are validated here, made
// contiguous, outputs come from the caching allocator, and the work is enqueued on the
// current HIP stream of A's device through the C-ABI in include/wmma_ops_amd.h.  Unlike
// the reference a device guard is taken, so the launch goes to the tensors' device.
//
// Additions the reference lacks: flash_attention (documented at README.md:221-251 but
// never bound) and its training entry points (forward with log-sum-exp, backward), the INT4
// entry points (prepack_int4, unpack_int4, unprepack_int4,
// matmul_int4), and the split-K workspace, which is taken from the caching allocator.
#include <torch/extension.h>

// ROCm torch reports HIP devices as DeviceType::CUDA; its guard and stream helpers for
// such devices are the "MasqueradingAsCUDA" variants.
#include <ATen/hip/impl/HIPGuardImplMasqueradingAsCUDA.h>
#include <ATen/hip/impl/HIPStreamMasqueradingAsCUDA.h>

#include <cmath>
#include <string>

#include "../../include/wmma_ops_amd.h"

namespace {

void check_status(int rc, const char* what) {
    TORCH_CHECK(rc == WMMA_OK, what, " failed (status ", rc, "): ", wmma_last_error());
}

void* current_stream(const torch::Tensor& t) {
    return static_cast<void*>(c10::hip::getCurrentHIPStreamMasqueradingAsCUDA(t.device().index()).stream());
}

// Shared checks of A and B (wmma_gemm.hip:1198-1212).
void check_ab(const torch::Tensor& A, const torch::Tensor& B, bool same_device_check) {
    TORCH_CHECK(A.is_cuda() && B.is_cuda(), "Inputs must be CUDA tensors");
    if (same_device_check) TORCH_CHECK(A.device() == B.device(), "Inputs must be on same device");
    TORCH_CHECK(A.dtype() == torch::kFloat16 && B.dtype() == torch::kFloat16,
                "Inputs must be float16");
    TORCH_CHECK(A.dim() == 2 && B.dim() == 2, "Inputs must be 2D");
    TORCH_CHECK(A.size(1) == B.size(0), "Inner dimensions must match");
}

void check_aligned(const torch::Tensor& t, const char* msg) {
    TORCH_CHECK((reinterpret_cast<uintptr_t>(t.data_ptr()) % 16) == 0, msg);
}

torch::Tensor workspace_for(size_t bytes, const torch::Tensor& like) {
    if (bytes == 0) return torch::Tensor();
    return torch::empty({(int64_t)bytes}, torch::dtype(torch::kUInt8).device(like.device()));
}

// One GEMM through the C-ABI.  C_in may be undefined; C_out preallocated.
void run_gemm(const torch::Tensor& A, const torch::Tensor& B, const torch::Tensor& C_in,
              torch::Tensor& C_out, double alpha, double beta, int tile_cfg) {
    const int M = (int)A.size(0), K = (int)A.size(1), N = (int)B.size(1);
    TORCH_CHECK(A.size(0) <= INT32_MAX && A.size(1) <= INT32_MAX && B.size(1) <= INT32_MAX,
                "dimensions exceed int32");
    const size_t ws_bytes = wmma_gemm_workspace_size(M, N, K, tile_cfg);
    torch::Tensor ws = workspace_for(ws_bytes, A);
    const float* cin = C_in.defined() ? C_in.data_ptr<float>() : nullptr;
    const int64_t ldcin = C_in.defined() ? C_in.stride(0) : N;
    int rc = wmma_gemm_f16f32(A.data_ptr(), A.stride(0), B.data_ptr(), B.stride(0), cin, ldcin,
                              C_out.data_ptr<float>(), C_out.stride(0), M, N, K,
                              static_cast<float>(alpha), static_cast<float>(beta), tile_cfg,
                              ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(A));
    check_status(rc, "wmma_gemm_f16f32");
}

// `vec_text`: the reference's matmul and matmul_tiled say "... aligned for vectorized loads"
// (wmma_gemm.hip:1443-1446, 1483-1486), its matmul_adaptive just "... aligned"
// (wmma_gemm.hip:1207-1210).
torch::Tensor matmul_impl(torch::Tensor A, torch::Tensor B, int tile_cfg, bool same_device,
                          bool vec_text) {
    check_ab(A, B, same_device);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(A.device());
    A = A.contiguous();
    B = B.contiguous();
    check_aligned(A, vec_text ? "A must be 16-byte aligned for vectorized loads"
                              : "A must be 16-byte aligned");
    check_aligned(B, vec_text ? "B must be 16-byte aligned for vectorized loads"
                              : "B must be 16-byte aligned");
    auto C = torch::empty({A.size(0), B.size(1)}, torch::dtype(torch::kFloat32).device(A.device()));
    run_gemm(A, B, torch::Tensor(), C, 1.0, 0.0, tile_cfg);
    return C;
}

// matmul (wmma_gemm.hip:1432-1470).  The tile is chosen by the planner.
torch::Tensor matmul(torch::Tensor A, torch::Tensor B) {
    return matmul_impl(A, B, WMMA_TILE_AUTO, true, true);
}

// matmul_adaptive (wmma_gemm.hip:1197-1263).
torch::Tensor matmul_adaptive(torch::Tensor A, torch::Tensor B) {
    return matmul_impl(A, B, WMMA_TILE_AUTO, true, false);
}

// matmul_tiled (wmma_gemm.hip:1473-1528): like the reference, no same-device check.
torch::Tensor matmul_tiled(torch::Tensor A, torch::Tensor B, int64_t tile_config) {
    TORCH_CHECK(A.is_cuda() && B.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(A.dtype() == torch::kFloat16 && B.dtype() == torch::kFloat16,
                "Inputs must be float16");
    TORCH_CHECK(A.dim() == 2 && B.dim() == 2, "Inputs must be 2D");
    TORCH_CHECK(A.size(1) == B.size(0), "Inner dimensions must match");
    TORCH_CHECK(tile_config >= 0 && tile_config < WMMA_TILE_COUNT,
                "Invalid tile_config: 0=64x64, 1=128x64, 2=256x64, 3=128x128, 4=256x128, "
                "5=256x256");
    return matmul_impl(A, B, (int)tile_config, false, true);
}

// gemm / gemm_adaptive (wmma_gemm.hip:1891-1945, 1997-2078): C is read only when
// beta != 0 and C is given; beta != 0 without C is silently ignored, as in the reference.
torch::Tensor gemm_impl(torch::Tensor A, torch::Tensor B, double alpha, double beta,
                        c10::optional<torch::Tensor> C_opt) {
    check_ab(A, B, true);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(A.device());
    A = A.contiguous();
    B = B.contiguous();
    check_aligned(A, "A must be 16-byte aligned");
    check_aligned(B, "B must be 16-byte aligned");
    const int64_t M = A.size(0), N = B.size(1);
    torch::Tensor C_in;
    if (beta != 0.0 && C_opt.has_value() && C_opt->defined()) {
        C_in = C_opt.value();
        TORCH_CHECK(C_in.is_cuda(), "C must be a CUDA tensor");
        TORCH_CHECK(C_in.device() == A.device(), "C must be on same device as A and B");
        TORCH_CHECK(C_in.dtype() == torch::kFloat32, "C must be float32");
        TORCH_CHECK(C_in.dim() == 2, "C must be 2D");
        TORCH_CHECK(C_in.size(0) == M && C_in.size(1) == N, "C dimensions must match output (M×N)");
        C_in = C_in.contiguous();
    }
    auto C_out = torch::empty({M, N}, torch::dtype(torch::kFloat32).device(A.device()));
    run_gemm(A, B, C_in, C_out, alpha, beta, WMMA_TILE_AUTO);
    return C_out;
}

torch::Tensor gemm(torch::Tensor A, torch::Tensor B, double alpha, double beta,
                   c10::optional<torch::Tensor> C) {
    return gemm_impl(A, B, alpha, beta, C);
}

torch::Tensor gemm_adaptive(torch::Tensor A, torch::Tensor B, double alpha, double beta,
                            c10::optional<torch::Tensor> C) {
    return gemm_impl(A, B, alpha, beta, C);
}

// gemm_inplace (wmma_gemm.hip:1949-1994).  The reference silently updates a contiguous
// copy when C is not contiguous (:1970); here a non-contiguous C is rejected instead, so
// the caller's tensor is always the one written.
void gemm_inplace(torch::Tensor A, torch::Tensor B, torch::Tensor C, double alpha, double beta) {
    TORCH_CHECK(A.is_cuda() && B.is_cuda() && C.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(A.device() == B.device() && A.device() == C.device(),
                "All tensors must be on same device");
    TORCH_CHECK(A.dtype() == torch::kFloat16 && B.dtype() == torch::kFloat16,
                "A and B must be float16");
    TORCH_CHECK(C.dtype() == torch::kFloat32, "C must be float32");
    TORCH_CHECK(A.dim() == 2 && B.dim() == 2 && C.dim() == 2, "Inputs must be 2D");
    TORCH_CHECK(A.size(1) == B.size(0), "Inner dimensions must match");
    TORCH_CHECK(C.size(0) == A.size(0) && C.size(1) == B.size(1),
                "C dimensions must match output (M×N)");
    TORCH_CHECK(C.is_contiguous(), "C must be contiguous for in-place update");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(A.device());
    A = A.contiguous();
    B = B.contiguous();
    check_aligned(A, "A must be 16-byte aligned");
    check_aligned(B, "B must be 16-byte aligned");
    run_gemm(A, B, C, C, alpha, beta, WMMA_TILE_AUTO);
}

// Checks of the dense attention inputs Q [B,H,Sq,D], K/V [B,Hkv,Sk,D] (flash_attention and
// its training entry points).
void check_flash_dense(const torch::Tensor& Q, const torch::Tensor& K, const torch::Tensor& V) {
    TORCH_CHECK(Q.is_cuda() && K.is_cuda() && V.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(Q.device() == K.device() && Q.device() == V.device(),
                "Inputs must be on same device");
    TORCH_CHECK(Q.dtype() == torch::kFloat16 && K.dtype() == torch::kFloat16 &&
                    V.dtype() == torch::kFloat16,
                "Inputs must be float16");
    TORCH_CHECK(Q.dim() == 4 && K.dim() == 4 && V.dim() == 4, "Inputs must be 4D [B, H, N, D]");
    TORCH_CHECK(K.sizes() == V.sizes(), "K and V must have the same shape");
    TORCH_CHECK(Q.size(0) == K.size(0) && Q.size(3) == K.size(3),
                "Q and K must agree in batch and head_dim");
    TORCH_CHECK(K.size(1) > 0 && Q.size(1) % K.size(1) == 0,
                "K/V heads must divide Q heads");
    TORCH_CHECK(Q.size(3) >= 1 && Q.size(3) <= 256, "head_dim must be between 1 and 256");
}

// Checks of the packed inputs q [total_q,H,D], k/v [total_k,Hkv,D], cu_seqlens int32 [B+1].
void check_flash_varlen(const torch::Tensor& q, const torch::Tensor& k, const torch::Tensor& v,
                        const torch::Tensor& cu_q, const torch::Tensor& cu_k) {
    TORCH_CHECK(q.is_cuda() && k.is_cuda() && v.is_cuda() && cu_q.is_cuda() && cu_k.is_cuda(),
                "Inputs must be CUDA tensors");
    TORCH_CHECK(q.device() == k.device() && q.device() == v.device() && q.device() == cu_q.device() &&
                    q.device() == cu_k.device(),
                "Inputs must be on same device");
    TORCH_CHECK(q.dtype() == torch::kFloat16 && k.dtype() == torch::kFloat16 &&
                    v.dtype() == torch::kFloat16,
                "Inputs must be float16");
    TORCH_CHECK(q.dim() == 3 && k.dim() == 3 && v.dim() == 3, "Inputs must be 3D [total, heads, D]");
    TORCH_CHECK(k.sizes() == v.sizes(), "K and V must have the same shape");
    TORCH_CHECK(q.size(2) == k.size(2), "Q and K must agree in head_dim");
    TORCH_CHECK(k.size(1) > 0 && q.size(1) % k.size(1) == 0, "K/V heads must divide Q heads");
    TORCH_CHECK(cu_q.dtype() == torch::kInt32 && cu_k.dtype() == torch::kInt32 && cu_q.dim() == 1 &&
                    cu_q.sizes() == cu_k.sizes() && cu_q.size(0) >= 1,
                "cu_seqlens must be int32 [B+1], equal for Q and K");
    TORCH_CHECK(q.size(2) >= 1 && q.size(2) <= 256, "head_dim must be between 1 and 256");
}

// Gradient-side checks: dO and O have Q's shape (fp16, same device), lse is fp32 of the
// given shape.
void check_flash_grad_inputs(const torch::Tensor& Q, const torch::Tensor& dO, const torch::Tensor& O,
                             const torch::Tensor& lse, at::IntArrayRef lse_shape) {
    TORCH_CHECK(dO.is_cuda() && O.is_cuda() && lse.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(dO.device() == Q.device() && O.device() == Q.device() && lse.device() == Q.device(),
                "Inputs must be on same device");
    TORCH_CHECK(dO.dtype() == torch::kFloat16 && O.dtype() == torch::kFloat16,
                "dO and O must be float16");
    TORCH_CHECK(dO.sizes() == Q.sizes() && O.sizes() == Q.sizes(), "dO and O must have Q's shape");
    TORCH_CHECK(lse.dtype() == torch::kFloat32 && lse.sizes() == lse_shape,
                "lse must be float32 ", lse_shape);
}

// The kernels take head dims that are multiples of 8 (16-byte rows).  Other head dims run on
// contiguous copies zero-padded to the next multiple of 8: the zero columns add nothing to
// the scores, give zero output and gradient columns, and are dropped from the results.
int64_t padded_head_dim(int64_t D) { return (D + 7) / 8 * 8; }

torch::Tensor pad_head(const torch::Tensor& t, int64_t Dp) {
    const int64_t D = t.size(-1);
    return D == Dp ? t.contiguous() : torch::constant_pad_nd(t, {0, Dp - D}).contiguous();
}

torch::Tensor unpad_head(const torch::Tensor& t, int64_t D) {
    return t.size(-1) == D ? t : t.narrow(-1, 0, D).contiguous();
}

float flash_scale(double scale, int64_t D) {
    return scale > 0.0 ? (float)scale : (float)(1.0 / std::sqrt((double)D));
}

// Runs the dense forward; lse_out (fp32 [B,H,Sq]) may be undefined (no log-sum-exp).
torch::Tensor flash_dense_fwd(torch::Tensor Q, torch::Tensor K, torch::Tensor V, bool causal,
                              double scale, torch::Tensor* lse_out) {
    check_flash_dense(Q, K, V);
    const int64_t D = Q.size(3), Dp = padded_head_dim(D);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(Q.device());
    Q = pad_head(Q, Dp);
    K = pad_head(K, Dp);
    V = pad_head(V, Dp);
    auto O = torch::empty_like(Q);
    float* lse = nullptr;
    if (lse_out) {
        *lse_out = torch::empty({Q.size(0), Q.size(1), Q.size(2)}, Q.options().dtype(torch::kFloat32));
        lse = lse_out->data_ptr<float>();
    }
    // decoding shapes split the key range; the partial sums come from the caching allocator
    const size_t ws_bytes = wmma_flash_attn_fwd_workspace_size(
        (int)Q.size(0), (int)Q.size(1), (int)K.size(1), (int)Q.size(2), (int)K.size(2), (int)Dp,
        causal ? 1 : 0);
    torch::Tensor ws = workspace_for(ws_bytes, Q);
    int rc = wmma_flash_attn_fwd_ws(Q.data_ptr(), K.data_ptr(), V.data_ptr(), O.data_ptr(), lse,
                                    (int)Q.size(0), (int)Q.size(1), (int)K.size(1),
                                    (int)Q.size(2), (int)K.size(2), (int)Dp, flash_scale(scale, D),
                                    causal ? 1 : 0, ws.defined() ? ws.data_ptr() : nullptr,
                                    ws_bytes, current_stream(Q));
    check_status(rc, "wmma_flash_attn_fwd_ws");
    return unpad_head(O, D);
}

// flash_attention(Q, K, V, causal=False, scale=-1.0) (README.md:221-251): Q [B,H,Sq,D],
// K/V [B,Hkv,Sk,D] fp16 with Hkv dividing H (Hkv < H: grouped-query attention, query head h
// reads key/value head h / (H/Hkv)); D from 1 to 256; scale <= 0 selects 1/sqrt(D).
// Returns fp16 [B,H,Sq,D].
torch::Tensor flash_attention(torch::Tensor Q, torch::Tensor K, torch::Tensor V, bool causal,
                              double scale) {
    return flash_dense_fwd(Q, K, V, causal, scale, nullptr);
}

// flash_attention_forward(Q, K, V, causal=False, scale=-1.0) -> (O, lse): the forward for
// training, with lse fp32 [B,H,Sq] (natural-log log-sum-exp of each scaled score row).
std::tuple<torch::Tensor, torch::Tensor> flash_attention_forward(torch::Tensor Q, torch::Tensor K,
                                                                 torch::Tensor V, bool causal,
                                                                 double scale) {
    torch::Tensor lse;
    auto O = flash_dense_fwd(Q, K, V, causal, scale, &lse);
    return {O, lse};
}

// flash_attention_backward(dO, Q, K, V, O, lse, causal=False, scale=-1.0) -> (dQ, dK, dV),
// fp16 with the shapes of Q, K, V; O and lse from flash_attention_forward with the same
// causal flag and scale.
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> flash_attention_backward(
    torch::Tensor dO, torch::Tensor Q, torch::Tensor K, torch::Tensor V, torch::Tensor O,
    torch::Tensor lse, bool causal, double scale) {
    check_flash_dense(Q, K, V);
    check_flash_grad_inputs(Q, dO, O, lse, {Q.size(0), Q.size(1), Q.size(2)});
    const int64_t B = Q.size(0), H = Q.size(1), Sq = Q.size(2), D = Q.size(3);
    const int64_t Dp = padded_head_dim(D);
    TORCH_CHECK(Sq == 0 || K.size(2) > 0, "K must have keys when Q has queries");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(Q.device());
    Q = pad_head(Q, Dp);
    K = pad_head(K, Dp);
    V = pad_head(V, Dp);
    O = pad_head(O, Dp);
    dO = pad_head(dO, Dp);
    lse = lse.contiguous();
    auto dQ = torch::empty_like(Q);
    auto dK = torch::empty_like(K);
    auto dV = torch::empty_like(V);
    // row statistics, plus the grouped-query split's partial dK/dV where it applies
    const size_t ws_bytes = wmma_flash_attn_bwd_split_workspace_size(
        (int)B, (int)H, (int)K.size(1), (int)Sq, (int)K.size(2), (int)Dp, causal ? 1 : 0);
    auto ws = torch::empty({(int64_t)((ws_bytes + 3) / 4)}, Q.options().dtype(torch::kFloat32));
    int rc = wmma_flash_attn_bwd(dO.data_ptr(), Q.data_ptr(), K.data_ptr(), V.data_ptr(),
                                 O.data_ptr(), lse.data_ptr<float>(), dQ.data_ptr(), dK.data_ptr(),
                                 dV.data_ptr(), ws.data_ptr(), ws_bytes, (int)B, (int)H,
                                 (int)K.size(1), (int)Sq, (int)K.size(2), (int)Dp,
                                 flash_scale(scale, D), causal ? 1 : 0, current_stream(Q));
    check_status(rc, "wmma_flash_attn_bwd");
    return {unpad_head(dQ, D), unpad_head(dK, D), unpad_head(dV, D)};
}

torch::Tensor flash_varlen_fwd(torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor cu_q,
                               torch::Tensor cu_k, int64_t max_q, int64_t max_k, bool causal,
                               double scale, torch::Tensor* lse_out) {
    check_flash_varlen(q, k, v, cu_q, cu_k);
    const int64_t D = q.size(2), Dp = padded_head_dim(D);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    q = pad_head(q, Dp);
    k = pad_head(k, Dp);
    v = pad_head(v, Dp);
    cu_q = cu_q.contiguous();
    cu_k = cu_k.contiguous();
    auto O = torch::empty_like(q);
    float* lse = nullptr;
    if (lse_out) {
        *lse_out = torch::empty({q.size(1), q.size(0)}, q.options().dtype(torch::kFloat32));
        lse = lse_out->data_ptr<float>();
    }
    int rc = wmma_flash_attn_varlen_fwd_lse(
        q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(), lse, cu_q.data_ptr<int32_t>(),
        cu_k.data_ptr<int32_t>(), (int)(cu_q.size(0) - 1), (int)q.size(1), (int)k.size(1),
        (int)q.size(0), (int)k.size(0), (int)max_q, (int)max_k, (int)Dp, flash_scale(scale, D),
        causal ? 1 : 0, current_stream(q));
    check_status(rc, "wmma_flash_attn_varlen_fwd_lse");
    return unpad_head(O, D);
}

// flash_attention_varlen(q [total_q, H, D], k/v [total_k, Hkv, D], cu_seqlens_q/k int32
// [B+1], max_seqlen_q, max_seqlen_k, causal=False, scale=-1.0) -> fp16 [total_q, H, D]
torch::Tensor flash_attention_varlen(torch::Tensor q, torch::Tensor k, torch::Tensor v,
                                     torch::Tensor cu_q, torch::Tensor cu_k, int64_t max_q,
                                     int64_t max_k, bool causal, double scale) {
    return flash_varlen_fwd(q, k, v, cu_q, cu_k, max_q, max_k, causal, scale, nullptr);
}

// flash_attention_varlen_forward(...) -> (O, lse fp32 [H, total_q])
std::tuple<torch::Tensor, torch::Tensor> flash_attention_varlen_forward(
    torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor cu_q, torch::Tensor cu_k,
    int64_t max_q, int64_t max_k, bool causal, double scale) {
    torch::Tensor lse;
    auto O = flash_varlen_fwd(q, k, v, cu_q, cu_k, max_q, max_k, causal, scale, &lse);
    return {O, lse};
}

// flash_attention_varlen_backward(dO, q, k, v, O, lse, cu_seqlens_q, cu_seqlens_k,
// max_seqlen_q, max_seqlen_k, causal=False, scale=-1.0) -> (dq, dk, dv)
std::tuple<torch::Tensor, torch::Tensor, torch::Tensor> flash_attention_varlen_backward(
    torch::Tensor dO, torch::Tensor q, torch::Tensor k, torch::Tensor v, torch::Tensor O,
    torch::Tensor lse, torch::Tensor cu_q, torch::Tensor cu_k, int64_t max_q, int64_t max_k,
    bool causal, double scale) {
    check_flash_varlen(q, k, v, cu_q, cu_k);
    check_flash_grad_inputs(q, dO, O, lse, {q.size(1), q.size(0)});
    const int64_t H = q.size(1), D = q.size(2), Dp = padded_head_dim(D);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(q.device());
    q = pad_head(q, Dp);
    k = pad_head(k, Dp);
    v = pad_head(v, Dp);
    O = pad_head(O, Dp);
    dO = pad_head(dO, Dp);
    lse = lse.contiguous();
    cu_q = cu_q.contiguous();
    cu_k = cu_k.contiguous();
    auto dq = torch::empty_like(q);
    auto dk = torch::empty_like(k);
    auto dv = torch::empty_like(v);
    // rows outside every sequence are not written by the kernels: start from zeros
    if (q.numel()) dq.zero_();
    if (k.numel()) {
        dk.zero_();
        dv.zero_();
    }
    const size_t ws_bytes = wmma_flash_attn_bwd_workspace_size(1, (int)H, (int)q.size(0));
    auto ws = torch::empty({(int64_t)(ws_bytes / 4)}, q.options().dtype(torch::kFloat32));
    int rc = wmma_flash_attn_varlen_bwd(
        dO.data_ptr(), q.data_ptr(), k.data_ptr(), v.data_ptr(), O.data_ptr(),
        lse.data_ptr<float>(), dq.data_ptr(), dk.data_ptr(), dv.data_ptr(),
        cu_q.data_ptr<int32_t>(), cu_k.data_ptr<int32_t>(), ws.data_ptr(), ws_bytes,
        (int)(cu_q.size(0) - 1), (int)H, (int)k.size(1), (int)q.size(0), (int)k.size(0),
        (int)max_q, (int)max_k, (int)Dp, flash_scale(scale, D), causal ? 1 : 0, current_stream(q));
    check_status(rc, "wmma_flash_attn_varlen_bwd");
    return {unpad_head(dq, D), unpad_head(dk, D), unpad_head(dv, D)};
}

void check_qweight(const torch::Tensor& q) {
    TORCH_CHECK(q.is_cuda(), "qweight must be a CUDA tensor");
    TORCH_CHECK(q.dtype() == torch::kInt32, "qweight must be int32");
    TORCH_CHECK(q.dim() == 2, "qweight must be 2D [K/8, N]");
}

// The prepacked weights are int32 [N/16, K/64, 32, 4] (include/wmma_ops_amd.h): a shape of
// their own, so a GPTQ qweight [K/8, N] passed where prepacked weights belong is rejected
// instead of being read as garbage.
void check_packed(const torch::Tensor& pk) {
    TORCH_CHECK(pk.is_cuda(), "packed must be a CUDA tensor");
    TORCH_CHECK(pk.dtype() == torch::kInt32 && pk.dim() == 4 && pk.size(2) == 32 &&
                    pk.size(3) == 4,
                "packed must be the int32 [N/16, K/64, 32, 4] output of prepack_int4 (a GPTQ "
                "qweight [K/8, N] must go through prepack_int4 first)");
}

// prepack_int4(qweight[K/8, N] int32, GPTQ order) -> prepacked int32 [N/16, K/64, 32, 4].
torch::Tensor prepack_int4(torch::Tensor qweight) {
    check_qweight(qweight);
    const int64_t K = qweight.size(0) * 8, N = qweight.size(1);
    TORCH_CHECK(K > 0 && N > 0, "K and N must be positive");
    TORCH_CHECK(K % 64 == 0, "K (", K, ") must be a multiple of 64");
    TORCH_CHECK(N % 32 == 0, "N (", N, ") must be a multiple of 32");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(qweight.device());
    qweight = qweight.contiguous();
    auto out = torch::empty({N / 16, K / 64, 32, 4}, qweight.options());
    check_status(wmma_int4_prepack(qweight.data_ptr<int32_t>(), (int)K, (int)N,
                                   out.data_ptr<int32_t>(), current_stream(qweight)),
                 "wmma_int4_prepack");
    return out;
}

// unprepack_int4(packed [N/16, K/64, 32, 4]) -> GPTQ qweight int32 [K/8, N].
torch::Tensor unprepack_int4(torch::Tensor packed) {
    check_packed(packed);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(packed.device());
    packed = packed.contiguous();
    const int64_t K = packed.size(1) * 64, N = packed.size(0) * 16;
    auto out = torch::empty({K / 8, N}, packed.options());
    check_status(wmma_int4_unprepack(packed.data_ptr<int32_t>(), (int)K, (int)N,
                                     out.data_ptr<int32_t>(), current_stream(packed)),
                 "wmma_int4_unprepack");
    return out;
}

// unpack_int4(qweight[K/8, N]) -> uint8 [K, N] of values 0..15.
torch::Tensor unpack_int4(torch::Tensor qweight) {
    check_qweight(qweight);
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(qweight.device());
    qweight = qweight.contiguous();
    const int K = (int)qweight.size(0) * 8, N = (int)qweight.size(1);
    auto out = torch::empty({K, N}, torch::dtype(torch::kUInt8).device(qweight.device()));
    check_status(wmma_int4_unpack(qweight.data_ptr<int32_t>(), K, N, out.data_ptr<uint8_t>(),
                                  current_stream(qweight)),
                 "wmma_int4_unpack");
    return out;
}

// int4_from_awq(qweight [K, N/8] int32, qzeros [K/G, N/8] int32) -- AutoAWQ checkpoint
// tensors -> (qweight [K/8, N] GPTQ layout, zeros [K/G, N/8] packed), bit-exact.
std::vector<torch::Tensor> int4_from_awq(torch::Tensor qweight, torch::Tensor qzeros) {
    TORCH_CHECK(qweight.is_cuda() && qzeros.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(qweight.device() == qzeros.device(), "Inputs must be on same device");
    TORCH_CHECK(qweight.dtype() == torch::kInt32 && qweight.dim() == 2,
                "AWQ qweight must be int32 [K, N/8]");
    TORCH_CHECK(qzeros.dtype() == torch::kInt32 && qzeros.dim() == 2 &&
                    qzeros.size(1) == qweight.size(1),
                "AWQ qzeros must be int32 [K/group_size, N/8]");
    const int64_t K = qweight.size(0), N = qweight.size(1) * 8, ng = qzeros.size(0);
    TORCH_CHECK(ng > 0 && K % ng == 0 && K % 8 == 0, "qzeros rows must divide K (a multiple of 8)");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(qweight.device());
    qweight = qweight.contiguous();
    qzeros = qzeros.contiguous();
    auto qo = torch::empty({K / 8, N}, qweight.options());
    auto zo = torch::empty({ng, N / 8}, qweight.options());
    int rc = wmma_int4_from_awq(qweight.data_ptr<int32_t>(), qzeros.data_ptr<int32_t>(), (int)K,
                                (int)N, (int)(K / ng), qo.data_ptr<int32_t>(),
                                zo.data_ptr<int32_t>(), current_stream(qweight));
    check_status(rc, "wmma_int4_from_awq");
    return {qo, zo};
}

// int4_from_gptq(qweight [K/8, N] int32, qzeros [K/G, N/8] int32, g_idx=None,
//                zero_format="v1") -> (qweight [K/8, N], zeros [K/G, N/8], perm or None).
// GPTQ checkpoints keep qweight and scales in this library's layout; the zero points need
// +1 per nibble in AutoGPTQ's v1 format ("v2": as stored).  g_idx (int32 [K], row -> group)
// equal to k / G, or None, is the plain layout (perm None).  Any other g_idx (act-order /
// desc_act) must give every group exactly G rows: the rows are then sorted by group (a
// stable sort) and perm (int64 [K]) is returned; pass it to matmul_int4 (perm=...), which
// multiplies A[:, perm].  One-time conversion: it synchronises to check the v1 zero range
// and the g_idx group sizes.
std::vector<c10::optional<torch::Tensor>> int4_from_gptq(torch::Tensor qweight, torch::Tensor qzeros,
                                                         c10::optional<torch::Tensor> g_idx,
                                                         const std::string& zero_format) {
    TORCH_CHECK(qweight.is_cuda() && qzeros.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(qweight.device() == qzeros.device(), "Inputs must be on same device");
    check_qweight(qweight);
    TORCH_CHECK(qzeros.dtype() == torch::kInt32 && qzeros.dim() == 2 &&
                    qzeros.size(1) * 8 == qweight.size(1),
                "GPTQ qzeros must be int32 [K/group_size, N/8]");
    TORCH_CHECK(zero_format == "v1" || zero_format == "v2", "zero_format must be \"v1\" or \"v2\"");
    const int64_t K = qweight.size(0) * 8, N = qweight.size(1), ng = qzeros.size(0);
    TORCH_CHECK(ng > 0 && K % ng == 0, "qzeros rows must divide K");
    const int64_t G = K / ng;
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(qweight.device());
    qweight = qweight.contiguous();
    qzeros = qzeros.contiguous();
    auto zo = torch::empty_like(qzeros);
    auto overflow = torch::zeros({1}, qzeros.options());
    int rc = wmma_int4_from_gptq_zeros(qzeros.data_ptr<int32_t>(), (int)K, (int)N, (int)G,
                                       zero_format == "v1" ? WMMA_GPTQ_V1 : WMMA_GPTQ_V2,
                                       zo.data_ptr<int32_t>(), overflow.data_ptr<int32_t>(),
                                       current_stream(qweight));
    check_status(rc, "wmma_int4_from_gptq_zeros");
    TORCH_CHECK(overflow.item<int32_t>() == 0,
                "GPTQ v1 qzeros hold a stored nibble 15 (zero point 16), which a 4-bit zero "
                "point cannot represent");
    c10::optional<torch::Tensor> perm;
    torch::Tensor qo = qweight;
    if (g_idx.has_value() && g_idx->defined()) {
        torch::Tensor gi = *g_idx;
        TORCH_CHECK(gi.device() == qweight.device(), "g_idx must be on the device of qweight");
        TORCH_CHECK(gi.dim() == 1 && gi.size(0) == K &&
                        (gi.dtype() == torch::kInt32 || gi.dtype() == torch::kInt64),
                    "g_idx must be an int32 or int64 vector of K entries");
        gi = gi.to(torch::kInt64);
        auto plain = torch::arange(K, gi.options()).floor_divide(G);
        if (!torch::equal(gi, plain)) {
            TORCH_CHECK(gi.min().item<int64_t>() >= 0 && gi.max().item<int64_t>() < ng,
                        "g_idx entries must lie in [0, K/group_size)");
            TORCH_CHECK(torch::equal(torch::bincount(gi, {}, ng), torch::full({ng}, G, gi.options())),
                        "act-order g_idx must assign exactly group_size rows to every group");
            auto p = std::get<1>(torch::sort(gi, c10::optional<bool>(true), /*dim=*/0, /*descending=*/false));
            auto p32 = p.to(torch::kInt32);
            qo = torch::empty_like(qweight);
            rc = wmma_int4_permute_rows(qweight.data_ptr<int32_t>(), p32.data_ptr<int32_t>(), (int)K,
                                        (int)N, qo.data_ptr<int32_t>(), current_stream(qweight));
            check_status(rc, "wmma_int4_permute_rows");
            perm = p;
        }
    }
    return {qo, zo, perm};
}

// prepack_int4_params(scales[K/G, N] fp16, zeros[K/G, N/8] int32 or [K/G, N] uint8)
//   -> (scales [N/16, K/G, 16] fp16, zeros [N/16, K/G, 2] int32): the slice-major layout
//   matmul_int4 also accepts (a 16-column slice's parameters contiguous).
std::vector<torch::Tensor> prepack_int4_params(torch::Tensor scales, torch::Tensor zeros) {
    TORCH_CHECK(scales.is_cuda() && zeros.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(scales.device() == zeros.device(), "Inputs must be on same device");
    TORCH_CHECK(scales.dtype() == torch::kFloat16 && scales.dim() == 2,
                "scales must be float16 [K/group_size, N]");
    const int64_t ng = scales.size(0), N = scales.size(1);
    TORCH_CHECK(N % 32 == 0 && ng > 0, "N must be a multiple of 32");
    int zfmt;
    if (zeros.dtype() == torch::kInt32) {
        TORCH_CHECK(zeros.dim() == 2 && zeros.size(0) == ng && zeros.size(1) * 8 == N,
                    "packed zeros must be int32 [K/group_size, N/8]");
        zfmt = WMMA_ZEROS_PACKED;
    } else {
        TORCH_CHECK(zeros.dtype() == torch::kUInt8 && zeros.dim() == 2 && zeros.size(0) == ng &&
                        zeros.size(1) == N,
                    "zeros must be int32 [K/group_size, N/8] or uint8 [K/group_size, N]");
        zfmt = WMMA_ZEROS_U8;
    }
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(scales.device());
    scales = scales.contiguous();
    zeros = zeros.contiguous();
    auto so = torch::empty({N / 16, ng, 16}, scales.options());
    auto zo = torch::empty({N / 16, ng, 2}, torch::dtype(torch::kInt32).device(scales.device()));
    // K and group_size only enter through K / group_size = ng: pass K = 64 ng, G = 64.
    int rc = wmma_int4_prepack_params(scales.data_ptr(), zeros.data_ptr(), zfmt, (int)(64 * ng),
                                      (int)N, 64, so.data_ptr(), zo.data_ptr<int32_t>(),
                                      current_stream(scales));
    check_status(rc, "wmma_int4_prepack_params");
    return {so, zo};
}

// prepack_int4_fused(qweight [K/8, N] int32, scales [K/G, N] fp16, zeros [K/G, N/8] int32
//   or [K/G, N] uint8, group_size=128) -> fused decode layout int32 [N/16, S/4] (S: bytes
//   per 16-column slice; include/wmma_ops_amd.h, WMMA_W4_FUSED), read by matmul_int4_fused.
torch::Tensor prepack_int4_fused(torch::Tensor qweight, torch::Tensor scales, torch::Tensor zeros,
                                 int64_t group_size) {
    check_qweight(qweight);
    TORCH_CHECK(scales.is_cuda() && zeros.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(qweight.device() == scales.device() && qweight.device() == zeros.device(),
                "Inputs must be on same device");
    const int64_t K = qweight.size(0) * 8, N = qweight.size(1);
    TORCH_CHECK(K > 0 && N > 0 && K % 128 == 0 && N % 32 == 0,
                "the fused layout needs K % 128 == 0 and N % 32 == 0");
    TORCH_CHECK(group_size > 0 && K % group_size == 0, "group_size must divide K");
    const int64_t ng = K / group_size;
    TORCH_CHECK(scales.dtype() == torch::kFloat16 && scales.dim() == 2 && scales.size(0) == ng &&
                    scales.size(1) == N,
                "scales must be float16 [K/group_size, N]");
    int zfmt;
    if (zeros.dtype() == torch::kInt32) {
        TORCH_CHECK(zeros.dim() == 2 && zeros.size(0) == ng && zeros.size(1) * 8 == N,
                    "packed zeros must be int32 [K/group_size, N/8]");
        zfmt = WMMA_ZEROS_PACKED;
    } else {
        TORCH_CHECK(zeros.dtype() == torch::kUInt8 && zeros.dim() == 2 && zeros.size(0) == ng &&
                        zeros.size(1) == N,
                    "zeros must be int32 [K/group_size, N/8] or uint8 [K/group_size, N]");
        zfmt = WMMA_ZEROS_U8;
    }
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(qweight.device());
    qweight = qweight.contiguous();
    scales = scales.contiguous();
    zeros = zeros.contiguous();
    const int64_t bytes = (int64_t)wmma_int4_fused_bytes((int)K, (int)N);
    auto out = torch::empty({N / 16, bytes / (N / 16) / 4}, qweight.options());
    check_status(wmma_int4_prepack_fused(qweight.data_ptr<int32_t>(), scales.data_ptr(),
                                         zeros.data_ptr(), zfmt, (int)K, (int)N, (int)group_size,
                                         out.data_ptr<int32_t>(), current_stream(qweight)),
                 "wmma_int4_prepack_fused");
    return out;
}

// K of a fused buffer from its words per slice (a header of 40 words per four 128-deep K
// steps, padded to 32-word lines, then 256 words per K step), or -1 when no K gives that size.
int64_t fused_k(int64_t words) {
    const int64_t bytes = words * 4;
    for (int64_t kp = bytes / 1024; kp >= 1 && kp * 1024 * 5 >= bytes * 4; --kp) {
        const int64_t hdr = (160 * ((kp + 3) / 4) + 127) / 128 * 128;
        if (hdr + kp * 1024 == bytes) return kp * 128;
    }
    return -1;
}

void check_fused(const torch::Tensor& f) {
    TORCH_CHECK(f.is_cuda(), "fused must be a CUDA tensor");
    TORCH_CHECK(f.dtype() == torch::kInt32 && f.dim() == 2 && fused_k(f.size(1)) > 0,
                "fused must be the int32 [N/16, words per slice] output of prepack_int4_fused");
}

// unprepack_int4_fused(fused [N/16, S/4], group_size=128) -> (qweight [K/8, N] int32,
//   scales [K/G, N] fp16, zeros [K/G, N/8] int32 packed).
std::vector<torch::Tensor> unprepack_int4_fused(torch::Tensor fused, int64_t group_size) {
    check_fused(fused);
    const int64_t K = fused_k(fused.size(1)), N = fused.size(0) * 16;
    TORCH_CHECK(group_size > 0 && K % group_size == 0, "group_size must divide K");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(fused.device());
    fused = fused.contiguous();
    auto qw = torch::empty({K / 8, N}, fused.options());
    auto sc = torch::empty({K / group_size, N}, torch::dtype(torch::kFloat16).device(fused.device()));
    auto zo = torch::empty({K / group_size, N / 8}, fused.options());
    check_status(wmma_int4_unprepack_fused(fused.data_ptr<int32_t>(), (int)K, (int)N,
                                           (int)group_size, qw.data_ptr<int32_t>(), sc.data_ptr(),
                                           zo.data_ptr<int32_t>(), current_stream(fused)),
                 "wmma_int4_unprepack_fused");
    return {qw, sc, zo};
}

// matmul_int4_fused(A [M,K] fp16, fused (from prepack_int4_fused), group_size=128,
//   out_dtype=None, perm=None) -> [M, N]: the W4A16 product for decode shapes (M <= 4)
//   with the weights and group parameters read from the fused layout.
torch::Tensor matmul_int4_fused(torch::Tensor A, torch::Tensor fused, int64_t group_size,
                                c10::optional<at::ScalarType> out_dtype,
                                c10::optional<torch::Tensor> perm) {
    const bool half_out = out_dtype.has_value() && *out_dtype == torch::kFloat16;
    TORCH_CHECK(!out_dtype.has_value() || *out_dtype == torch::kFloat16 ||
                    *out_dtype == torch::kFloat32,
                "out_dtype must be float32 or float16");
    TORCH_CHECK(A.is_cuda() && fused.is_cuda(), "Inputs must be CUDA tensors");
    TORCH_CHECK(A.device() == fused.device(), "Inputs must be on same device");
    TORCH_CHECK(A.dtype() == torch::kFloat16, "A must be float16");
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    check_fused(fused);
    const int64_t K = fused_k(fused.size(1)), N = fused.size(0) * 16;
    TORCH_CHECK(A.size(1) == K, "Inner dimensions must match");
    TORCH_CHECK(group_size > 0 && K % group_size == 0, "group_size must divide K");
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(A.device());
    if (perm.has_value() && perm->defined()) {
        TORCH_CHECK(perm->device() == A.device() && perm->dim() == 1 && perm->size(0) == K &&
                        perm->dtype() == torch::kInt64,
                    "perm must be the int64 [K] permutation returned by int4_from_gptq");
        A = A.index_select(1, *perm);
    }
    A = A.contiguous();
    fused = fused.contiguous();
    check_aligned(A, "A must be 16-byte aligned");
    const int M = (int)A.size(0);
    auto Y = torch::empty({A.size(0), N},
                          torch::dtype(half_out ? torch::kFloat16 : torch::kFloat32).device(A.device()));
    int rc;
    if (half_out)
        rc = wmma_w4a16_gemm_f16out(A.data_ptr(), A.stride(0), fused.data_ptr<int32_t>(), nullptr,
                                    nullptr, WMMA_W4_FUSED, M, (int)N, (int)K, (int)group_size,
                                    Y.data_ptr(), Y.stride(0), nullptr, 0, current_stream(A));
    else
        rc = wmma_w4a16_gemm(A.data_ptr(), A.stride(0), fused.data_ptr<int32_t>(), nullptr, nullptr,
                             WMMA_W4_FUSED, M, (int)N, (int)K, (int)group_size, Y.data_ptr<float>(),
                             Y.stride(0), nullptr, 0, current_stream(A));
    check_status(rc, "wmma_w4a16_gemm");
    return Y;
}

// matmul_int4(A[M,K] fp16, packed (from prepack_int4), scales[K/G, N] fp16,
//             zeros[K/G, N/8] int32 packed or [K/G, N] uint8, group_size=128) -> fp32 [M, N];
// or scales and zeros as returned by prepack_int4_params.
torch::Tensor matmul_int4(torch::Tensor A, torch::Tensor packed, torch::Tensor scales,
                          torch::Tensor zeros, int64_t group_size,
                          c10::optional<at::ScalarType> out_dtype,
                          c10::optional<torch::Tensor> perm) {
    const bool half_out = out_dtype.has_value() && *out_dtype == torch::kFloat16;
    TORCH_CHECK(!out_dtype.has_value() || *out_dtype == torch::kFloat16 ||
                    *out_dtype == torch::kFloat32,
                "out_dtype must be float32 or float16");
    TORCH_CHECK(A.is_cuda() && packed.is_cuda() && scales.is_cuda() && zeros.is_cuda(),
                "Inputs must be CUDA tensors");
    TORCH_CHECK(A.device() == packed.device() && A.device() == scales.device() &&
                    A.device() == zeros.device(),
                "Inputs must be on same device");
    TORCH_CHECK(A.dtype() == torch::kFloat16, "A must be float16");
    TORCH_CHECK(A.dim() == 2, "A must be 2D");
    check_packed(packed);
    const int64_t K = packed.size(1) * 64, N = packed.size(0) * 16;
    TORCH_CHECK(A.size(1) == K, "Inner dimensions must match");
    TORCH_CHECK(group_size > 0 && K % group_size == 0, "group_size must divide K");
    const int64_t ng = K / group_size;
    int zfmt;
    if (scales.dim() == 3) {  // slice-major parameters from prepack_int4_params
        TORCH_CHECK(scales.dtype() == torch::kFloat16 && scales.size(0) * 16 == N &&
                        scales.size(1) == ng && scales.size(2) == 16,
                    "sliced scales must be float16 [N/16, K/group_size, 16]");
        TORCH_CHECK(zeros.dtype() == torch::kInt32 && zeros.dim() == 3 &&
                        zeros.size(0) * 16 == N && zeros.size(1) == ng && zeros.size(2) == 2,
                    "sliced zeros must be int32 [N/16, K/group_size, 2]");
        zfmt = WMMA_ZEROS_SLICED;
    } else if (!(scales.dtype() == torch::kFloat16 && scales.dim() == 2 &&
                 scales.size(0) == ng && scales.size(1) == N)) {
        TORCH_CHECK(false, "scales must be float16 [K/group_size, N]");
    } else if (zeros.dtype() == torch::kInt32) {
        TORCH_CHECK(zeros.dim() == 2 && zeros.size(0) == ng && zeros.size(1) * 8 == N,
                    "packed zeros must be int32 [K/group_size, N/8]");
        zfmt = WMMA_ZEROS_PACKED;
    } else {
        TORCH_CHECK(zeros.dtype() == torch::kUInt8 && zeros.dim() == 2 && zeros.size(0) == ng &&
                        zeros.size(1) == N,
                    "zeros must be int32 [K/group_size, N/8] or uint8 [K/group_size, N]");
        zfmt = WMMA_ZEROS_U8;
    }
    const c10::hip::HIPGuardMasqueradingAsCUDA guard(A.device());
    if (perm.has_value() && perm->defined()) {  // act-order weights from int4_from_gptq
        TORCH_CHECK(perm->device() == A.device() && perm->dim() == 1 && perm->size(0) == K &&
                        perm->dtype() == torch::kInt64,
                    "perm must be the int64 [K] permutation returned by int4_from_gptq");
        A = A.index_select(1, *perm);
    }
    A = A.contiguous();
    packed = packed.contiguous();
    scales = scales.contiguous();
    zeros = zeros.contiguous();
    check_aligned(A, "A must be 16-byte aligned");
    const int M = (int)A.size(0);
    auto Y = torch::empty({A.size(0), N},
                          torch::dtype(half_out ? torch::kFloat16 : torch::kFloat32).device(A.device()));
    const size_t ws_bytes = wmma_w4a16_workspace_size(M, (int)N, (int)K, (int)group_size);
    torch::Tensor ws = workspace_for(ws_bytes, A);
    int rc;
    if (half_out)
        rc = wmma_w4a16_gemm_f16out(A.data_ptr(), A.stride(0), packed.data_ptr<int32_t>(),
                                    scales.data_ptr(), zeros.data_ptr(), zfmt, M, (int)N, (int)K,
                                    (int)group_size, Y.data_ptr(), Y.stride(0),
                                    ws.defined() ? ws.data_ptr() : nullptr, ws_bytes,
                                    current_stream(A));
    else
        rc = wmma_w4a16_gemm(A.data_ptr(), A.stride(0), packed.data_ptr<int32_t>(),
                             scales.data_ptr(), zeros.data_ptr(), zfmt, M, (int)N, (int)K,
                             (int)group_size, Y.data_ptr<float>(), Y.stride(0),
                             ws.defined() ? ws.data_ptr() : nullptr, ws_bytes, current_stream(A));
    check_status(rc, "wmma_w4a16_gemm");
    return Y;
}

// Planner introspection: (kernel, tile_cfg, tile_m, tile_n, split_k, k_per_split, grid,
// workspace_bytes, edge_dim, edge_at) for a shape on the current device.
std::vector<int64_t> gemm_plan(int64_t M, int64_t N, int64_t K, int64_t tile_cfg, int64_t num_cus) {
    wmma_gemm_plan p{};
    check_status(wmma_gemm_plan_make((int)M, (int)N, (int)K, (int)tile_cfg, (int)num_cus, &p),
                 "wmma_gemm_plan_make");
    return {p.kernel, p.tile_cfg, p.tile_m, p.tile_n, p.split_k, p.k_per_split, p.grid,
            (int64_t)p.workspace_bytes, p.edge_dim, p.edge_at};
}

// W4A16 planner introspection: (kernel, split_k, k_per_split, workspace_bytes).
std::vector<int64_t> w4a16_plan(int64_t M, int64_t N, int64_t K, int64_t group_size,
                                int64_t num_cus) {
    wmma_w4a16_plan p{};
    check_status(wmma_w4a16_plan_make((int)M, (int)N, (int)K, (int)group_size, (int)num_cus, &p),
                 "wmma_w4a16_plan_make");
    return {p.kernel, p.split_k, p.k_per_split, (int64_t)p.workspace_bytes};
}

}  // namespace

PYBIND11_MODULE(TORCH_EXTENSION_NAME, m) {
    m.doc() = "MI355X (gfx950) MFMA implementation of the wmma_ops API";
    m.def("matmul", &matmul, "MFMA GEMM (FP16->FP32), tile chosen by the planner");
    m.def("matmul_adaptive", &matmul_adaptive, "MFMA GEMM with automatic tile / split-K choice");
    m.def("matmul_tiled", &matmul_tiled,
          "MFMA GEMM with a fixed tile: 0=64x64, 1=128x64, 2=256x64, 3=128x128, 4=256x128, 5=256x256");
    m.def("gemm", &gemm, "BLAS-style GEMM: C = alpha * A @ B + beta * C", py::arg("A"), py::arg("B"),
          py::arg("alpha") = 1.0, py::arg("beta") = 0.0, py::arg("C") = py::none());
    m.def("gemm_inplace", &gemm_inplace, "In-place GEMM: C = alpha * A @ B + beta * C (modifies C)",
          py::arg("A"), py::arg("B"), py::arg("C"), py::arg("alpha") = 1.0, py::arg("beta") = 0.0);
    m.def("gemm_adaptive", &gemm_adaptive,
          "Auto-tuned GEMM: C = alpha * A @ B + beta * C (planner-selected tile)", py::arg("A"),
          py::arg("B"), py::arg("alpha") = 1.0, py::arg("beta") = 0.0, py::arg("C") = py::none());
    m.def("flash_attention", &flash_attention, "Flash-attention forward (fp16 in/out, fp32 softmax)",
          py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("causal") = false,
          py::arg("scale") = -1.0);
    m.def("flash_attention_varlen", &flash_attention_varlen,
          "Flash-attention forward on packed variable-length sequences", py::arg("q"), py::arg("k"),
          py::arg("v"), py::arg("cu_seqlens_q"), py::arg("cu_seqlens_k"), py::arg("max_seqlen_q"),
          py::arg("max_seqlen_k"), py::arg("causal") = false, py::arg("scale") = -1.0);
    m.def("flash_attention_forward", &flash_attention_forward,
          "Flash-attention forward for training: returns (O, lse fp32 [B, H, Sq])", py::arg("Q"),
          py::arg("K"), py::arg("V"), py::arg("causal") = false, py::arg("scale") = -1.0);
    m.def("flash_attention_backward", &flash_attention_backward,
          "Flash-attention backward: (dQ, dK, dV) from dO, Q, K, V, O and lse", py::arg("dO"),
          py::arg("Q"), py::arg("K"), py::arg("V"), py::arg("O"), py::arg("lse"),
          py::arg("causal") = false, py::arg("scale") = -1.0);
    m.def("flash_attention_varlen_forward", &flash_attention_varlen_forward,
          "Variable-length forward for training: returns (O, lse fp32 [H, total_q])", py::arg("q"),
          py::arg("k"), py::arg("v"), py::arg("cu_seqlens_q"), py::arg("cu_seqlens_k"),
          py::arg("max_seqlen_q"), py::arg("max_seqlen_k"), py::arg("causal") = false,
          py::arg("scale") = -1.0);
    m.def("flash_attention_varlen_backward", &flash_attention_varlen_backward,
          "Variable-length backward: (dq, dk, dv)", py::arg("dO"), py::arg("q"), py::arg("k"),
          py::arg("v"), py::arg("O"), py::arg("lse"), py::arg("cu_seqlens_q"),
          py::arg("cu_seqlens_k"), py::arg("max_seqlen_q"), py::arg("max_seqlen_k"),
          py::arg("causal") = false, py::arg("scale") = -1.0);
    m.def("prepack_int4", &prepack_int4, "GPTQ int4 qweight [K/8,N] -> MFMA layout", py::arg("qweight"));
    m.def("unprepack_int4", &unprepack_int4, "Inverse of prepack_int4", py::arg("packed"));
    m.def("unpack_int4", &unpack_int4, "GPTQ int4 qweight [K/8,N] -> uint8 [K,N]", py::arg("qweight"));
    m.def("prepack_int4_params", &prepack_int4_params,
          "scales/zeros -> slice-major layout accepted by matmul_int4", py::arg("scales"),
          py::arg("zeros"));
    m.def("prepack_int4_fused", &prepack_int4_fused,
          "GPTQ qweight + scales + zeros -> fused decode layout (one run per 16 columns)",
          py::arg("qweight"), py::arg("scales"), py::arg("zeros"), py::arg("group_size") = 128);
    m.def("unprepack_int4_fused", &unprepack_int4_fused,
          "Inverse of prepack_int4_fused: (qweight, scales, packed zeros)", py::arg("fused"),
          py::arg("group_size") = 128);
    m.def("matmul_int4_fused", &matmul_int4_fused,
          "W4A16 for decode shapes (M <= 4) from the fused layout", py::arg("A"), py::arg("fused"),
          py::arg("group_size") = 128, py::arg("out_dtype") = py::none(),
          py::arg("perm") = py::none());
    m.def("matmul_int4", &matmul_int4,
          "W4A16 dequant GEMM: fp16 A @ int4 W -> fp32 (or fp16 with out_dtype=torch.float16)",
          py::arg("A"), py::arg("packed"), py::arg("scales"), py::arg("zeros"),
          py::arg("group_size") = 128, py::arg("out_dtype") = py::none(),
          py::arg("perm") = py::none());
    m.def("int4_from_gptq", &int4_from_gptq,
          "GPTQ qweight [K/8,N] / qzeros [K/G,N/8] (+ g_idx) -> (qweight, packed zeros, perm or None)",
          py::arg("qweight"), py::arg("qzeros"), py::arg("g_idx") = py::none(),
          py::arg("zero_format") = "v1");
    m.def("int4_from_awq", &int4_from_awq,
          "AutoAWQ qweight [K,N/8] / qzeros [K/G,N/8] -> GPTQ-layout qweight and packed zeros",
          py::arg("qweight"), py::arg("qzeros"));
    m.def("w4a16_plan", &w4a16_plan, "Planner decision for a W4A16 shape", py::arg("M"),
          py::arg("N"), py::arg("K"), py::arg("group_size") = 128, py::arg("num_cus") = 256);
    m.def("gemm_plan", &gemm_plan,
          "Planner decision for a GEMM shape: [kernel, tile_cfg, tile_m, tile_n, split_k, "
          "k_per_split, grid, workspace_bytes, edge_dim, edge_at] (edge_dim 1 / 2: rows / "
          "columns from edge_at run as a second GEMM)",
          py::arg("M"), py::arg("N"),
          py::arg("K"), py::arg("tile_cfg") = -1, py::arg("num_cus") = 256);
}
