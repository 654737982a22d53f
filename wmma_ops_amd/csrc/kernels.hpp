// Internal launch interface between the C-ABI layer (capi.hip) and the kernel files.
// Every launcher only enqueues work on `stream`; argument checking happens in capi.hip.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/wmma_ops_amd.h"

namespace wmma_amd {

struct GemmLaunch {
    const void* A;
    const void* B;
    const float* C_in;
    float* C_out;
    void* workspace;
    int64_t lda, ldb, ldc_in, ldc;
    int M, N, K;
    float alpha, beta;
    bool vec;  // 16-byte vector path: K, N, lda, ldb multiples of 8, A and B 16-byte aligned
    // Skinny kernel when !vec: 0 = element-wise; 2 / 3 = A in 16-byte vectors, B 4-byte
    // aligned with ldb even / odd (rows read in place by dword-aligned 16-byte loads)
    int skinny_b;
    wmma_gemm_plan plan;
};
hipError_t launch_gemm(const GemmLaunch& g, hipStream_t stream);
// Dense zero-padded copy of a [rows][cols] fp16 matrix (leading dimension ld, any
// alignment) into dst [rows][cols rounded up to 8]; dst 4-byte aligned.
hipError_t launch_gemm_repack(const void* src, int64_t ld, int rows, int cols, void* dst,
                              hipStream_t stream);

// INT4 weight layout conversions (w4a16.hip).
hipError_t launch_int4_prepack(const int32_t* qweight, int K, int N, int32_t* packed,
                               hipStream_t stream);
hipError_t launch_int4_unprepack(const int32_t* packed, int K, int N, int32_t* qweight,
                                 hipStream_t stream);
// Scales [KG][N] and zeros (packed or uint8) to the slice-major layout (WMMA_ZEROS_SLICED).
hipError_t launch_int4_params_slice(const void* scales, const void* zeros, int zeros_format,
                                    int KG, int N, void* scales_out, int32_t* zeros_out,
                                    hipStream_t stream);
// AutoAWQ tensors (qweight [K][N/8], qzeros [KG][N/8], nibbles in AWQ order) to this
// library's GPTQ-layout qweight [K/8][N] and packed zeros [KG][N/8].
hipError_t launch_int4_from_awq(const int32_t* qweight_awq, const int32_t* qzeros_awq, int K,
                                int N, int KG, int32_t* qweight, int32_t* zeros,
                                hipStream_t stream);
hipError_t launch_int4_unpack(const int32_t* qweight, int K, int N, uint8_t* q,
                              hipStream_t stream);
// GPTQ checkpoint zero points (packed [KG][N/8]) + add (1 for AutoGPTQ's v1 format, 0 for
// v2) per nibble; *overflow (may be NULL) set to 1 where a nibble would exceed 15.
hipError_t launch_int4_gptq_zeros(const int32_t* qzeros, int KG, int N, int add, int32_t* zeros,
                                  int32_t* overflow, hipStream_t stream);
// GPTQ-layout weights with rows permuted: output row k = input row perm[k].
hipError_t launch_int4_permute_rows(const int32_t* qweight, const int32_t* perm, int K, int N,
                                    int32_t* out, hipStream_t stream);
// Fused decode layout (WMMA_W4_FUSED, w4a16.hip), per 16-column slice: a header of one
// 160-byte parameter block per four 128-deep K steps, zero-padded to a multiple of 128
// bytes, then the slice's prepacked weights (1 KB per K step).  K % 128 == 0.
__host__ __device__ inline int64_t fused_hdr_bytes(int K) {
    const int blocks = (K / 128 + 3) / 4;
    return ((int64_t)160 * blocks + 127) / 128 * 128;
}
__host__ __device__ inline int64_t fused_slice_bytes(int K) {
    return fused_hdr_bytes(K) + (int64_t)(K / 128) * 1024;
}
// GPTQ qweight + scales [KG][N] + zeros (packed or uint8) -> fused buffer, and back
// (scales [KG][N], packed zeros [KG][N/8]); G % 128 == 0.
hipError_t launch_int4_prepack_fused(const int32_t* qweight, const void* scales, const void* zeros,
                                     int zeros_format, int K, int N, int G, int32_t* fused,
                                     hipStream_t stream);
hipError_t launch_int4_unprepack_fused(const int32_t* fused, int K, int N, int G, int32_t* qweight,
                                       void* scales, int32_t* zeros, hipStream_t stream);

// W4A16 kernel families.
enum W4A16Kind {
    W4_DECODE_MFMA = 0,  // M <= 4, G = 128 * 2^j: one workgroup per 16 columns, matrix-pipe dots
    W4_DECODE = 1,       // M <= 4: one workgroup per 16 columns, VALU dots
    W4_GEMV_SPLIT = 2,   // M <= 4, other shapes: 32 columns per workgroup, K split + reduce
    W4_MFMA = 3,         // larger M: tiled MFMA kernel, K split + reduce when few tiles
    W4_SKINNY = 4,       // 4 < M <= 32: 32 columns per workgroup, K split + reduce when few tiles
    W4_GEMM = 5,         // M > 32: LDS-DMA MFMA GEMM, K split + reduce when few tiles
    W4_ROWS = 6,         // M > 32: row groups x column groups, register-staged, no LDS ring
};

struct W4A16Plan {
    int kind;         // W4A16Kind
    int split;        // K partitions (1: no workspace)
    int k_per_split;  // multiple of 64 (and of G when split > 1)
    int big = 0;      // W4_GEMM: tile (W4G_TILE_*); W4_SKINNY, W4_ROWS: 16-column slices per workgroup
    int mb = 0;       // W4_ROWS: 16-row blocks per workgroup
};

struct W4A16Launch {
    const void* A;
    int64_t lda;
    const int32_t* packed;
    const void* scales;
    const void* zeros;
    int zeros_format;
    int M, N, K, G;
    float* Y;          // fp32 [M][ldy], or fp16 when y_half
    int64_t ldy;
    void* workspace;
    W4A16Plan plan;
    bool y_half = false;
};
hipError_t launch_w4a16(const W4A16Launch& w, hipStream_t stream);
// Planner for the W4A16 kernels (host-only).  `aligned`: scales 8-byte aligned and, for
// uint8 zeros, zeros 4-byte aligned (the vector loads of the matrix-pipe decode kernel).
W4A16Plan w4a16_plan(int M, int N, int K, int G, int num_cus, bool aligned);
// Whether the matrix-pipe decode kernel (the one reader of the fused layout) takes M rows
// at this K: M <= 4 and its staged activations within its LDS budget.
bool w4a16_fused_decode_ok(int M, int K);

struct FlashLaunch {
    const void* Q;
    const void* K;
    const void* V;
    void* O;
    int B, H, Sq, Sk, D;
    int Hkv;  // key/value heads (H % Hkv == 0; H for multi-head attention)
    float scale;
    bool causal;
    // Variable length: packed Q/O [total_q][H][D], K/V [total_k][Hkv][D], sequence b in
    // rows cu_q[b] .. cu_q[b+1] (cu_k likewise); Sq/Sk are then the longest lengths.
    const int* cu_q = nullptr;
    const int* cu_k = nullptr;
    int total_q = 0, total_k = 0;
    // Optional log-sum-exp output (fp32, natural log): [B*H][Sq], or [H][total_q] for
    // variable length.
    float* lse = nullptr;
    // Dense layout only: split the key range into kv_split chunks (> 1) whose partial
    // sums go to workspace (flash_fwd_workspace_bytes, 16-byte aligned), merged by a
    // second kernel.
    int kv_split = 1;
    void* workspace = nullptr;
};
hipError_t launch_flash_fwd(const FlashLaunch& f, hipStream_t stream);
// Key-range split the forward uses for a dense shape on num_cus CUs (1: none): only when
// the query blocks leave more than half the CUs idle and the partial sums stay small.
int flash_kv_split(int B, int H, int Hkv, int Sq, int Sk, int D, int num_cus);
// Workspace bytes of a split (0 for split <= 1); D is the head dim passed to the kernels.
size_t flash_fwd_workspace_bytes(int B, int H, int Sq, int Sk, int D, int split);

// Flash-attention backward: dQ, dK, dV (fp16, the layouts of Q, K, V) from dO, Q, K, V, O
// and the forward's log-sum-exp.  ws: fp32 workspace of 2 * flash_bwd_workspace_rows().
struct FlashBwdLaunch {
    const void* Q;
    const void* K;
    const void* V;
    const void* O;
    const void* dO;
    const float* lse;
    void* dQ;
    void* dK;
    void* dV;
    float* ws;
    int B, H, Hkv, Sq, Sk, D;
    float scale;
    bool causal;
    const int* cu_q = nullptr;
    const int* cu_k = nullptr;
    int total_q = 0, total_k = 0;
    // Dense grouped-query attention: split the dK/dV kernel's query heads of a group over
    // gsplit workgroups (> 1) whose fp32 partial dK, dV go to kv_part
    // (flash_bwd_split_bytes, 16-byte aligned), added by a second kernel.
    int gsplit = 1;
    float* kv_part = nullptr;
};
int64_t flash_bwd_workspace_rows(const FlashBwdLaunch& f);
// Grouped-query split of the dK/dV kernel for a dense shape on num_cus CUs (1: none): when
// its workgroups would fill less than half of one wave, or (causal) at most one wave.
int flash_bwd_group_split(int B, int H, int Hkv, int Sq, int Sk, int D, bool causal,
                          int num_cus);
size_t flash_bwd_split_bytes(int B, int Hkv, int Sk, int D, int gsplit);
hipError_t launch_flash_bwd(const FlashBwdLaunch& f, hipStream_t stream);

}  // namespace wmma_amd
