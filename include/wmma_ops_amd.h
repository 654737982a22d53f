/*
 * wmma_ops_amd.h -- C-ABI of the MI355X (gfx950 / CDNA4) matrix-core hot path.
 *
 * Plain pointers, sizes and an opaque stream handle; no torch or HIP types appear in
 * any signature.  Every entry point is asynchronous on `stream` (a hipStream_t passed
 * as void*; NULL means the null stream), never synchronises, never allocates device
 * memory, and returns a status code (WMMA_OK == 0).  On failure the text of the last
 * error on the calling thread is available from wmma_last_error().  Arguments are
 * validated completely before anything touches the GPU, so every validation error is
 * reachable without a device.
 *
 * The reference (glovepost/wmma_ops) exposes its path as pybind functions inside one
 * PyTorch extension (wmma_gemm.hip:2120-2157).  Each function below names the reference
 * interface it replaces.  Matrices are row-major; leading dimensions are in elements.
 */
#ifndef WMMA_OPS_AMD_H
#define WMMA_OPS_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WMMA_OPS_AMD_ABI_VERSION 2

/* Status codes. */
#define WMMA_OK 0
#define WMMA_ERR_INVALID_ARG 1   /* bad shape, null pointer, bad leading dimension      */
#define WMMA_ERR_UNSUPPORTED 2   /* valid request this build does not implement         */
#define WMMA_ERR_MISALIGNED 3    /* pointer or leading dimension breaks 16-byte vectors  */
#define WMMA_ERR_WORKSPACE 4     /* workspace missing or smaller than *_workspace_size  */
#define WMMA_ERR_HIP 5           /* launch or runtime error reported by HIP              */

/* GEMM tile configurations.  0..3 are the reference's matmul_tiled menu
 * (wmma_gemm.hip:1500-1523: 0=64x64, 1=128x64, 2=256x64, 3=128x128); 4 and 5 add the
 * larger CDNA4 tiles.  WMMA_TILE_AUTO lets the planner choose tile and split-K. */
#define WMMA_TILE_AUTO (-1)
#define WMMA_TILE_64x64 0
#define WMMA_TILE_128x64 1
#define WMMA_TILE_256x64 2
#define WMMA_TILE_128x128 3
#define WMMA_TILE_256x128 4
#define WMMA_TILE_256x256 5
#define WMMA_TILE_COUNT 6

/* Kernel families a GEMM plan can select. */
#define WMMA_KERNEL_TILED 0   /* MFMA tiled kernel (optionally split-K + reduce)        */
#define WMMA_KERNEL_SKINNY 1  /* M <= 64 streaming kernel (planner: M <= 32), split-K   */

/* Two-part GEMMs (wmma_gemm_plan.edge_dim).  A shape whose 256x256 tiles fill some whole
 * waves of the chip plus a small partial one can run as two launches: the bulk (rows or
 * columns [0, edge_at)) on whole waves of 256x256 tiles, then the edge (the rest) as a
 * GEMM of its own, with the plan wmma_gemm_plan_make gives for that shape (always a
 * one-launch plan). */
#define WMMA_EDGE_NONE 0  /* one launch                                                  */
#define WMMA_EDGE_ROWS 1  /* rows [edge_at, M) run as the second GEMM                    */
#define WMMA_EDGE_COLS 2  /* columns [edge_at, N) run as the second GEMM                 */

typedef struct wmma_gemm_plan {
    int kernel;            /* WMMA_KERNEL_*                                              */
    int tile_cfg;          /* WMMA_TILE_* actually used (-1 for the skinny kernel)       */
    int tile_m, tile_n;    /* output tile of one workgroup                               */
    int split_k;           /* number of K partitions (1 = no split, no workspace)        */
    int k_per_split;       /* K elements per partition (multiple of 64)                  */
    int grid;              /* workgroups of the main kernel                              */
    size_t workspace_bytes;/* fp32 partial sums: split_k * M * N * 4, 0 when split_k==1;
                              for a two-part plan the larger of the two parts' needs      */
    int edge_dim;          /* WMMA_EDGE_*; the fields above then describe the bulk launch */
    int edge_at;           /* first row / column of the edge GEMM (0 without one)        */
} wmma_gemm_plan;

/* Text of the last error reported on this thread ("" if none). */
const char* wmma_last_error(void);

/* ABI version of the loaded library (WMMA_OPS_AMD_ABI_VERSION). */
int wmma_abi_version(void);

/* Number of compute units the planner assumes for device `device` (queried from HIP
 * once per device; 256 for an MI355X).  Returns 256 when no device can be queried. */
int wmma_device_cu_count(int device);

/* Host-only planner: the kernel, tile, split-K and workspace a GEMM of this shape uses
 * on a device with `num_cus` compute units, and whether it runs as two parts (edge_dim;
 * only with tile_cfg WMMA_TILE_AUTO).  tile_cfg as for wmma_gemm_f16f32.
 * Replaces the reference's select_optimal_tile (wmma_tile_selection.hpp:30-66) and
 * split_k::compute_config (wmma_xor_swizzle.hpp:293-332). */
int wmma_gemm_plan_make(int M, int N, int K, int tile_cfg, int num_cus, wmma_gemm_plan* out);

/* The same planner's choice among the plans whose split-K partial sums fit
 * max_workspace_bytes (a plan without a K split needs none, so one always exists): for
 * callers with a fixed workspace budget; wmma_gemm_f16f32_noalloc plans this way within
 * its scratch array.  No counterpart in the reference (its split-K wrapper allocates its
 * own workspace, wmma_xor_swizzle.hpp:1208-1215). */
int wmma_gemm_plan_make_within(int M, int N, int K, int tile_cfg, int num_cus,
                               size_t max_workspace_bytes, wmma_gemm_plan* out);

/* Workspace bytes wmma_gemm_f16f32 uses for this shape on the current device, for
 * contiguous 16-byte-aligned operands (lda = K, ldb = N): the split-K partial sums
 * (plan.workspace_bytes) plus, when K or N is not a multiple of 8, room for zero-padded
 * copies of the operands whose rows then break 16-byte vectors (A [M][K rounded up to 8],
 * B [K][N rounded up to 8], 256-byte aligned, 256 bytes of slack). */
size_t wmma_gemm_workspace_size(int M, int N, int K, int tile_cfg);

/*
 * C_out[M,N] = alpha * (A[M,K] @ B[K,N]) + beta * C_in[M,N]      (fp16 in, fp32 accumulate
 * and out).  C_in is read only when beta != 0 and C_in != NULL; C_in may equal C_out
 * (in-place).  tile_cfg: WMMA_TILE_AUTO or 0..WMMA_TILE_COUNT-1.  workspace: device
 * memory of at least plan.workspace_bytes (the split-K partial sums; may be NULL when that
 * is 0), 4-byte aligned.  An operand whose rows break 16-byte vectors (K or N not a
 * multiple of 8, lda or ldb not a multiple of 8, A or B not 16-byte aligned) is copied into
 * a zero-padded dense buffer taken from the workspace behind the partial sums when the
 * workspace holds it (wmma_gemm_workspace_size(M,N,K,tile_cfg) bytes always do for
 * contiguous operands), and the 16-byte vector kernels run on the copy; with less
 * workspace the element-wise kernels read it in place (same result, several times
 * slower).
 * Replaces wmma_matmul (wmma_gemm.hip:1432-1470), wmma_matmul_tiled (:1473-1528),
 * wmma_matmul_adaptive (:1197-1263), wmma_gemm (:1891-1945), wmma_gemm_inplace
 * (:1949-1994) and wmma_gemm_adaptive (:1997-2078), and the unreachable split-K wrapper
 * (wmma_xor_swizzle.hpp:1172-1219).
 */
int wmma_gemm_f16f32(const void* A, int64_t lda, const void* B, int64_t ldb,
                     const float* C_in, int64_t ldc_in, float* C_out, int64_t ldc,
                     int M, int N, int K, float alpha, float beta, int tile_cfg,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Allocation-free variant of wmma_gemm_f16f32: the same computation and kernels, but no
 * workspace argument -- the split-K partial sums go to a device array inside this library
 * (wmma_gemm_noalloc_scratch_bytes() = 32 MiB per GPU, held until the process ends), so the
 * call performs no allocation of any kind.  Its plan is wmma_gemm_plan_make_within(...,
 * wmma_gemm_noalloc_scratch_bytes(), ...): the same as wmma_gemm_f16f32's wherever that
 * plan's partial sums fit the array, else the planner's next choice that fits (a smaller
 * K split, so a bit-different fp32 sum order).  Every call on one GPU shares that GPU's array and nothing in it has to
 * start at zero (each split writes its whole partial tile before the reduction reads it).
 * Calls outside stream capture are ordered by the library: a call on another stream than
 * the previous split-K call on the GPU first waits (hipStreamWaitEvent) for an event
 * recorded after that call's launches (the event is created by the first such call; host
 * threads are serialised around wait + launch + record).  Under stream capture nothing is
 * waited on or recorded: replays of a captured graph use the same array, so the caller
 * must not let them overlap each other or other calls on the GPU.  The first call on a GPU
 * (which looks up the array's address) may itself be made under capture.
 * Operands whose rows break 16-byte vectors are read in place
 * by the element-wise kernels (no repacked copy).  No counterpart in the reference: for
 * callers that cannot allocate (code under stream capture, tight serving loops, harnesses
 * that forbid it).
 */
int wmma_gemm_f16f32_noalloc(const void* A, int64_t lda, const void* B, int64_t ldb,
                             const float* C_in, int64_t ldc_in, float* C_out, int64_t ldc, int M,
                             int N, int K, float alpha, float beta, int tile_cfg, void* stream);
size_t wmma_gemm_noalloc_scratch_bytes(void);

/*
 * Explicit plans.  wmma_gemm_plan_custom builds the plan of one kernel (WMMA_KERNEL_*),
 * tile (WMMA_TILE_*, ignored by the skinny kernel) and K split for a shape, completed as
 * the planner completes its own; wmma_gemm_f16f32_plan runs wmma_gemm_f16f32 with such a
 * plan (it must describe this M, N, K; workspace: plan->workspace_bytes).  They replace the
 * reference's tuned dispatch (autotune.py:131-283 emits select_tuned_tile): the autotuner
 * (wmma_ops_amd/autotune.py) times plans through them, and its table of measured winners
 * is compiled into the planner.
 */
int wmma_gemm_plan_custom(int M, int N, int K, int kernel, int tile_cfg, int split_k,
                          wmma_gemm_plan* out);
int wmma_gemm_f16f32_plan(const void* A, int64_t lda, const void* B, int64_t ldb,
                          const float* C_in, int64_t ldc_in, float* C_out, int64_t ldc, int M,
                          int N, int K, float alpha, float beta, const wmma_gemm_plan* plan,
                          void* workspace, size_t workspace_bytes, void* stream);

/*
 * INT4 weights.  The reference has no INT4 code; the layout is this library's own.
 * "GPTQ layout": qweight is int32 [K/8, N]; weight q[k][n] (0..15) sits in bits
 * 4*(k%8) .. 4*(k%8)+3 of qweight[k/8][n].  K % 64 == 0 and N % 32 == 0 are required.
 * Prepacked layout: int32 [N/16][K/64][32][4]; entry l of block kc of 16-column slice s
 * holds column n = 16*s + l%16 and the four GPTQ words of k-groups 8*kc + 4*(l/16) + 0..3,
 * each with its nibbles reordered to k-offsets {0,2,4,6,1,3,5,7}.  A slice's weights are
 * one contiguous run over all of K.
 */
int wmma_int4_prepack(const int32_t* qweight, int K, int N, int32_t* packed, void* stream);
/* Inverse of wmma_int4_prepack (prepacked layout back to the GPTQ layout). */
int wmma_int4_unprepack(const int32_t* packed, int K, int N, int32_t* qweight, void* stream);
/* Debug unpack: GPTQ-layout qweight -> uint8 q[K][N] (row-major). */
int wmma_int4_unpack(const int32_t* qweight, int K, int N, uint8_t* q, void* stream);

#define WMMA_ZEROS_PACKED 0  /* zeros int32 [K/G, N/8]; z[g][n] in bits 4*(n%8).. of [g][n/8] */
#define WMMA_ZEROS_U8 1      /* zeros uint8 [K/G, N]                                       */
#define WMMA_ZEROS_SLICED 2  /* scales AND zeros in the slice-major layout of
                                wmma_int4_prepack_params: scales fp16 [N/16][K/G][16],
                                zeros int32 [N/16][K/G][2] (word w: columns 16*i+8w.., nibble
                                n%8) -- a 16-column slice's parameters are contiguous      */

/*
 * Group parameters to the slice-major layout (WMMA_ZEROS_SLICED), bit-exact: scales
 * fp16 [K/G, N] -> scales_out [N/16][K/G][16]; zeros (WMMA_ZEROS_PACKED int32 [K/G, N/8]
 * or WMMA_ZEROS_U8 uint8 [K/G, N]) -> zeros_out int32 [N/16][K/G][2].  A one-time layout
 * conversion like wmma_int4_prepack: the decode kernel reads a slice's parameters as one
 * contiguous run.  N % 32 == 0, K % group_size == 0.  No reference counterpart.
 */
int wmma_int4_prepack_params(const void* scales, const void* zeros, int zeros_format, int K,
                             int N, int group_size, void* scales_out, int32_t* zeros_out,
                             void* stream);

/*
 * Fused decode layout (zeros_format WMMA_W4_FUSED of wmma_w4a16_gemm): the prepacked
 * weights, scales and zero points of each 16-column slice in one contiguous run, so that
 * a decode workgroup streams a single region of memory.  Per slice (wmma_int4_fused_bytes(K,
 * N) / (N/16) bytes each):
 *   header   one 160-byte block per four 128-deep K steps 4r .. 4r+3 (the last block covers
 *            the steps left), zero-padded to a multiple of 128 bytes:
 *              bytes [0, 128)   scales fp16 [4][16]: entry (u, c) = s[g][16*slice + c] of K
 *                               step 4r+u, g = 128 (4r+u) / G
 *              bytes [128, 160) zero points [4][16] as nibbles: byte 128 + 8u + c/2, nibble
 *                               c % 2 (even columns in the low nibble)
 *   weights  the slice's run of the prepacked layout above (1 KB per K step).
 * With G = 128 and K % 4096 == 0 these are exactly the bytes of the prepacked weights plus
 * the scales and packed zeros; a larger G repeats a group's parameters in each of its K
 * steps.  Requirements: K % 128 == 0, N % 32 == 0, G % 128 == 0 with G / 128 a power of two.
 * wmma_w4a16_gemm reads this layout for M <= 4 (decode shapes: the kernel this layout is
 * for); other M return WMMA_ERR_UNSUPPORTED.  No reference counterpart.
 */
#define WMMA_W4_FUSED 3
size_t wmma_int4_fused_bytes(int K, int N);
/* GPTQ qweight [K/8, N] + scales fp16 [K/G, N] + zeros (WMMA_ZEROS_PACKED or WMMA_ZEROS_U8)
 * -> fused buffer (16-byte aligned, wmma_int4_fused_bytes bytes), bit-exact. */
int wmma_int4_prepack_fused(const int32_t* qweight, const void* scales, const void* zeros,
                            int zeros_format, int K, int N, int group_size, int32_t* fused,
                            void* stream);
/* Inverse: fused buffer -> qweight [K/8, N], scales fp16 [K/G, N], packed zeros int32
 * [K/G, N/8] (each group's parameters read from its first K step). */
int wmma_int4_unprepack_fused(const int32_t* fused, int K, int N, int group_size,
                              int32_t* qweight, void* scales, int32_t* zeros, void* stream);

/* Workspace bytes wmma_w4a16_gemm needs (fp32 split-K partials). */
size_t wmma_w4a16_workspace_size(int M, int N, int K, int group_size);

#define WMMA_W4_KERNEL_DECODE_MFMA 0  /* M <= 4: one workgroup per 16 columns, matrix pipe */
#define WMMA_W4_KERNEL_DECODE 1       /* M <= 4, other group sizes: VALU dot products      */
#define WMMA_W4_KERNEL_GEMV_SPLIT 2   /* M <= 4, narrow N: 32 columns per workgroup, split-K */
#define WMMA_W4_KERNEL_MFMA 3         /* other shapes: tiled MFMA kernel                     */
#define WMMA_W4_KERNEL_SKINNY 4       /* 4 < M <= 32: 32/64 columns per workgroup, matrix pipe */
#define WMMA_W4_KERNEL_GEMM 5         /* M > 32: LDS-DMA MFMA GEMM                           */
#define WMMA_W4_KERNEL_ROWS 6         /* M > 4, short K or wide N: 16/32 rows x 16-64
                                         columns per workgroup over all of K, no LDS ring,
                                         no split                                          */

typedef struct wmma_w4a16_plan {
    int kernel;             /* WMMA_W4_KERNEL_*                                           */
    int split_k;            /* K partitions (1 = no split, no workspace)                  */
    int k_per_split;        /* K elements per partition                                   */
    size_t workspace_bytes; /* fp32 partial sums: split_k * M * N * 4, 0 when split_k==1  */
} wmma_w4a16_plan;

/* Host-only planner for wmma_w4a16_gemm on a device with `num_cus` compute units, for
 * 8-byte-aligned scales (the case of every torch allocation).  No reference counterpart;
 * the W4A16 analogue of wmma_gemm_plan_make. */
int wmma_w4a16_plan_make(int M, int N, int K, int group_size, int num_cus, wmma_w4a16_plan* out);

/*
 * Y[M,N] (fp32) = A[M,K] (fp16) @ W[K,N], W[k][n] = fp16((q[k][n] - z[k/G][n]) * s[k/G][n])
 * (dequantised value rounded once to fp16).  packed: output of wmma_int4_prepack.
 * scales: fp16 [K/G, N] (or [N/16][K/G][16] with WMMA_ZEROS_SLICED).  zeros: per
 * zeros_format.  G = group_size, G % 32 == 0, K % G == 0.  With WMMA_W4_FUSED, packed is
 * the output of wmma_int4_prepack_fused and scales / zeros are not read (may be NULL).
 * Arithmetic by path (wmma_w4a16_plan_make reports the path of a shape).  The tiled
 * kernels (WMMA_W4_KERNEL_SKINNY, _GEMM, _ROWS, _MFMA, _GEMV_SPLIT) and the decode kernel at
 * M = 3, 4 form each weight exactly as written above before its fp32-accumulated product.
 * Two decode paths form no per-weight fp16 value: WMMA_W4_KERNEL_DECODE_MFMA at M <= 2
 * and WMMA_W4_KERNEL_DECODE (M <= 4).  For each 128-deep (resp. 32-deep) K run inside a
 * group they accumulate the exact products a * (1024 + q) (a * (64 + q) at k % 8 in
 * {2,3,6,7}) and the activation sums in fp32 and add s * (D - P - z Q) once per run: the
 * same value up to fp32 rounding and the omitted fp16 rounding of each dequantised weight
 * (measured max relative error 2.2e-4 at K = 4096).  The bits of a row therefore depend
 * on the path M selects: row 0 of an M = 2 call can differ in the last bits from row 0 of
 * an M = 3 call (not batch-invariant across that boundary).  Every path is deterministic
 * (no atomics; a K split is summed in a fixed order).
 * No reference counterpart (BASELINE-defined W4A16 path).
 */
int wmma_w4a16_gemm(const void* A, int64_t lda, const int32_t* packed, const void* scales,
                    const void* zeros, int zeros_format, int M, int N, int K, int group_size,
                    float* Y, int64_t ldy, void* workspace, size_t workspace_bytes, void* stream);

/* The same with an fp16 Y (each fp32 result rounded once to fp16; split-K partials stay
 * fp32).  No reference counterpart: the fp16-output option of the W4A16 path. */
int wmma_w4a16_gemm_f16out(const void* A, int64_t lda, const int32_t* packed,
                           const void* scales, const void* zeros, int zeros_format, int M, int N,
                           int K, int group_size, void* Y, int64_t ldy, void* workspace,
                           size_t workspace_bytes, void* stream);

/*
 * AutoAWQ checkpoint tensors to this library's inputs, bit-exact: qweight_awq int32
 * [K, N/8] and qzeros_awq int32 [K/G, N/8], eight columns per word in AutoAWQ's nibble
 * order (column 8c + {0,2,4,6,1,3,5,7}[i] in nibble i) -> qweight int32 [K/8, N] (GPTQ
 * layout, for wmma_int4_prepack) and zeros int32 [K/G, N/8] (WMMA_ZEROS_PACKED).  AWQ's
 * scales fp16 [K/G, N] are already this library's layout.  No reference counterpart.
 */
int wmma_int4_from_awq(const int32_t* qweight_awq, const int32_t* qzeros_awq, int K, int N,
                       int group_size, int32_t* qweight, int32_t* zeros, void* stream);

/*
 * GPTQ checkpoint zero points to this library's packed zeros (WMMA_ZEROS_PACKED), bit-exact.
 * qzeros int32 [K/G, N/8] holds z[g][n] in nibble n%8 of word [g][n/8] -- the layout of
 * WMMA_ZEROS_PACKED -- but AutoGPTQ's "gptq" checkpoint format (WMMA_GPTQ_V1) packs z - 1
 * there and dequantises with (stored + 1); GPTQModel's "gptq_v2" format (WMMA_GPTQ_V2)
 * stores z.  zeros[g][n] = stored + 1 (v1) or stored (v2).  A v1 stored nibble of 15 means
 * z = 16 (the result of packing z = 0 as z - 1), which a 4-bit zero point cannot hold: its
 * nibble becomes 0 and *overflow, when overflow != NULL (device int32), is set to 1; the
 * call never clears *overflow, so the caller zeroes it first and checks it after.  GPTQ's
 * qweight [K/8, N] and scales [K/G, N] are this library's layout already.  No reference
 * counterpart.
 */
#define WMMA_GPTQ_V1 1
#define WMMA_GPTQ_V2 2
int wmma_int4_from_gptq_zeros(const int32_t* qzeros, int K, int N, int group_size,
                              int zero_format, int32_t* zeros, int32_t* overflow, void* stream);

/*
 * Act-order GPTQ checkpoints (desc_act, a g_idx that is not k / G): row k of the quantised
 * weights belongs to group g_idx[k].  With perm = a stable sort of the rows by g_idx (G rows
 * per group), qweight_out row k = qweight row perm[k] (GPTQ layout, int32 [K/8, N]; perm
 * int32 [K], entries clamped into [0, K)), so that the groups are contiguous again and
 * Y = A[:, perm] @ W_out equals A @ W.  No reference counterpart.
 */
int wmma_int4_permute_rows(const int32_t* qweight, const int32_t* perm, int K, int N,
                           int32_t* qweight_out, void* stream);

/*
 * Flash-attention forward.  Q [B,H,Sq,D], K and V [B,H,Sk,D], O [B,H,Sq,D]; fp16,
 * contiguous.  O = softmax(scale * Q K^T (+ causal mask: key j <= query i, aligned to
 * the top left for any Sq, Sk, as torch's scaled_dot_product_attention(is_causal=True)))
 * V, FP32 online softmax and accumulation.  D: a multiple of 8 from 8 to 256 for this and
 * every flash entry point below (other head dims return WMMA_ERR_UNSUPPORTED; the torch
 * layer zero-pads D to a multiple of 8).
 * A query row whose keys are all masked (i.e. none, since key 0 is always kept) cannot
 * occur.
 * Replaces the documented (unbound) flash_attention(Q,K,V,causal=False,scale=-1.0)
 * (README.md:221-251).  A caller's scale <= 0 is resolved to 1/sqrt(D) before this call.
 */
int wmma_flash_attn_fwd(const void* Q, const void* K, const void* V, void* O, int B, int H,
                        int Sq, int Sk, int D, float scale, int causal, void* stream);

/*
 * The same with grouped-query / multi-query attention: K and V are [B,Hkv,Sk,D] with
 * H % Hkv == 0, and query head h reads key/value head h / (H/Hkv) -- the head mapping of
 * torch's scaled_dot_product_attention(enable_gqa=True).  Hkv == H is
 * wmma_flash_attn_fwd.  No counterpart in the reference: its documented flash_attention
 * (README.md:221-251) takes equal head counts; this is the grouped-query extension of
 * that API.
 */
int wmma_flash_attn_fwd_gqa(const void* Q, const void* K, const void* V, void* O, int B, int H,
                            int Hkv, int Sq, int Sk, int D, float scale, int causal,
                            void* stream);

/*
 * Variable-length (packed) batches: Q and O [total_q, H, D], K and V [total_k, Hkv, D]
 * fp16; sequence b is rows cu_seqlens_q[b] .. cu_seqlens_q[b+1] of Q/O and
 * cu_seqlens_k[b] .. cu_seqlens_k[b+1] of K/V (int32 [B+1], device memory, non-decreasing,
 * lengths at most max_seqlen_q / max_seqlen_k).  Causal masking is top-left aligned per
 * sequence, as in wmma_flash_attn_fwd; a query row of a sequence with no keys gets zeros.
 * Offsets outside [0, total] are clamped, so inconsistent cu_seqlens give wrong rows, never
 * an access outside the tensors.  No counterpart in the reference: the variable-length
 * extension of its documented flash_attention (README.md:221-251).
 */
int wmma_flash_attn_varlen_fwd(const void* Q, const void* K, const void* V, void* O,
                               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k, int B,
                               int H, int Hkv, int total_q, int total_k, int max_seqlen_q,
                               int max_seqlen_k, int D, float scale, int causal, void* stream);

/*
 * Forward for training: wmma_flash_attn_fwd_gqa that also writes lse [B,H,Sq] fp32, the
 * natural-log log-sum-exp of each row of scale * Q K^T over its unmasked keys (+inf for a
 * row with none), which wmma_flash_attn_bwd consumes.  lse may be NULL (no output).  No
 * counterpart in the reference, whose documented flash_attention (README.md:221-251) is
 * forward-only; this and the entry points below are its training extension.
 */
int wmma_flash_attn_fwd_lse(const void* Q, const void* K, const void* V, void* O, float* lse,
                            int B, int H, int Hkv, int Sq, int Sk, int D, float scale, int causal,
                            void* stream);

/*
 * wmma_flash_attn_fwd_lse with a workspace.  When the (batch, head, 256-query block)
 * workgroups would leave more than half the GPU's CUs idle -- decoding: few queries against
 * many keys -- the key range is split over more workgroups, each writing its chunk's
 * unnormalised output, running max and row sum to the workspace, and a second kernel
 * merges them (results within fp32 rounding of the one-pass forward, not bit-identical).
 * workspace: at least wmma_flash_attn_fwd_workspace_size(...) bytes (same shape and causal
 * flag), 16-byte aligned, or NULL / smaller: the one-pass forward.  Every dense forward
 * (this one, wmma_flash_attn_fwd_lse / _gqa / wmma_flash_attn_fwd) runs the query heads
 * of a grouped-query group as one sequence when there is no causal mask, so each K/V tile
 * is read once per group (bit-identical results).  No counterpart in the reference (its
 * flash_attention, README.md:221-251, has no decoding path).
 */
size_t wmma_flash_attn_fwd_workspace_size(int B, int H, int Hkv, int Sq, int Sk, int D,
                                          int causal);
int wmma_flash_attn_fwd_ws(const void* Q, const void* K, const void* V, void* O, float* lse,
                           int B, int H, int Hkv, int Sq, int Sk, int D, float scale, int causal,
                           void* workspace, size_t workspace_bytes, void* stream);

/* The variable-length forward with lse [H, total_q] (row r of head h at h * total_q + r). */
int wmma_flash_attn_varlen_fwd_lse(const void* Q, const void* K, const void* V, void* O,
                                   float* lse, const int32_t* cu_seqlens_q,
                                   const int32_t* cu_seqlens_k, int B, int H, int Hkv,
                                   int total_q, int total_k, int max_seqlen_q, int max_seqlen_k,
                                   int D, float scale, int causal, void* stream);

/*
 * Bytes of fp32 workspace wmma_flash_attn_bwd needs: 2 * 4 * B * H * Sq (two row
 * statistics per query row).  For the variable-length backward pass B = 1, Sq = total_q.
 */
size_t wmma_flash_attn_bwd_workspace_size(int B, int H, int Sq);

/*
 * Workspace bytes with which wmma_flash_attn_bwd (dense layout, same shape and causal flag)
 * also splits a grouped-query group's query heads over more dK/dV workgroups, for shapes
 * whose dK/dV workgroups would fill less than half of one wave of the CUs, or with a causal
 * mask at most one wave (its first key blocks carry twice the average work): the row
 * statistics rounded up to 256 bytes, then fp32 partial dK and dV per part, added by a
 * second kernel in part order (deterministic; within fp32 rounding of the unsplit pass).
 * Equals wmma_flash_attn_bwd_workspace_size(B, H, Sq) when no split applies; any workspace
 * of at least that size (16-byte aligned for the split) works, a smaller one than this
 * runs unsplit.  No counterpart in the reference.
 */
size_t wmma_flash_attn_bwd_split_workspace_size(int B, int H, int Hkv, int Sq, int Sk, int D,
                                                int causal);

/*
 * Flash-attention backward.  Given dO [B,H,Sq,D] and the forward's Q, K, V, O and lse
 * (from wmma_flash_attn_fwd_lse with the same scale and causal flag), writes dQ [B,H,Sq,D],
 * dK and dV [B,Hkv,Sk,D], fp16, the gradients of sum(O * dO): with P = softmax(scale Q K^T
 * + mask), dV = P^T dO, dS = P o (dO V^T - rowsum(dO o O)), dQ = scale dS K,
 * dK = scale dS^T Q; with Hkv < H, dK and dV of a key/value head are summed over the query
 * heads that read it.  FP32 accumulation throughout; deterministic (no atomics; the same
 * inputs give the same bits).  Sq == 0 gives dK = dV = 0.  workspace: at least
 * wmma_flash_attn_bwd_workspace_size(B, H, Sq) bytes, 4-byte aligned, overwritten.
 * Two kernels on `stream`.  No counterpart in the reference (its flash_attention,
 * README.md:221-251, is forward-only).
 */
int wmma_flash_attn_bwd(const void* dO, const void* Q, const void* K, const void* V, const void* O,
                        const float* lse, void* dQ, void* dK, void* dV, void* workspace,
                        size_t workspace_bytes, int B, int H, int Hkv, int Sq, int Sk, int D,
                        float scale, int causal, void* stream);

/*
 * The variable-length backward pass: dO, dQ as Q [total_q, H, D]; dK, dV as K [total_k,
 * Hkv, D]; lse [H, total_q] from wmma_flash_attn_varlen_fwd_lse; workspace of
 * wmma_flash_attn_bwd_workspace_size(1, H, total_q) bytes.  A sequence with no keys gets
 * dQ = 0, one with no queries dK = dV = 0; rows outside every sequence are not written.
 */
int wmma_flash_attn_varlen_bwd(const void* dO, const void* Q, const void* K, const void* V,
                               const void* O, const float* lse, void* dQ, void* dK, void* dV,
                               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                               void* workspace, size_t workspace_bytes, int B, int H, int Hkv,
                               int total_q, int total_k, int max_seqlen_q, int max_seqlen_k,
                               int D, float scale, int causal, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* WMMA_OPS_AMD_H */
