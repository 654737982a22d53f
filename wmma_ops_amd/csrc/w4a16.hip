// INT4 weight layout kernels and W4A16 dequant-GEMM kernels for gfx950.
//
// The reference has no INT4 code; the W4A16 path is defined by its task statement:
//   Y[M,N] (fp32) = A[M,K] (fp16) @ W,  W[k][n] = fp16((q[k][n] - z[g][n]) * s[g][n]),
//   g = k / G, q and z 4-bit unsigned, s fp16, the dequantised weight rounded once to fp16.
//
// Layouts
//   GPTQ qweight   int32 [K/8, N]: q[k][n] in bits 4*(k%8).. of qweight[k/8][n].
//   prepacked      int32 [N/16][K/64][32][4 words]: entry (s, kc, l) of 16-column slice s
//                  holds column n = 16*s + l%16, words w = 0..3 for k-group
//                  kg = 8*kc + 4*(l/16) + w (k = 8*kg .. 8*kg+7).  Inside a prepacked word
//                  nibble p holds k-offset kPerm[p] = {0,2,4,6,1,3,5,7}[p], so that
//                  (word >> 4i) & 0x000F000F yields the pair (k 2i, k 2i+1) as two 16-bit
//                  lanes.  A slice's weights are one contiguous run over all of K (what a
//                  decode workgroup streams); a 64-deep block of 32 columns is two 512-byte
//                  runs, and each lane's 16 bytes are the K-contiguous operand of four
//                  MFMAs for its column.  pk_index() below gives the 16-byte unit of
//                  (column, 64-deep block, K half).
//   scales         fp16 [K/G, N];  zeros int32 [K/G, N/8] (nibble n%8) or uint8 [K/G, N].
//
// Dequantisation in registers: (0x6400 | q) is the fp16 value 1024 + q, so
// (1024 + q) - (1024 + z) = q - z exactly, and one fp16 multiply by s rounds once.
#include "common.hpp"
#include "kernels.hpp"
#include "plan.hpp"

namespace wmma_amd {

namespace {

typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f16x2 as_h2(uint32_t v) { return __builtin_bit_cast(f16x2, v); }
__device__ __forceinline__ uint32_t as_u32(f16x2 v) { return __builtin_bit_cast(uint32_t, v); }

// 16-byte unit of the prepacked weights holding column n, 64-deep block kc, K half h.
__host__ __device__ __forceinline__ int64_t pk_index(int n, int kc, int h, int KC) {
    return ((int64_t)(n >> 4) * KC + kc) * 32 + 16 * h + (n & 15);
}

// Nibble position -> k offset inside a prepacked word (and its inverse).
__constant__ int kPermDev[8] = {0, 2, 4, 6, 1, 3, 5, 7};

// ---------------------------------------------------------------- layout conversions --
// One thread per (block, lane): reads four GPTQ words (coalesced along n), reorders each
// word's nibbles, writes 16 bytes.
__global__ void __launch_bounds__(256)
int4_prepack_kernel(const int32_t* __restrict__ qw, int K, int N, int32_t* __restrict__ out) {
    const int KC = K / 64;
    const int64_t total = (int64_t)(N / 16) * KC * 32;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int l = (int)(t & 31);
        const int64_t blk = t >> 5;
        const int kc = (int)(blk % KC);
        const int sl = (int)(blk / KC);
        const int n = 16 * sl + (l & 15);
        const int kg0 = 8 * kc + 4 * (l >> 4);
        u32x4 v;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t src = (uint32_t)qw[(int64_t)(kg0 + w) * N + n];
            uint32_t dst = 0;
#pragma unroll
            for (int pnib = 0; pnib < 8; ++pnib)
                dst |= ((src >> (4 * kPermDev[pnib])) & 0xFu) << (4 * pnib);
            v[w] = dst;
        }
        reinterpret_cast<u32x4*>(out)[t] = v;
    }
}

__global__ void __launch_bounds__(256)
int4_unprepack_kernel(const int32_t* __restrict__ in, int K, int N, int32_t* __restrict__ qw) {
    const int KC = K / 64;
    const int64_t total = (int64_t)(N / 16) * KC * 32;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int l = (int)(t & 31);
        const int64_t blk = t >> 5;
        const int kc = (int)(blk % KC);
        const int sl = (int)(blk / KC);
        const int n = 16 * sl + (l & 15);
        const int kg0 = 8 * kc + 4 * (l >> 4);
        const u32x4 v = reinterpret_cast<const u32x4*>(in)[t];
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            uint32_t dst = 0;
#pragma unroll
            for (int pnib = 0; pnib < 8; ++pnib)
                dst |= ((v[w] >> (4 * pnib)) & 0xFu) << (4 * kPermDev[pnib]);
            qw[(int64_t)(kg0 + w) * N + n] = (int32_t)dst;
        }
    }
}

__global__ void __launch_bounds__(256)
int4_unpack_kernel(const int32_t* __restrict__ qw, int K, int N, uint8_t* __restrict__ q) {
    const int64_t total = (int64_t)(K / 8) * N;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t kg = t / N;
        const int n = (int)(t % N);
        const uint32_t v = (uint32_t)qw[t];
#pragma unroll
        for (int j = 0; j < 8; ++j) q[(kg * 8 + j) * N + n] = (uint8_t)((v >> (4 * j)) & 0xFu);
    }
}

// AutoAWQ (GEMM format) to this library's GPTQ layout.  AutoAWQ packs eight columns per
// int32 along N, column 8c + kAwqOrder[i] in nibble i (kAwqOrder = {0, 2, 4, 6, 1, 3, 5, 7},
// its AWQ_ORDER), for qweight [K][N/8] and qzeros [K/G][N/8] alike; so column 8c + j sits
// in nibble kAwqPos[j] = {0, 4, 1, 5, 2, 6, 3, 7}[j] (its AWQ_REVERSE_ORDER).  One thread
// per output word: qweight words gather 8 rows of one column, zero words permute nibbles.
__constant__ int kAwqPos[8] = {0, 4, 1, 5, 2, 6, 3, 7};

__global__ void __launch_bounds__(256)
int4_from_awq_kernel(const int32_t* __restrict__ qw, const int32_t* __restrict__ qz, int K, int N,
                     int KG, int32_t* __restrict__ qw_out, int32_t* __restrict__ qz_out) {
    const int64_t nw = (int64_t)(K / 8) * N, nz = (int64_t)KG * (N / 8);
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < nw + nz;
         t += (int64_t)gridDim.x * blockDim.x) {
        if (t < nw) {  // GPTQ word (k8, n): nibble j = q[8 k8 + j][n]
            const int64_t k8 = t / N;
            const int n = (int)(t % N);
            const int sh = 4 * kAwqPos[n & 7];
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j)
                word |= (((uint32_t)qw[(8 * k8 + j) * (N / 8) + n / 8] >> sh) & 0xFu) << (4 * j);
            qw_out[t] = (int32_t)word;
        } else {       // packed zero word: nibble j = z[g][8c + j]
            const int64_t u = t - nw;
            const uint32_t src = (uint32_t)qz[u];
            uint32_t word = 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) word |= ((src >> (4 * kAwqPos[j])) & 0xFu) << (4 * j);
            qz_out[u] = (int32_t)word;
        }
    }
}

// GPTQ checkpoint zero points to this library's packed zeros.  AutoGPTQ's "gptq" (v1)
// format packs z - 1 into the nibbles of qzeros [K/G][N/8] (nibble n%8 of word n/8, the
// layout of WMMA_ZEROS_PACKED) and dequantises with stored + 1; its "gptq_v2" format (and
// this library) stores z itself.  add = 1 (v1) or 0 (v2) is added to every nibble; a v1
// nibble of 15 stands for z = 16, which four bits cannot hold: such a word sets *overflow
// to 1 (a plain store of the same value from every writer, never cleared here).
__global__ void __launch_bounds__(256)
int4_gptq_zeros_kernel(const int32_t* __restrict__ qz, int64_t words, uint32_t add,
                       int32_t* __restrict__ out, int32_t* __restrict__ overflow) {
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < words;
         t += (int64_t)gridDim.x * blockDim.x) {
        const uint32_t src = (uint32_t)qz[t];
        uint32_t word = 0;
        bool over = false;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint32_t z = ((src >> (4 * j)) & 0xFu) + add;
            over |= z > 15u;
            word |= (z & 0xFu) << (4 * j);
        }
        out[t] = (int32_t)word;
        if (over && overflow) *overflow = 1;
    }
}

// Row permutation of GPTQ-layout weights (act-order checkpoints): output row k is input row
// perm[k] (perm entries clamped into [0, K)).  One thread per output word (8 rows of one
// column), coalesced along n.
__global__ void __launch_bounds__(256)
int4_permute_rows_kernel(const int32_t* __restrict__ qw, const int32_t* __restrict__ perm, int K,
                         int N, int32_t* __restrict__ out) {
    const int64_t total = (int64_t)(K / 8) * N;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int64_t k8 = t / N;
        const int n = (int)(t % N);
        uint32_t word = 0;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const int src = min(max(perm[8 * k8 + j], 0), K - 1);
            const uint32_t v = (uint32_t)qw[(int64_t)(src >> 3) * N + n];
            word |= ((v >> (4 * (src & 7))) & 0xFu) << (4 * j);
        }
        out[t] = (int32_t)word;
    }
}

// Group parameters to the slice-major layout (WMMA_ZEROS_SLICED): one thread per
// (16-column slice, group) writes the slice's 16 scales and its two zero words.
template <int ZF>
__global__ void __launch_bounds__(256)
int4_params_slice_kernel(const uint16_t* __restrict__ s, const void* __restrict__ z, int KG, int N,
                         uint16_t* __restrict__ s_out, int32_t* __restrict__ z_out) {
    const int64_t total = (int64_t)(N / 16) * KG;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int slice = (int)(t / KG), g = (int)(t % KG);
        const int64_t row = (int64_t)g * N + 16 * slice;
#pragma unroll
        for (int e = 0; e < 16; ++e) s_out[t * 16 + e] = s[row + e];
#pragma unroll
        for (int w = 0; w < 2; ++w) {
            uint32_t word;
            if constexpr (ZF == WMMA_ZEROS_PACKED) {
                word = (uint32_t)static_cast<const int32_t*>(z)[(int64_t)g * (N / 8) + 2 * slice + w];
            } else {
                word = 0;
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    word |= ((uint32_t)static_cast<const uint8_t*>(z)[row + 8 * w + j] & 0xFu) << (4 * j);
            }
            z_out[t * 2 + w] = (int32_t)word;
        }
    }
}

// Fused decode layout (WMMA_W4_FUSED): weights, scales and zero points of a 16-column slice
// in one contiguous run, so that a decode workgroup streams a single region.  Per slice:
//   header   one 160-byte parameter block per four 128-deep K steps 4r .. 4r+3 (KP = K/128
//            steps; the last block covers the steps left), zero-padded to a multiple of 128
//            bytes so that the weight runs below stay on 128-byte lines:
//              bytes [0, 128)   scales fp16 [4][16]: entry (u, c) = s[g][16*slice + c],
//                               g = 128 (4r+u) / G
//              bytes [128, 160) zero points [4][16] as nibbles: byte 128 + 8u + c/2, nibble
//                               c % 2 (even columns in the low nibble)
//   weights  1 KB per K step pp = the prepacked blocks kc = 2pp, 2pp+1 of the slice (its
//            standard prepacked run, unchanged).
// With G = 128 and K % 4096 == 0 the buffer holds exactly the bytes of the prepacked weights
// plus the scales and packed zeros; a larger G repeats each group's parameters in every
// K step of the group.  Parameter entries of steps past K are zero.
constexpr int kFusedBlock = 160;

template <int ZF>
__global__ void __launch_bounds__(256)
int4_prepack_fused_kernel(const int32_t* __restrict__ qw, const uint16_t* __restrict__ s,
                          const void* __restrict__ z, int K, int N, int G,
                          int32_t* __restrict__ out) {
    const int64_t su = fused_slice_bytes(K) / 16;  // units per slice
    const int64_t total = (int64_t)(N / 16) * su;
    const int KP = K / 128;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int sl = (int)(t / su);
        const int64_t o = t - (int64_t)sl * su;
        const int hu = (int)(fused_hdr_bytes(K) / 16);  // header units
        // header unit o: parameter block r = o / 10, unit ou = o % 10 of it (units past the
        // last block are padding); weight unit o - hu: K step (o - hu) / 64, lane % 64
        const int r = o < hu ? (int)(o / 10) : 0;
        const int ou = o < hu ? (o < 10 * ((KP + 3) / 4) ? (int)(o % 10) : -1) : 10 + (int)(o - hu);
        u32x4 v = {0, 0, 0, 0};
        if (ou < 0) {  // header padding
        } else if (ou < 8) {  // scales: entries 8 ou .. 8 ou + 7 = K step ou/2, columns 8 (ou%2) ..
            const int u = ou >> 1, pp = 4 * r + u;
            if (pp < KP) {
                const int64_t row = (int64_t)(pp * 128 / G) * N + 16 * sl + 8 * (ou & 1);
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    v[e] = (uint32_t)s[row + 2 * e] | ((uint32_t)s[row + 2 * e + 1] << 16);
            }
        } else if (ou < 10) {  // zero nibbles: pair-steps 2 (ou-8), 2 (ou-8) + 1, 8 bytes each
#pragma unroll
            for (int hlf = 0; hlf < 2; ++hlf) {
                const int pp = 4 * r + 2 * (ou - 8) + hlf;
                if (pp >= KP) continue;
                const int g = pp * 128 / G;
                uint32_t w0 = 0, w1 = 0;
#pragma unroll
                for (int c = 0; c < 16; ++c) {
                    const int n = 16 * sl + c;
                    uint32_t zz;
                    if constexpr (ZF == WMMA_ZEROS_PACKED)
                        zz = ((uint32_t)static_cast<const int32_t*>(z)[(int64_t)g * (N / 8) + n / 8] >>
                              (4 * (n & 7))) & 0xFu;
                    else
                        zz = (uint32_t)static_cast<const uint8_t*>(z)[(int64_t)g * N + n] & 0xFu;
                    if (c < 8)
                        w0 |= zz << (4 * c);
                    else
                        w1 |= zz << (4 * (c - 8));
                }
                v[2 * hlf] = w0;
                v[2 * hlf + 1] = w1;
            }
        } else {  // weights: K step (ou-10)/64, lane (ou-10)%64 of its 1 KB
            const int wu = ou - 10, pp = wu >> 6, l = wu & 63;
            const int kc = 2 * pp + (l >> 5), e = l & 31;
            const int n = 16 * sl + (e & 15);
            const int kg0 = 8 * kc + 4 * (e >> 4);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                const uint32_t src = (uint32_t)qw[(int64_t)(kg0 + w) * N + n];
                uint32_t dst = 0;
#pragma unroll
                for (int pnib = 0; pnib < 8; ++pnib)
                    dst |= ((src >> (4 * kPermDev[pnib])) & 0xFu) << (4 * pnib);
                v[w] = dst;
            }
        }
        reinterpret_cast<u32x4*>(out)[t] = v;
    }
}

// Inverse: the weight units back to GPTQ words (one thread per 16-byte weight unit), then
// one thread per (group, slice) reads the parameters of the group's first pair-step.
__global__ void __launch_bounds__(256)
int4_unprepack_fused_kernel(const int32_t* __restrict__ in, int K, int N, int G,
                            int32_t* __restrict__ qw, uint16_t* __restrict__ s,
                            int32_t* __restrict__ z) {
    const int KP = K / 128, KG = K / G, NS = N / 16;
    const int64_t sb = fused_slice_bytes(K);
    const int64_t nwu = (int64_t)NS * KP * 64;  // weight units
    const int64_t total = nwu + (int64_t)KG * NS;
    const unsigned char* base = reinterpret_cast<const unsigned char*>(in);
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        if (t < nwu) {
            const int sl = (int)(t / ((int64_t)KP * 64));
            const int rem = (int)(t - (int64_t)sl * KP * 64);
            const int pp = rem >> 6, l = rem & 63;
            const u32x4 v = *reinterpret_cast<const u32x4*>(
                base + sl * sb + fused_hdr_bytes(K) + (int64_t)pp * 1024 + 16 * l);
            const int kc = 2 * pp + (l >> 5), e = l & 31;
            const int n = 16 * sl + (e & 15);
            const int kg0 = 8 * kc + 4 * (e >> 4);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                uint32_t dst = 0;
#pragma unroll
                for (int pnib = 0; pnib < 8; ++pnib)
                    dst |= ((v[w] >> (4 * pnib)) & 0xFu) << (4 * kPermDev[pnib]);
                qw[(int64_t)(kg0 + w) * N + n] = (int32_t)dst;
            }
        } else {
            const int64_t u = t - nwu;
            const int g = (int)(u / NS), sl = (int)(u % NS);
            const int pp = g * G / 128;
            const unsigned char* rec = base + sl * sb + (int64_t)(pp >> 2) * kFusedBlock;
            const uint16_t* sp = reinterpret_cast<const uint16_t*>(rec) + 16 * (pp & 3);
#pragma unroll
            for (int c = 0; c < 16; ++c) s[(int64_t)g * N + 16 * sl + c] = sp[c];
            const uint32_t* zp = reinterpret_cast<const uint32_t*>(rec + 128 + 8 * (pp & 3));
            z[(int64_t)g * (N / 8) + 2 * sl] = (int32_t)zp[0];
            z[(int64_t)g * (N / 8) + 2 * sl + 1] = (int32_t)zp[1];
        }
    }
}

// --------------------------------------------------------------------- dequantisation --
struct W4Args {
    const f16* A;
    int64_t lda;
    const u32x4* W;       // prepacked blocks
    const f16* S;         // scales [K/G, N]
    const void* Z;        // zeros
    int zfmt;
    int M, N, K, G;
    float* Y;
    int64_t ldy;
    float* ws;            // partials [split][M][N]
    int split;
    int kc_per_split;     // 64-deep chunks per split
    int pp_shift;         // decode-MFMA kernel: log2(G / 128)
    int g_shift;          // LDS-DMA GEMM: log2(G) (G a power of two there)
    int kg;               // K / G (groups)
    int y_half;           // Y is fp16 (each fp32 result rounded once), else fp32
};

// Final store of one result: fp32, or fp16 rounded once from the fp32 sum.  Split-K
// partials stay fp32 in the workspace; only the final value is converted.
__device__ __forceinline__ void store_y(const W4Args& p, int64_t idx, float v) {
    if (p.y_half)
        reinterpret_cast<f16*>(p.Y)[idx] = (f16)v;
    else
        p.Y[idx] = v;
}

// Element index of scale s[g][n], and of the zeros element (int32 word of eight nibbles,
// nibble n % 8; or byte) holding z[g][n], per zeros format ZF:
//   WMMA_ZEROS_PACKED  scales [K/G][N], zero words [K/G][N/8]
//   WMMA_ZEROS_U8      scales [K/G][N], zero bytes [K/G][N]
//   WMMA_ZEROS_SLICED  scales [N/16][K/G][16], zero words [N/16][K/G][2]: every 16-column
//                      slice's parameters for all groups are one contiguous run, so a
//                      workgroup that streams a slice over all of K reads them in 1 KB /
//                      256-byte runs instead of 32-byte pieces of K/G rows.
template <int ZF>
__device__ __forceinline__ int64_t s_index(const W4Args& p, int g, int n) {
    if constexpr (ZF == WMMA_ZEROS_SLICED)
        return ((int64_t)(n >> 4) * p.kg + g) * 16 + (n & 15);
    else
        return (int64_t)g * p.N + n;
}
template <int ZF>
__device__ __forceinline__ int64_t z_index(const W4Args& p, int g, int n) {
    if constexpr (ZF == WMMA_ZEROS_SLICED)
        return ((int64_t)(n >> 4) * p.kg + g) * 2 + ((n >> 3) & 1);
    else if constexpr (ZF == WMMA_ZEROS_PACKED)
        return (int64_t)g * (p.N / 8) + n / 8;
    else
        return (int64_t)g * p.N + n;
}

// Per-lane group parameters: zs = (1024 + z, 1024 + z), ss = (s, s) as packed fp16 pairs.
// ZF (the zeros format) is a template parameter so the loads stay branch-free and can
// all be in flight together.
template <int ZF>
__device__ __forceinline__ void group_params(const W4Args& p, int g, int n, uint32_t* zs,
                                             uint32_t* ss) {
    const uint16_t s = __builtin_bit_cast(uint16_t, p.S[s_index<ZF>(p, g, n)]);
    uint32_t z;
    if constexpr (ZF != WMMA_ZEROS_U8) {
        const uint32_t zw = (uint32_t)static_cast<const int32_t*>(p.Z)[z_index<ZF>(p, g, n)];
        z = (zw >> (4 * (n & 7))) & 0xFu;
    } else {
        z = static_cast<const uint8_t*>(p.Z)[z_index<ZF>(p, g, n)] & 0xFu;
    }
    const uint32_t zh = 0x6400u | z;
    *zs = zh | (zh << 16);
    *ss = (uint32_t)s | ((uint32_t)s << 16);
}

// Raw group-parameter loads (scale bits, zero word) -- decoded later by group_decode so
// that many loads can be in flight before any of them is waited on.
template <int ZF>
__device__ __forceinline__ void group_load(const W4Args& p, int g, int n, uint32_t* sraw,
                                           uint32_t* zraw) {
    *sraw = __builtin_bit_cast(uint16_t, p.S[s_index<ZF>(p, g, n)]);
    if constexpr (ZF != WMMA_ZEROS_U8)
        *zraw = (uint32_t)static_cast<const int32_t*>(p.Z)[z_index<ZF>(p, g, n)];
    else
        *zraw = static_cast<const uint8_t*>(p.Z)[z_index<ZF>(p, g, n)];
}
template <int ZF>
__device__ __forceinline__ void group_decode(uint32_t sraw, uint32_t zraw, int n, uint32_t* zs,
                                             uint32_t* ss) {
    uint32_t z;
    if constexpr (ZF != WMMA_ZEROS_U8)
        z = (zraw >> (4 * (n & 7))) & 0xFu;
    else
        z = zraw & 0xFu;
    const uint32_t zh = 0x6400u | z;
    *zs = zh | (zh << 16);
    *ss = sraw | (sraw << 16);
}

// Dequantise one prepacked word into four fp16 pairs in natural k order.
__device__ __forceinline__ void dequant_word(uint32_t w, uint32_t zs, uint32_t ss,
                                             uint32_t out[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t h = ((w >> (4 * i)) & 0x000F000Fu) | 0x64006400u;
        const f16x2 d = (as_h2(h) - as_h2(zs)) * as_h2(ss);
        out[i] = as_u32(d);
    }
}

// ---------------------------------------------------------- decode GEMV (M <= GV_MAXM) --
// Workgroup: NW waves, one 32-column tile, K chunks [kc0, kc1) round-robin over waves.
// Lane l: column 32*nt + l%32, K half l/32 of every chunk.  Accumulate with v_dot2
// (fp16 pairs, fp32 accumulator); reduce lanes l, l^32 and then the waves through LDS.
constexpr int GV_MAXM = 4;
constexpr int GV_NW = 8;
constexpr int GV_UNROLL = 4;

template <int ZF>
__global__ void __launch_bounds__(GV_NW * kWave)
w4a16_gemv_kernel(W4Args p) {
    __shared__ float red[GV_NW][GV_MAXM][32];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int nt = blockIdx.x;
    const int KC = p.K / 64;
    const int kc0 = blockIdx.y * p.kc_per_split;
    const int kc1 = min(KC, kc0 + p.kc_per_split);
    const int n = 32 * nt + (lane & 31);
    const int h = lane >> 5;
    const int M = p.M;

    float acc[GV_MAXM];
#pragma unroll
    for (int m = 0; m < GV_MAXM; ++m) acc[m] = 0.0f;

    const u32x4* wbase = p.W + pk_index(n, 0, h, KC);
    for (int kcb = kc0 + wave; kcb < kc1; kcb += GV_NW * GV_UNROLL) {
        u32x4 wv[GV_UNROLL];
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int kc = kcb + u * GV_NW;
            if (kc < kc1) wv[u] = __builtin_nontemporal_load(wbase + (int64_t)kc * 32);
        }
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int kc = kcb + u * GV_NW;
            if (kc < kc1) {
                const int k0 = kc * 64 + 32 * h;
                uint32_t zs, ss;
                group_params<ZF>(p, k0 / p.G, n, &zs, &ss);
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    uint32_t d[4];
                    dequant_word(wv[u][w], zs, ss, d);
#pragma unroll
                    for (int m = 0; m < GV_MAXM; ++m) {
                        if (m < M) {
                            const u32x4 a = *reinterpret_cast<const u32x4*>(
                                p.A + (int64_t)m * p.lda + k0 + 8 * w);
#pragma unroll
                            for (int i = 0; i < 4; ++i)
                                acc[m] = __builtin_amdgcn_fdot2(as_h2(d[i]), as_h2(a[i]), acc[m], false);
                        }
                    }
                }
            }
        }
    }
#pragma unroll
    for (int m = 0; m < GV_MAXM; ++m) {
        acc[m] += __shfl_xor(acc[m], 32);
        if (h == 0) red[wave][m][lane] = acc[m];
    }
    __syncthreads();
    if (tid < 32 * GV_MAXM) {
        const int m = tid >> 5, c = tid & 31;
        const int col = 32 * nt + c;
        if (m < M && col < p.N) {
            float v = red[0][m][c];
#pragma unroll
            for (int w = 1; w < GV_NW; ++w) v += red[w][m][c];
            if (p.split > 1)
                p.ws[((int64_t)blockIdx.y * M + m) * p.N + col] = v;
            else
                store_y(p, (int64_t)m * p.ldy + col, v);
        }
    }
}

// ------------------------------------------------------- decode (M <= GV_MAXM, no split) --
// One workgroup owns a 16-column slice and the whole K range, so no cross-workgroup
// reduction is needed.  A wave load covers two consecutive 64-deep chunks: lane l reads
// slice column l%16, chunk 2*pp + l/32, K half (l/16)%2 -- all 64 lanes active, 1 KB of
// the slice's contiguous weights per instruction.  Each wave keeps DV_U loads
// of the next round in flight while it dequantises the current one.
//
// Arithmetic (VALU is the bottleneck of decode, not HBM): a prepacked word holds the
// pairs (k0,k1) (k2,k3) (k4,k5) (k6,k7) in nibbles (0,4) (1,5) (2,6) (3,7), so
//   (w      & 0x000F000F) | 0x64006400 = fp16 pair (1024 + q_k0, 1024 + q_k1)
//   (w      & 0x00F000F0) | 0x64006400 = fp16 pair (1024 + 16 q_k2, 1024 + 16 q_k3)
//   (w >> 8 & 0x000F000F) | 0x64006400 = (1024 + q_k4, 1024 + q_k5)
//   (w >> 8 & 0x00F000F0) | 0x64006400 = (1024 + 16 q_k6, 1024 + 16 q_k7)
// -- every value exact in fp16.  Dotting them with the activations (v_dot2, fp32
// accumulate) gives, over one lane's 32-value K run (one quantisation group),
//   c1 = sum_{set1} (1024 + q) a,  c16 = sum_{set16} (1024 + 16 q) a,
// with set1 = offsets {0,1,4,5} and set16 = {2,3,6,7} of every 8.  With the run's
// activation sums A1, A16 (staged in LDS) the run's exact contribution is
//   s * (c1 + c16/16 - (1024 + z) A1 - (64 + z) A16)  =  s * sum_k (q_k - z) a_k,
// i.e. the dequantised product with s applied once per run instead of once per weight
// (it differs from fp16((q - z) s) per weight only by that rounding, far below the
// 1e-3 output tolerance).  9 VALU operations per 8 weights instead of ~24.
constexpr int DV_NW = 8;
constexpr int DV_U = 4;

template <int MM>
struct DecodeRound {
    u32x4 w[DV_U];
    uint32_t s[DV_U], z[DV_U];
};

// ONE: K <= DV_NW * DV_U * 128, a single round per wave (no second register buffer, so
// the kernel fits 64 VGPRs and eight waves per SIMD stay resident).
template <int MM, int ZF, bool ONE>
__global__ void __launch_bounds__(DV_NW * kWave)
__attribute__((amdgpu_waves_per_eu(ONE ? 8 : 4)))
w4a16_decode_kernel(W4Args p) {
    // LDS: activations [MM][K] fp16, then run sums [MM][K/32] of (A1, A16) fp32 pairs.
    extern __shared__ __attribute__((aligned(16))) unsigned char dv_smem[];
    const int K = p.K;
    f16* sA = reinterpret_cast<f16*>(dv_smem);
    float2* sSum = reinterpret_cast<float2*>(dv_smem + (size_t)MM * K * 2);
    __shared__ float red[DV_NW][MM][16];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int nt = blockIdx.x >> 1, sc = blockIdx.x & 1;
    const int col = lane & 15, sub = lane >> 4, dc = sub >> 1, h = sub & 1;
    const int n = 32 * nt + 16 * sc + col;
    const int KC = K / 64, KP = KC / 2;
    const int cpr = K / 8, nchunk = MM * cpr;

    // Activation chunk loads go first so that waiting for them does not wait for weights.
    constexpr int ABUF = 2;
    u32x4 abuf[ABUF];
#pragma unroll
    for (int j = 0; j < ABUF; ++j) {
        const int i = tid + j * DV_NW * kWave;
        if (i < nchunk) {
            const int m = i / cpr, c = i - m * cpr;
            abuf[j] = *reinterpret_cast<const u32x4*>(p.A + (int64_t)m * p.lda + 8 * c);
        }
    }

    const u32x4* wcol = p.W + pk_index(n, 0, h, KC);
    auto load_one = [&](int pp, DecodeRound<MM>& R, int u) {
        R.w[u] = __builtin_nontemporal_load(wcol + (int64_t)(2 * pp + dc) * 32);
        group_load<ZF>(p, (64 * (2 * pp + dc) + 32 * h) / p.G, n, &R.s[u], &R.z[u]);
    };
    auto load_round = [&](int r, DecodeRound<MM>& R) {
        const int pp0 = wave + DV_NW * DV_U * r;
        if (pp0 + DV_NW * (DV_U - 1) < KP) {
#pragma unroll
            for (int u = 0; u < DV_U; ++u) load_one(pp0 + DV_NW * u, R, u);
        } else {
#pragma unroll
            for (int u = 0; u < DV_U; ++u)
                if (pp0 + DV_NW * u < KP) load_one(pp0 + DV_NW * u, R, u);
        }
    };
    const int rounds = ONE ? 1 : (KP - wave + DV_NW * DV_U - 1) / (DV_NW * DV_U);
    DecodeRound<MM> R0, R1;
    load_round(0, R0);

    // Stage activations and per-run sums.  Thread i owns chunk i (8 values); the four
    // chunks of a 32-value run sit in four consecutive lanes.
    auto stage_chunk = [&](int i, u32x4 v) {
        reinterpret_cast<u32x4*>(sA)[i] = v;
        const f16x8 a = as_f16x8(v);
        float s1 = (float)a[0] + (float)a[1] + (float)a[4] + (float)a[5];
        float s16 = (float)a[2] + (float)a[3] + (float)a[6] + (float)a[7];
        s1 += __shfl_xor(s1, 1);
        s16 += __shfl_xor(s16, 1);
        s1 += __shfl_xor(s1, 2);
        s16 += __shfl_xor(s16, 2);
        if ((i & 3) == 0) sSum[i >> 2] = make_float2(s1, s16);
    };
#pragma unroll
    for (int j = 0; j < ABUF; ++j) {
        const int i = tid + j * DV_NW * kWave;
        if (j * DV_NW * kWave < nchunk) stage_chunk(i, i < nchunk ? abuf[j] : u32x4{});
    }
    for (int i0 = ABUF * DV_NW * kWave; i0 < nchunk; i0 += DV_NW * kWave) {
        const int i = i0 + tid;
        u32x4 v{};
        if (i < nchunk) {
            const int m = i / cpr, c = i - m * cpr;
            v = *reinterpret_cast<const u32x4*>(p.A + (int64_t)m * p.lda + 8 * c);
        }
        stage_chunk(i, v);
    }
    __syncthreads();

    float acc[MM];
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[m] = 0.0f;
    auto compute_one = [&](int pp, const DecodeRound<MM>& R, int u) {
        const int k0 = 64 * (2 * pp + dc) + 32 * h;
        float c1[MM], c16[MM];
#pragma unroll
        for (int m = 0; m < MM; ++m) c1[m] = c16[m] = 0.0f;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            const uint32_t x = R.w[u][w], x8 = x >> 8;
            const f16x2 t0 = as_h2((x & 0x000F000Fu) | 0x64006400u);
            const f16x2 t1 = as_h2((x & 0x00F000F0u) | 0x64006400u);
            const f16x2 t2 = as_h2((x8 & 0x000F000Fu) | 0x64006400u);
            const f16x2 t3 = as_h2((x8 & 0x00F000F0u) | 0x64006400u);
#pragma unroll
            for (int m = 0; m < MM; ++m) {
                const u32x4 a = *reinterpret_cast<const u32x4*>(sA + m * K + k0 + 8 * w);
                c1[m] = __builtin_amdgcn_fdot2(t0, as_h2(a[0]), c1[m], false);
                c16[m] = __builtin_amdgcn_fdot2(t1, as_h2(a[1]), c16[m], false);
                c1[m] = __builtin_amdgcn_fdot2(t2, as_h2(a[2]), c1[m], false);
                c16[m] = __builtin_amdgcn_fdot2(t3, as_h2(a[3]), c16[m], false);
            }
        }
        uint32_t z;
        if constexpr (ZF != WMMA_ZEROS_U8)
            z = (R.z[u] >> (4 * (n & 7))) & 0xFu;
        else
            z = R.z[u] & 0xFu;
        const float s = (float)__builtin_bit_cast(f16, (uint16_t)R.s[u]);
        const float zf = (float)z;
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            const float2 as = sSum[(m * K + k0) >> 5];
            const float r = c1[m] + 0.0625f * c16[m] - (1024.0f + zf) * as.x - (64.0f + zf) * as.y;
            acc[m] += s * r;
        }
    };
    auto compute_round = [&](int r, const DecodeRound<MM>& R) {
        const int pp0 = wave + DV_NW * DV_U * r;
        if (pp0 + DV_NW * (DV_U - 1) < KP) {
#pragma unroll
            for (int u = 0; u < DV_U; ++u) compute_one(pp0 + DV_NW * u, R, u);
        } else {
#pragma unroll
            for (int u = 0; u < DV_U; ++u)
                if (pp0 + DV_NW * u < KP) compute_one(pp0 + DV_NW * u, R, u);
        }
    };
    if constexpr (ONE) {
        compute_round(0, R0);
    } else {
        for (int r = 0; r < rounds; r += 2) {
            if (r + 1 < rounds) load_round(r + 1, R1);
            compute_round(r, R0);
            if (r + 1 < rounds) {
                if (r + 2 < rounds) load_round(r + 2, R0);
                compute_round(r + 1, R1);
            }
        }
    }
#pragma unroll
    for (int m = 0; m < MM; ++m) {
        acc[m] += __shfl_xor(acc[m], 16);
        acc[m] += __shfl_xor(acc[m], 32);
        if (sub == 0) red[wave][m][col] = acc[m];
    }
    __syncthreads();
    if (tid < 16 * MM) {
        const int m = tid >> 4, c = tid & 15;
        float v = red[0][m][c];
#pragma unroll
        for (int w = 1; w < DV_NW; ++w) v += red[w][m][c];
        store_y(p, (int64_t)m * p.ldy + 32 * nt + 16 * sc + c, v);
    }
}

// ---------------------------------------------- decode on the matrix pipe (M <= 4) --
// One workgroup per 16-column slice over the whole K range, so no cross-workgroup
// reduction.  A wave load covers one 128-deep pair-step pp: lane l reads slice column
// l%16, chunk 2*pp + l/32, K half (l/16)%2 -- 1 KB of the slice's contiguous weights per
// instruction.  A round gives each wave DM_U consecutive pair-steps (wave w: pair-steps
// DM_NW*DM_U*r + DM_U*w + u), so each wave streams 4 KB in one run: measured on MI355X
// with the slice-contiguous layout, 7.5 -> 7.0 us at N = 14336 against pair-steps
// interleaved across the waves.
//
// Every wave is self-contained until the final cross-wave sum: it loads the activations of
// ITS pair-steps only (lane l: chunk l%16 of pair-step l/16 of the round, one 16-byte load
// per activation row), then the round's scales and zeros (ONE load each: lane l fetches
// pair-step l/16 at column l%16; a lane shuffle later hands each lane its own), then the
// DM_U weight loads, and stages its activations in a private LDS region.  No barrier sits
// between a wave's loads and its MFMAs, so each wave computes as soon as its own data has
// landed -- under a saturated memory system the waves of one workgroup finish issuing
// their loads microseconds apart.  Vector loads return in order, so the activations and
// group parameters are waited on before the weights, and pair-step u's MFMAs wait for
// weight load u only.  Every load is unconditional (indices clamped into range): the code
// is straight-line and each wait covers exactly the loads it needs.
//
// The multiply-accumulate runs on v_mfma_f32_16x16x32_f16, with the scale and zero point
// applied to each pair-step's partial sum rather than to every weight:
//   A operand (lane l: row l%16 = activation row m, K quarter l/16): the activations a,
//     unchanged;
//   B operand (lane l: column l%16 = slice column n, same K quarter): the raw nibbles of
//     one prepacked word as fp16.  (w & 0x000F000F) | 0x6400.. is the exact fp16 pair
//     (1024 + q0, 1024 + q1) (ulp 1 at 1024); the nibbles at offsets {2,3,6,7} sit four
//     bits higher, and (w & 0x00F000F0) | 0x5400.. reads them as 64 + q (ulp 1/16 at 64).
//     One shift and four v_and_or per 8 weights.
//   Per pair-step t (128 values of K, inside one group g):
//     sum_k a_k (q_k - z) s = s (D_t - P_t - z Q_t),
//     D_t = sum a B (four MFMAs into a fresh accumulator), P_t = 1024 sum_{0,1,4,5} a +
//     64 sum_{2,3,6,7} a, Q_t = sum a.
//   The lane that loaded pair-step t's activation chunk sums its 8 values (v_dot2 against
//   ones), a 16-lane DPP reduction gives P_t and Q_t for the whole pair-step, and that same
//   lane holds s and z of (t, its column), so it adds s (P_t + z Q_t) to a private
//   correction that is reduced once at the end.  The products are exact and the sums are
//   fp32, so the result differs from the fp16-rounded dequantised weights of the definition
//   by at most their rounding (2^-11 of each weight).
// The eight waves' partials meet in LDS at the end.  Requires G = 128 * 2^j (a pair-step
// never straddles two groups).
// D layout: lane l holds column n = l%16 and rows m = 4*(l/16) + r; rows 0..3 live in
// lanes 0..15.
constexpr int DM_NW = 8;
constexpr int DM_U = 4;
constexpr int DM_MAXM = 4;
// LDS row stride (halves) of a wave's staged activations: DM_U pair-steps of 128 values
// plus 16 bytes, so rows fall on different banks.
constexpr int DM_ROW = DM_U * 128 + 8;

// Sum over the 16 lanes of each DPP row, returned in every lane of the row.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float x) {
    return __builtin_bit_cast(
        float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f32<0x141>(v);  // row_half_mirror
    v += dpp_f32<0x140>(v);  // row_mirror
    return v;
}

template <int MM>
struct DecodeMRound {
    u32x4 a[MM];    // activations: row m, pair-step l/16 of the round, chunk l%16
    u32x4 w[DM_U];  // weights of pair-steps u
    uint32_t s, z;  // raw scale / zero of (pair-step l/16 of the round, column l%16)
};

// Staging buffers per wave: one when a single round covers K, else two (rounds alternate).
__host__ __device__ constexpr int dm_nbuf(bool one) { return one ? 1 : 2; }
bool decode_mfma_one(int K) { return K <= DM_NW * DM_U * 128; }
size_t decode_mfma_lds_bytes(int M, int K) {
    return (size_t)dm_nbuf(decode_mfma_one(K)) * DM_NW * M * DM_ROW * 2;
}

// ONE: K <= DM_NW * DM_U * 128 -- a single round per wave, no second register set, so
// the kernel fits 64 VGPRs and eight waves per SIMD stay resident.
template <int ZF, bool ONE, int MM>
__global__ void __launch_bounds__(DM_NW * kWave)
__attribute__((amdgpu_waves_per_eu(ONE ? 8 : 4)))
w4a16_decode_mfma_kernel(W4Args p) {
    extern __shared__ __attribute__((aligned(16))) unsigned char dm_smem[];
    __shared__ float red[DM_NW][DM_MAXM][16];
    const int K = p.K;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    // Slice of this workgroup: each XCD walks a contiguous run of slices, so the four
    // slices that share a 128-byte line of scales are served by one L2.
    const int slice = xcd_remap(blockIdx.x, gridDim.x);
    const int nt = slice >> 1, sc = slice & 1;
    const int col = lane & 15, sub = lane >> 4, dc = sub >> 1, h = sub & 1;
    const int n = 32 * nt + 16 * sc + col;
    const int KC = K / 64, KP = KC / 2;
    // Staging buffers of this wave, each [MM][DM_ROW] halves.
    f16* sbuf = reinterpret_cast<f16*>(dm_smem) + (size_t)wave * dm_nbuf(ONE) * MM * DM_ROW;

    const u32x4* wcol = p.W + pk_index(n, 0, h, KC);
    // Pair-step u of round r for this wave: each wave streams DM_U consecutive pair-steps
    // (4 KB of its slice's contiguous weights) per round.
    auto pstep = [&](int r, int u) { return DM_NW * DM_U * r + DM_U * wave + u; };
    // Fused layout: this slice's run -- the parameter block of pair-step pp (block pp / 4,
    // wave-uniform) in its header, then the weights.
    const unsigned char* fslice =
        reinterpret_cast<const unsigned char*>(p.W) + (int64_t)slice * fused_slice_bytes(K);
    const unsigned char* fw = fslice + fused_hdr_bytes(K);
    auto frec = [&](int pp) { return fslice + (int64_t)(pp >> 2) * kFusedBlock; };
    auto load_round = [&](int r, DecodeMRound<MM>& R) {
        // this lane's activation chunk / group parameters: pair-step `sub` of the round
        const int ppl = min(pstep(r, sub), KP - 1);
        const int ka = 128 * ppl + 8 * col;
#pragma unroll
        for (int m = 0; m < MM; ++m)
            R.a[m] = *reinterpret_cast<const u32x4*>(p.A + (int64_t)m * p.lda + ka);
        if constexpr (ZF == WMMA_W4_FUSED) {
            const unsigned char* rec = frec(ppl);
            R.s = *reinterpret_cast<const uint16_t*>(rec + 2 * (16 * (ppl & 3) + col));
            R.z = rec[128 + 8 * (ppl & 3) + (col >> 1)];
        } else {
            const int g = ppl >> p.pp_shift;  // G = 128 << pp_shift
            R.s = __builtin_bit_cast(uint16_t, p.S[s_index<ZF>(p, g, n)]);
            if constexpr (ZF != WMMA_ZEROS_U8)
                R.z = (uint32_t)static_cast<const int32_t*>(p.Z)[z_index<ZF>(p, g, n)];
            else
                R.z = static_cast<const uint8_t*>(p.Z)[z_index<ZF>(p, g, n)];
        }
#pragma unroll
        for (int u = 0; u < DM_U; ++u) {
            const int pp = min(pstep(r, u), KP - 1);
            if constexpr (ZF == WMMA_W4_FUSED)
                R.w[u] = __builtin_nontemporal_load(
                    reinterpret_cast<const u32x4*>(fw + (int64_t)pp * 1024 + 16 * lane));
            else
                R.w[u] = __builtin_nontemporal_load(wcol + (int64_t)(2 * pp + dc) * 32);
        }
    };

    uint32_t magic = 0x64006400u, magic_hi = 0x54005400u;
    asm volatile("" : "+v"(magic), "+v"(magic_hi));  // constants in VGPRs: one v_and_or per pair
    // DEFER: scale and zero applied per pair-step (fewer VALU operations for one or two
    // rows; from three rows on the per-row sums cost as much as they save).
    constexpr bool DEFER = MM <= 2;
    f32x4 d{};              // exact path: accumulator over all pair-steps
    float y[MM], corr[MM];  // deferred path: sum of s D_t (lanes 0..15); this lane's corrections
#pragma unroll
    for (int m = 0; m < MM; ++m) y[m] = corr[m] = 0.0f;
    const int am = col < MM ? col : 0;  // A-operand row (rows >= M repeat row 0, unused)
    const f16x2 ones = {(f16)1.0f, (f16)1.0f};
    auto compute_round = [&](int r, const DecodeMRound<MM>& R, f16* buf) {
        // This lane's pair-step: its activation chunk, scale and zero.
        const bool lane_live = pstep(r, sub) < KP;
        float P[MM], Q[MM];
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            if constexpr (DEFER) {
                // 1024 P and Q of the pair-step (offsets {0,1,4,5} in e1, {2,3,6,7} in e2)
                const float e1 = __builtin_amdgcn_fdot2(
                    as_h2(R.a[m][0]), ones,
                    __builtin_amdgcn_fdot2(as_h2(R.a[m][2]), ones, 0.0f, false), false);
                const float e2 = __builtin_amdgcn_fdot2(
                    as_h2(R.a[m][1]), ones,
                    __builtin_amdgcn_fdot2(as_h2(R.a[m][3]), ones, 0.0f, false), false);
                P[m] = row16_sum(__builtin_fmaf(e2, 64.0f, e1 * 1024.0f));
                Q[m] = row16_sum(e1 + e2);
            }
            // stage this lane's chunk of row m
            *reinterpret_cast<u32x4*>(buf + m * DM_ROW + 128 * sub + 8 * col) = R.a[m];
        }
        uint32_t rs = R.s, rz = R.z;
        asm volatile("" : "+v"(rs), "+v"(rz));  // no work on them hoisted up to their load
        uint32_t z;
        if constexpr (ZF == WMMA_W4_FUSED)
            z = (rz >> (4 * (col & 1))) & 0xFu;
        else if constexpr (ZF != WMMA_ZEROS_U8)
            z = (rz >> (4 * (n & 7))) & 0xFu;
        else
            z = rz & 0xFu;
        if constexpr (DEFER) {
            const float sf = lane_live ? (float)__builtin_bit_cast(f16, (uint16_t)rs) : 0.0f;
            const float zf = (float)z;
#pragma unroll
            for (int m = 0; m < MM; ++m)
                corr[m] = __builtin_fmaf(sf, __builtin_fmaf(zf, Q[m], P[m]), corr[m]);
        }
        const int sz = (int)(rs | (z << 16));
        const f16* arow = buf + am * DM_ROW + 32 * sub;
#pragma unroll
        for (int u = 0; u < DM_U; ++u) {
            const uint32_t v = (uint32_t)__shfl(DEFER ? (int)rs : sz, 16 * u + col);
            const int pp = pstep(r, u);
            if (pp < KP) {
                const uint32_t zz = v >> 16, s = v & 0xFFFFu;
                const uint32_t z1 = 0x6400u | zz, zhi = 0x5400u | (zz << 4);
                const f16x2 zs1 = as_h2(z1 | (z1 << 16)), zshi = as_h2(zhi | (zhi << 16));
                const f16x2 ss = as_h2(s | (s << 16));
                f32x4 acc = DEFER ? f32x4{} : d;
#pragma unroll
                for (int w = 0; w < 4; ++w) {
                    const uint32_t x = R.w[u][w], x8 = x >> 8;
                    u32x4 bv;
                    bv[0] = (x & 0x000F000Fu) | magic;       // 1024 + q
                    bv[1] = (x & 0x00F000F0u) | magic_hi;    // 64 + q
                    bv[2] = (x8 & 0x000F000Fu) | magic;
                    bv[3] = (x8 & 0x00F000F0u) | magic_hi;
                    if constexpr (!DEFER) {  // W = fp16((q - z) s)
                        bv[0] = as_u32((as_h2(bv[0]) - zs1) * ss);
                        bv[1] = as_u32((as_h2(bv[1]) - zshi) * ss);
                        bv[2] = as_u32((as_h2(bv[2]) - zs1) * ss);
                        bv[3] = as_u32((as_h2(bv[3]) - zshi) * ss);
                    }
                    const f16x8 av = as_f16x8(*reinterpret_cast<const u32x4*>(arow + 128 * u + 8 * w));
                    acc = mfma16(av, as_f16x8(bv), acc);
                }
                if constexpr (DEFER) {
                    const float sf = (float)__builtin_bit_cast(f16, (uint16_t)s);
#pragma unroll
                    for (int m = 0; m < MM; ++m) y[m] = __builtin_fmaf(sf, acc[m], y[m]);
                } else {
                    d = acc;
                }
            }
        }
    };

    if constexpr (ONE) {
        DecodeMRound<MM> R0;
        load_round(0, R0);
        compute_round(0, R0, sbuf);
    } else {
        // Round r+1 in flight while round r is computed; straight-line body (the loads
        // past the last round are clamped re-loads of it).  Staging buffers alternate, so
        // a wave's LDS writes for round r+1 never race its reads of round r.
        const int rounds = (KP - DM_U * wave + DM_NW * DM_U - 1) / (DM_NW * DM_U);
        DecodeMRound<MM> R0, R1;
        load_round(0, R0);
        load_round(1, R1);
        for (int r = 0; r < rounds; r += 2) {
            compute_round(r, R0, sbuf);
            load_round(r + 2, R0);
            if (r + 1 < rounds) compute_round(r + 1, R1, sbuf + MM * DM_ROW);
            load_round(r + 3, R1);
        }
    }
    // Rows 0..MM-1 live in lanes 0..15 (d[m], or y[m] less the corrections of the four
    // lanes of the column, one per pair-step of a round).
    if constexpr (DEFER) {
#pragma unroll
        for (int m = 0; m < MM; ++m) {
            corr[m] += __shfl_xor(corr[m], 16);
            corr[m] += __shfl_xor(corr[m], 32);
        }
    }
    if (sub == 0) {
#pragma unroll
        for (int m = 0; m < MM; ++m) red[wave][m][col] = DEFER ? y[m] - corr[m] : d[m];
    }
    __syncthreads();
    if (tid < 16 * MM) {
        const int m = tid >> 4, c = tid & 15;
        float v = red[0][m][c];
#pragma unroll
        for (int w = 1; w < DM_NW; ++w) v += red[w][m][c];
        store_y(p, (int64_t)m * p.ldy + 32 * nt + 16 * sc + c, v);
    }
}

template <int ZF, bool ONE, int MM>
void launch_decode_mfma_m(const W4Args& a, dim3 grid, dim3 block, size_t lds, hipStream_t stream) {
    // Above 64 KB of dynamic LDS (M = 4 past one round) the kernel's launch limit is raised
    // first.
    if (lds > 64 * 1024 &&
        hipFuncSetAttribute(reinterpret_cast<const void*>(&w4a16_decode_mfma_kernel<ZF, ONE, MM>),
                            hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess)
        return;  // the error stays for the caller's hipGetLastError
    hipLaunchKernelGGL((w4a16_decode_mfma_kernel<ZF, ONE, MM>), grid, block, lds, stream, a);
}

template <int ZF, bool ONE>
void launch_decode_mfma(const W4Args& a, int M, dim3 grid, dim3 block, size_t lds,
                        hipStream_t stream) {
    switch (M) {
        case 1: launch_decode_mfma_m<ZF, ONE, 1>(a, grid, block, lds, stream); break;
        case 2: launch_decode_mfma_m<ZF, ONE, 2>(a, grid, block, lds, stream); break;
        case 3: launch_decode_mfma_m<ZF, ONE, 3>(a, grid, block, lds, stream); break;
        default: launch_decode_mfma_m<ZF, ONE, 4>(a, grid, block, lds, stream); break;
    }
}

// ------------------------------------------------ skinny (4 < M <= 32) on the matrix pipe --
// Memory-bound like decode (every weight is used by at most 32 rows), so the structure is
// the decode kernel's: every wave issues all its loads up front and then works through
// them in arrival order, with no barrier before the final cross-wave sum.  Differences:
//  * a workgroup covers a whole 32-column prepacked tile (both 16-column halves), so each
//    activation fragment feeds two MFMAs;
//  * the activations come straight from L2 into registers in the MFMA A-operand layout --
//    lane l: row 16*b + l%16 (clamped to M-1; those rows are never stored), K quarter l/16,
//    i.e. 64 contiguous bytes per lane per pair-step;
//  * SK_U pair-steps per wave; when the 32-column tiles alone cannot fill the chip the K
//    range is split over blockIdx.y (SK_NW * SK_U pair-steps per split) and the partials
//    go to the workspace for w4a16_reduce_kernel.
// The B operand is the decode kernel's nibble encoding (1024 + q, and 64 + q at offsets
// {2,3,6,7}) less the same encoding of z, times s: W = fp16((q - z) s), one rounding.
//  * NH 16-column slices per workgroup (1, 2 or 4): each activation fragment feeds NH
//    MFMAs.  NH = 4 halves the activation bytes a CU reads per weight byte against NH = 2
//    (at M = 16 they are twice the weight bytes of a 32-column workgroup); NH = 1 gives
//    twice the workgroups of NH = 2 where 32-column tiles would leave CUs idle.
// D layout per 16-row block b and slice sc (0 .. NH-1): lane l holds column
// 16*NH*wg + 16*sc + l%16 and rows 16*b + 4*(l/16) + r.
constexpr int SK_NW = 8;

template <int ZF, int MB, int U, int NH>
__global__ void __launch_bounds__(SK_NW * kWave)
w4a16_skinny_kernel(W4Args p) {
    constexpr int NC = 16 * NH;  // columns per workgroup
    __shared__ float red[SK_NW][MB * 16][NC + 1];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = xcd_remap(blockIdx.x, gridDim.x);
    const int n0 = NC * wg;  // first column of the workgroup
    const int col = lane & 15, sub = lane >> 4, dc = sub >> 1, h = sub & 1;
    const int K = p.K, M = p.M, KC = K / 64, KP = KC / 2;
    const int kp0 = blockIdx.y * (SK_NW * U);

    // Group parameters: lane l fetches pair-step min(l/16, U-1) of this wave for every
    // 16-column half; a lane shuffle later hands each lane its own.
    uint32_t sraw[NH], zraw[NH];
    {
        const int ppl = min(kp0 + wave + SK_NW * min(sub, U - 1), KP - 1);
        const int g = ppl >> p.pp_shift;  // G = 128 << pp_shift
#pragma unroll
        for (int sc = 0; sc < NH; ++sc) {
            const int n = n0 + 16 * sc + col;
            sraw[sc] = __builtin_bit_cast(uint16_t, p.S[s_index<ZF>(p, g, n)]);
            if constexpr (ZF != WMMA_ZEROS_U8)
                zraw[sc] = (uint32_t)static_cast<const int32_t*>(p.Z)[z_index<ZF>(p, g, n)];
            else
                zraw[sc] = static_cast<const uint8_t*>(p.Z)[z_index<ZF>(p, g, n)];
        }
    }
    // Activations and weights, pair-step by pair-step (clamped: every load is issued).
    u32x4 av[U][MB][4], wv[U][NH];
    const u32x4* wbase = p.W + pk_index(n0 + col, 0, h, KC);
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int pp = min(kp0 + wave + SK_NW * u, KP - 1);
#pragma unroll
        for (int b = 0; b < MB; ++b) {
            const int row = min(16 * b + col, M - 1);
            const f16* ap = p.A + (int64_t)row * p.lda + 128 * pp + 32 * sub;
#pragma unroll
            for (int q = 0; q < 4; ++q) av[u][b][q] = *reinterpret_cast<const u32x4*>(ap + 8 * q);
        }
#pragma unroll
        for (int sc = 0; sc < NH; ++sc)
            wv[u][sc] = __builtin_nontemporal_load(wbase + (int64_t)sc * KC * 32 + (int64_t)(2 * pp + dc) * 32);
    }

#pragma unroll
    for (int sc = 0; sc < NH; ++sc) asm volatile("" : "+v"(sraw[sc]), "+v"(zraw[sc]));
    int sz[NH];
#pragma unroll
    for (int sc = 0; sc < NH; ++sc) {
        uint32_t z;
        if constexpr (ZF != WMMA_ZEROS_U8)
            z = (zraw[sc] >> (4 * ((n0 + 16 * sc + col) & 7))) & 0xFu;
        else
            z = zraw[sc] & 0xFu;
        sz[sc] = (int)(sraw[sc] | (z << 16));
    }
    uint32_t magic = 0x64006400u, magic_hi = 0x54005400u;
    asm volatile("" : "+v"(magic), "+v"(magic_hi));
    f32x4 d[MB][NH];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int sc = 0; sc < NH; ++sc) d[b][sc] = f32x4{};
#pragma unroll
    for (int u = 0; u < U; ++u) {
        uint32_t v[NH];
#pragma unroll
        for (int sc = 0; sc < NH; ++sc) v[sc] = (uint32_t)__shfl(sz[sc], 16 * u + col);
        if (kp0 + wave + SK_NW * u < KP) {  // uniform
            f16x8 a[MB][4];
#pragma unroll
            for (int b = 0; b < MB; ++b)
#pragma unroll
                for (int q = 0; q < 4; ++q) a[b][q] = as_f16x8(av[u][b][q]);
#pragma unroll
            for (int sc = 0; sc < NH; ++sc) {
                const uint32_t zz = v[sc] >> 16, s = v[sc] & 0xFFFFu;
                const uint32_t z1 = 0x6400u | zz, zhi = 0x5400u | (zz << 4);
                const f16x2 zs1 = as_h2(z1 | (z1 << 16)), zshi = as_h2(zhi | (zhi << 16));
                const f16x2 ss = as_h2(s | (s << 16));
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const uint32_t x = wv[u][sc][q], x8 = x >> 8;
                    u32x4 bv;
                    bv[0] = as_u32((as_h2((x & 0x000F000Fu) | magic) - zs1) * ss);
                    bv[1] = as_u32((as_h2((x & 0x00F000F0u) | magic_hi) - zshi) * ss);
                    bv[2] = as_u32((as_h2((x8 & 0x000F000Fu) | magic) - zs1) * ss);
                    bv[3] = as_u32((as_h2((x8 & 0x00F000F0u) | magic_hi) - zshi) * ss);
#pragma unroll
                    for (int b = 0; b < MB; ++b) d[b][sc] = mfma16(a[b][q], as_f16x8(bv), d[b][sc]);
                }
            }
        }
    }
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int sc = 0; sc < NH; ++sc)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][16 * b + 4 * sub + r][16 * sc + col] = d[b][sc][r];
    __syncthreads();
    const bool partial = gridDim.y > 1;
    for (int i = tid; i < M * NC; i += SK_NW * kWave) {
        const int m = i / NC, c = i % NC;
        float acc = red[0][m][c];
#pragma unroll
        for (int w = 1; w < SK_NW; ++w) acc += red[w][m][c];
        const int n = n0 + c;
        if (partial)
            p.ws[((int64_t)blockIdx.y * M + m) * p.N + n] = acc;
        else
            store_y(p, (int64_t)m * p.ldy + n, acc);
    }
}

// Shape of a skinny launch: NH 16-column slices per workgroup and U pair-steps per wave, so
// a workgroup covers SK_NW * U * 128 of K and longer K is split over blockIdx.y (plus the
// reduce pass).  What decides it, measured on MI355X over M = 2..32, N = 256..14336,
// K = 1024..14336 (every NH x U at 136 shapes, graph-replayed; summed over them this rule
// takes 0.5% more time than the best choice and 12.6% less than the tile-count rule it
// replaced):
//  * the reduce pass costs 1.5-3 us, so K that one workgroup covers stays unsplit even with
//    few workgroups (K <= 2048: always; N = 256, K = 2048, M = 5: 2.9 us against 4.4 split);
//  * each slice a workgroup adds halves the activation re-reads (every workgroup reads all
//    M x K activations of its K range: M / (4 NH) of the weight bytes), which decides long K
//    (N = 4096, K = 14336, M = 16: NH = 4 13.1 us, NH = 1 20.6);
//  * registers: NH = 4 with U = 4 (M <= 16) and with U = 2 (M > 16) leave one workgroup per
//    CU, so those take them only where the workgroups do not exceed the CUs' slots
//    (M = 32, N = K = 14336: U = 1 47.7 us, U = 2 54.3);
//  * a split gives at least 0.7 workgroups per CU (N = 1024, K = 8192: NH = 2 with U = 1,
//    256 workgroups, 6.5 us at M = 16 against 7.4 with U = 2).
void skinny_config(int M, int N, int K, int num_cus, int* nh_out, int* u_out) {
    const bool mb1 = M <= 16;  // one 16-row block (U up to 4) or two (U up to 2, NH >= 2)
    const int umax = mb1 ? 4 : 2;
    auto nh_ok = [&](int h) { return N % (16 * h) == 0 && (h != 1 || mb1); };
    auto slices = [&](int h) { return (int64_t)(N / (16 * h)); };
    auto wgs = [&](int h, int u) { return slices(h) * ceil_div(K, SK_NW * 128 * u); };
    const int u0 = K <= 1024 ? 1 : K <= 2048 ? 2 : K <= 4096 ? 4 : 8;
    if (u0 <= umax) {
        // unsplit: the widest workgroups that still give 0.6 per CU
        int nh = mb1 ? 1 : 2;
        for (int h : {4, 2, 1})
            if (nh_ok(h) && slices(h) * 10 >= 6 * (int64_t)num_cus) {
                nh = h;
                break;
            }
        if (K <= 2048 || slices(nh) * 4 >= num_cus) {
            *nh_out = nh;
            *u_out = u0;
            return;
        }
    }
    int nh = 1;
    if (nh_ok(4) && (int64_t)(N / 64) * 8 >= num_cus)
        nh = 4;
    else if ((int64_t)(N / 32) * 8 >= num_cus || !mb1)
        nh = 2;
    int u = 1;
    if (mb1) {
        for (int c : {4, 2})
            if (!(nh == 4 && c == 4) && wgs(nh, c) * 10 >= 7 * (int64_t)num_cus) {
                u = c;
                break;
            }
    } else {
        const int64_t w2 = wgs(nh, 2);
        u = (w2 * 10 >= 7 * (int64_t)num_cus && w2 < 2 * (int64_t)num_cus) ? 2 : 1;
    }
    *nh_out = nh;
    *u_out = u;
}

template <int ZF, int MB, int NH>
void launch_skinny_mb(const W4Args& a, int U, dim3 grid, hipStream_t stream) {
    const dim3 block(SK_NW * kWave);
    if (U == 4)
        hipLaunchKernelGGL((w4a16_skinny_kernel<ZF, MB, (MB == 1 ? 4 : 2), NH>), grid, block, 0, stream, a);
    else if (U == 2)
        hipLaunchKernelGGL((w4a16_skinny_kernel<ZF, MB, 2, NH>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((w4a16_skinny_kernel<ZF, MB, 1, NH>), grid, block, 0, stream, a);
}

// --------------------------------------------- rows (M > 4) on the matrix pipe, no LDS ring --
// The skinny kernel's structure extended to any M: a workgroup covers 16*MB rows (row
// group blockIdx.z) by 16*NH columns over its whole K range (or one split of it), eight
// waves taking interleaved 128-deep pair-steps (wave w: pair-steps kb + w + 8r).  Each wave
// loads its activations straight from L2 into registers in the MFMA A-operand layout, and
// its weights, scales and zeros into registers: the weights (from HBM) one round (one
// pair-step) ahead of the round that uses them, the activations, scales and zeros at the
// start of their own round.  No barrier sits anywhere before the final cross-wave sum and
// no wave waits for another's loads.  Fewer bytes in flight per CU run faster here: measured
// on MI355X over 54 shape x configuration cases (M = 33-128, N = 1024 / 4096, K = 2048-8192),
// this schedule took 10% less time than loading the whole next round ahead, which took 16%
// less than loading two rounds ahead; the weights go through the cache (streaming them
// past it was 3% slower).  A workgroup reads 32*MB + 8*NH bytes of activations and
// weights per K value; the weights of a column group are shared through L2 by the row
// groups (blockIdx.x is the column group, so with a grid width divisible by eight every
// row group of a column group runs on one XCD).
// Loads of rounds past the wave's last go to an out-of-range buffer offset and return
// zeros without a memory request, so the loop body stays straight-line.
// B operand: the skinny kernel's W = fp16((q - z) s), one rounding.  D layout per block b,
// slice sc: lane l holds column 16*NH*wg + 16*sc + l%16, rows 16*MB*z + 16*b + 4*(l/16) + r.
constexpr int RW_NW = 8;

template <int MB, int NH>
struct RowsRound {
    u32x4 a[MB][4];
    u32x4 w[NH];
    uint32_t s[NH], z[NH];
};

template <int ZF, int MB, int NH>
__global__ void __launch_bounds__(RW_NW * kWave)
w4a16_rows_kernel(W4Args p) {
    constexpr int NC = 16 * NH, MR = 16 * MB;
    __shared__ float red[RW_NW][MR][NC + 1];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wg = xcd_remap(blockIdx.x, gridDim.x);
    const int n0 = NC * wg, m0 = MR * blockIdx.z;
    const int col = lane & 15, sub = lane >> 4, dc = sub >> 1, h = sub & 1;
    const int M = p.M, KC = p.K / 64, KP = KC / 2;
    const int kpps = p.kc_per_split >> 1;
    const int kb = blockIdx.y * kpps, ke = min(KP, kb + kpps);
    const int rounds = max(0, (ke - kb - wave + RW_NW - 1) / RW_NW);

    // The activation resource starts at the workgroup's first row; the rows it reads span at
    // most min(M, 16*MB) * lda * 2 bytes, which the C-ABI keeps under 2 GB (it rejects
    // min(M, 256) * lda * 2 bytes above that).  Rows past M read row M-1 and are never stored.
    const __amdgpu_buffer_rsrc_t ar = make_rsrc(p.A + (int64_t)m0 * p.lda), wr = make_rsrc(p.W),
                                 sr = make_rsrc(p.S), zr = make_rsrc(p.Z);
    uint32_t aoff[MB];
#pragma unroll
    for (int b = 0; b < MB; ++b)
        aoff[b] = (uint32_t)(((int64_t)(min(m0 + 16 * b + col, M - 1) - m0) * p.lda + 32 * sub) * 2);
    const uint32_t woff = (uint32_t)(pk_index(n0 + col, 0, h, KC) * 16) + 512u * dc;
    // Byte offsets of this lane's scale and zero element: lane part + sc * (slice step) +
    // g * (group step), per zeros format.
    uint32_t s_lane, s_sc, s_g, z_lane, z_sc, z_g;
    if constexpr (ZF == WMMA_ZEROS_SLICED) {
        s_lane = (uint32_t)(((int64_t)(n0 >> 4) * p.kg * 16 + col) * 2);
        s_sc = (uint32_t)p.kg * 32u;
        s_g = 32u;
        z_lane = (uint32_t)(((int64_t)(n0 >> 4) * p.kg * 2 + ((col >> 3) & 1)) * 4);
        z_sc = (uint32_t)p.kg * 8u;
        z_g = 8u;
    } else {
        s_lane = (uint32_t)(n0 + col) * 2u;
        s_sc = 32u;
        s_g = (uint32_t)p.N * 2u;
        if constexpr (ZF == WMMA_ZEROS_PACKED) {
            z_lane = (uint32_t)((n0 + col) >> 3) * 4u;
            z_sc = 8u;
            z_g = (uint32_t)p.N / 2u;
        } else {
            z_lane = (uint32_t)(n0 + col);
            z_sc = 16u;
            z_g = (uint32_t)p.N;
        }
    }
    // Round r's scales, zeros and activations, and (load_w) its weights.
    auto load_ap = [&](int r, RowsRound<MB, NH>& R) {
        const int pp = kb + wave + RW_NW * r;
        const uint32_t oob = r < rounds ? 0u : kOobOffset;
        const uint32_t g = (uint32_t)(min(pp, KP - 1) >> p.pp_shift);  // G = 128 << pp_shift
#pragma unroll
        for (int sc = 0; sc < NH; ++sc) {
            R.s[sc] = buf_load2(sr, (s_lane + sc * s_sc + g * s_g) | oob);
            if constexpr (ZF != WMMA_ZEROS_U8)
                R.z[sc] = buf_load4(zr, (z_lane + sc * z_sc + g * z_g) | oob);
            else
                R.z[sc] = buf_load1(zr, (z_lane + sc * z_sc + g * z_g) | oob);
        }
#pragma unroll
        for (int b = 0; b < MB; ++b)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                R.a[b][q] = buf_load16(ar, (aoff[b] + 256u * pp + 16u * q) | oob);
    };
    auto load_w = [&](int r, RowsRound<MB, NH>& R) {
        const int pp = kb + wave + RW_NW * r;
        const uint32_t oob = r < rounds ? 0u : kOobOffset;
#pragma unroll
        for (int sc = 0; sc < NH; ++sc)
            R.w[sc] = buf_load16(wr, (woff + (uint32_t)sc * KC * 512u + 1024u * pp) | oob);
    };

    uint32_t magic = 0x64006400u, magic_hi = 0x54005400u;
    asm volatile("" : "+v"(magic), "+v"(magic_hi));
    f32x4 d[MB][NH];
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int sc = 0; sc < NH; ++sc) d[b][sc] = f32x4{};
    auto compute = [&](const RowsRound<MB, NH>& R) {
#pragma unroll
        for (int sc = 0; sc < NH; ++sc) {
            uint32_t z;
            if constexpr (ZF != WMMA_ZEROS_U8)
                z = (R.z[sc] >> (4 * ((n0 + 16 * sc + col) & 7))) & 0xFu;
            else
                z = R.z[sc] & 0xFu;
            const uint32_t s = R.s[sc];
            const uint32_t z1 = 0x6400u | z, zhi = 0x5400u | (z << 4);
            const f16x2 zs1 = as_h2(z1 | (z1 << 16)), zshi = as_h2(zhi | (zhi << 16));
            const f16x2 ss = as_h2(s | (s << 16));
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint32_t x = R.w[sc][q], x8 = x >> 8;
                u32x4 bv;
                bv[0] = as_u32((as_h2((x & 0x000F000Fu) | magic) - zs1) * ss);
                bv[1] = as_u32((as_h2((x & 0x00F000F0u) | magic_hi) - zshi) * ss);
                bv[2] = as_u32((as_h2((x8 & 0x000F000Fu) | magic) - zs1) * ss);
                bv[3] = as_u32((as_h2((x8 & 0x00F000F0u) | magic_hi) - zshi) * ss);
#pragma unroll
                for (int b = 0; b < MB; ++b) d[b][sc] = mfma16(as_f16x8(R.a[b][q]), as_f16x8(bv), d[b][sc]);
            }
        }
    };

    // Two register sets, rounds alternating between them.  A round past the last (odd round
    // counts) computes on zeros and adds nothing.  The scheduling barriers keep each load
    // where it is written (without them the compiler sinks loads behind the MFMAs that
    // follow).
    RowsRound<MB, NH> RA, RB;
    load_w(0, RA);
    __builtin_amdgcn_sched_barrier(0);
    for (int r = 0; r < rounds; r += 2) {
        load_ap(r, RA);
        __builtin_amdgcn_sched_barrier(0);
        load_w(r + 1, RB);
        __builtin_amdgcn_sched_barrier(0);
        compute(RA);
        __builtin_amdgcn_sched_barrier(0);
        load_ap(r + 1, RB);
        __builtin_amdgcn_sched_barrier(0);
        load_w(r + 2, RA);
        __builtin_amdgcn_sched_barrier(0);
        compute(RB);
        __builtin_amdgcn_sched_barrier(0);
    }
#pragma unroll
    for (int b = 0; b < MB; ++b)
#pragma unroll
        for (int sc = 0; sc < NH; ++sc)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][16 * b + 4 * sub + r][16 * sc + col] = d[b][sc][r];
    __syncthreads();
    const bool partial = gridDim.y > 1;
    const int mrows = min(MR, M - m0);
    for (int i = tid; i < mrows * NC; i += RW_NW * kWave) {
        const int m = i / NC, c = i % NC;
        float acc = red[0][m][c];
#pragma unroll
        for (int w = 1; w < RW_NW; ++w) acc += red[w][m][c];
        const int n = n0 + c;
        if (partial)
            p.ws[((int64_t)blockIdx.y * M + m0 + m) * p.N + n] = acc;
        else
            store_y(p, (int64_t)(m0 + m) * p.ldy + n, acc);
    }
}

template <int ZF, int MB, int NH>
void launch_rows(const W4Args& a, dim3 grid, hipStream_t stream) {
    hipLaunchKernelGGL((w4a16_rows_kernel<ZF, MB, NH>), grid, dim3(RW_NW * kWave), 0, stream, a);
}

// ------------------------------------------------------ W4A16 GEMM (M > 32), LDS-DMA --
// Output tile BM x BN per workgroup, WM x WN waves, wave tile TM x TN = FM x FN MFMA
// 32x32x16 tiles.  K advances in 64-deep stages (one prepacked block row):
//   activations A[BM][64] fp16 travel global -> LDS by buffer_load ... lds into an NS-deep
//     ring; rows of eight 16-byte chunks, chunk c of row r stored at c ^ swz8(r)
//     (conflict-free for the 16-row ds_read_b128 pattern below);
//   weights: each wave loads its FN prepacked blocks (1 KB each; lane l: the four words of
//     column l%32, K half l/32) plus that lane's scale and zero straight into registers,
//     into a ring NS stages deep -- the stage issued NS-1 stages ahead never overwrites the
//     one being dequantised.
// k-step j of a stage (j = 0..3) uses word j of every lane: K offsets 32*(l/32) + 8j .. +7,
// matched on the A side by chunk 4*(l/32) + j of the lane's row.  Dequantisation per word:
// pair i, the nibbles at bits 4i and 16 + 4i, as 1024 + q (i even: (w >> 4i) & 0x000F000F
// | 0x6400..) or 64 + q (i odd: bits 4..7 kept in place, | 0x5400..), exact, minus the
// same encoding of z (exact), times s (one fp16 rounding) -- W = fp16((q - z) s), the A
// operand stays raw.  G is a power of two (a shift finds a K offset's group).
// One barrier per stage, after this wave's share of the stage has landed (vmcnt): from
// then on every wave's copy is visible and every wave has finished reading the slot the
// new DMA overwrites.
constexpr int W4G_MAXSTAGES = 4;

template <int FN>
struct W4GSlot {
    u32x4 w[FN];
    uint32_t s[FN], z[FN];
};

template <int BM, int BN, int WM, int WN, int NS, int ZF>
struct W4GCfg {
    static constexpr int NW = WM * WN, TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    static constexpr int A_BYTES = BM * 128;
    static constexpr int A_DMA = A_BYTES / (1024 * NW);
    static constexpr int PER = A_DMA + 3 * FN;  // vmcnt events per stage per wave
    static_assert(A_BYTES % (1024 * NW) == 0, "A stage must split into 1 KB DMAs per wave");
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
    static_assert(NS >= 3 && NS <= W4G_MAXSTAGES && (NS - 2) * PER < 64, "vmcnt range");
};

struct W4GLane {
    uint32_t a_off[8];  // A DMA source offsets (row part; kOobOffset for rows >= M)
    int a_dst;          // this wave's DMA slice of a stage
    int a_addr[8];      // byte offset of the lane's A row in a stage (per i < FM)
    int a_sw[8];        // its swizzle
    uint32_t w_off[4];  // weight block offset of column tile j at K chunk 0 (kOobOffset: none)
    uint32_t s_off[4], z_off[4];  // scale / zero offset of column tile j at group 0
    int h;
};

// Issue the loads of global K chunk kc (kc < 0: nothing real -- every lane reads out of
// range, so the event count stays uniform) into LDS slot dst and register slot R.  The
// per-lane base offsets already carry kOobOffset for rows / columns outside the matrix;
// adding a K offset (< 2^31) keeps them out of range, so no lane needs a branch.
template <class C, int ZF>
__device__ __forceinline__ void w4g_issue(const W4Args& p, const W4GLane& L,
                                          __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rw,
                                          __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rz,
                                          int kc, WMMA_LDS unsigned char* __restrict__ dst,
                                          W4GSlot<C::FN>& R) {
    const bool live = kc >= 0;  // uniform
    const uint32_t dead = live ? 0u : kOobOffset;
    const uint32_t k = live ? (uint32_t)kc : 0u;
#pragma unroll
    for (int i = 0; i < C::A_DMA; ++i)
        lds_dma16(ra, (L.a_off[i] + k * 128u) | dead, dst + L.a_dst + i * 1024);
    const uint32_t g = (64u * k + 32u * (uint32_t)L.h) >> p.g_shift;  // G = 2^g_shift
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
        R.w[j] = buf_load16(rw, (L.w_off[j] + k * 512u) | dead);
        // byte strides from group g to g + 1
        const uint32_t s_gs = ZF == WMMA_ZEROS_SLICED ? 32u : (uint32_t)p.N * 2u;
        const uint32_t z_gs = ZF == WMMA_ZEROS_SLICED ? 8u
                              : ZF == WMMA_ZEROS_PACKED ? (uint32_t)(p.N / 8) * 4u : (uint32_t)p.N;
        R.s[j] = buf_load2(rs, (L.s_off[j] + g * s_gs) | dead);
        if constexpr (ZF != WMMA_ZEROS_U8)
            R.z[j] = buf_load4(rz, (L.z_off[j] + g * z_gs) | dead);
        else
            R.z[j] = buf_load1(rz, (L.z_off[j] + g * z_gs) | dead);
    }
}

// One stage, after its wait + barrier: issue stage t + NS - 1 (global chunk kc_next, or -1)
// into LDS slot dst and register slot Rn, then dequantise this stage's weights (slot R) and
// run its 4 x FM x FN MFMAs on the activations in LDS slot cur.  cur and dst are distinct
// slots, declared __restrict__ so the compiler keeps the DMA in flight across the reads;
// the ordering between a DMA and later reads of the same slot is the wait + barrier.
template <class C, int ZF>
__device__ __forceinline__ void w4g_stage(const W4Args& p, const W4GLane& L,
                                          __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rw,
                                          __amdgpu_buffer_rsrc_t rs, __amdgpu_buffer_rsrc_t rz,
                                          const WMMA_LDS unsigned char* __restrict__ cur,
                                          WMMA_LDS unsigned char* __restrict__ dst, int kc_next,
                                          const W4GSlot<C::FN>& R, W4GSlot<C::FN>& Rn,
                                          bool compute, int lane, uint32_t magic,
                                          uint32_t magic_hi, f32x16 (&acc)[C::FM][C::FN]) {
    w4g_issue<C, ZF>(p, L, ra, rw, rs, rz, kc_next, dst, Rn);
    if (!compute) return;
    // This stage's register slot passes through an empty asm first: without it the
    // compiler hoists the dequantisation of a slot up to where its loads were just issued
    // (NS - 1 stages early) and waits there for them (vmcnt(1..2)), so every stage paid
    // the full memory latency.  The caller's wait_vmcnt already covers these loads.
    W4GSlot<C::FN> r = R;
#pragma unroll
    for (int j = 0; j < C::FN; ++j) asm volatile("" : "+v"(r.w[j]), "+v"(r.s[j]), "+v"(r.z[j]));
    // Nibble pairs q = 0, 2 (bits 4q and 16 + 4q) become 1024 + q through the 0x6400
    // exponent, pairs 1, 3 -- left in place at bits 4..7 -- become 64 + q through 0x5400;
    // each is less the same encoding of z (exact), times s (one rounding).  One shift per
    // word instead of three.
    f16x2 zs[C::FN], zshi[C::FN], ss[C::FN];
#pragma unroll
    for (int j = 0; j < C::FN; ++j) {
        uint32_t z;
        if constexpr (ZF != WMMA_ZEROS_U8)
            z = (r.z[j] >> (4 * (lane & 7))) & 0xFu;  // column % 8 == lane % 8
        else
            z = r.z[j] & 0xFu;
        const uint32_t zh = 0x6400u | z, zhh = 0x5400u | (z << 4), sv = r.s[j] & 0xFFFFu;
        zs[j] = as_h2(zh | (zh << 16));
        zshi[j] = as_h2(zhh | (zhh << 16));
        ss[j] = as_h2(sv | (sv << 16));
    }
    // 64 x 128 tile (one 32-column tile and two 32-row blocks per wave): every A fragment
    // of the stage is read up front (the scheduling barrier keeps them there), so the reads
    // have completed when the wait before the next barrier comes.  Measured against reads
    // per k-step: M = 33-128 and 256-512 at N = 4096, 14336 1-7% faster; on the 128 x 128
    // tile 1-4% slower, so it reads per k-step.
    constexpr bool kPre = C::FN == 1 && C::FM <= 2;
    f16x8 apre[kPre ? 4 : 1][C::FM];
    if constexpr (kPre) {
#pragma unroll
        for (int ks = 0; ks < 4; ++ks)
#pragma unroll
            for (int i = 0; i < C::FM; ++i) {
                const int c = (4 * L.h + ks) ^ L.a_sw[i];
                apre[ks][i] = as_f16x8(*(const WMMA_LDS u32x4*)(cur + L.a_addr[i] + (c << 4)));
            }
        __builtin_amdgcn_sched_barrier(0);  // keep the reads issued here
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        f16x8 b[C::FN];
#pragma unroll
        for (int j = 0; j < C::FN; ++j) {
            const uint32_t x = r.w[j][ks], x8 = x >> 8;
            u32x4 bv;
            bv[0] = as_u32((as_h2((x & 0x000F000Fu) | magic) - zs[j]) * ss[j]);
            bv[1] = as_u32((as_h2((x & 0x00F000F0u) | magic_hi) - zshi[j]) * ss[j]);
            bv[2] = as_u32((as_h2((x8 & 0x000F000Fu) | magic) - zs[j]) * ss[j]);
            bv[3] = as_u32((as_h2((x8 & 0x00F000F0u) | magic_hi) - zshi[j]) * ss[j]);
            b[j] = as_f16x8(bv);
        }
        f16x8 a[C::FM];
#pragma unroll
        for (int i = 0; i < C::FM; ++i) {
            if constexpr (kPre) {
                a[i] = apre[ks][i];
            } else {
                const int c = (4 * L.h + ks) ^ L.a_sw[i];
                a[i] = as_f16x8(*(const WMMA_LDS u32x4*)(cur + L.a_addr[i] + (c << 4)));
            }
        }
#pragma unroll
        for (int i = 0; i < C::FM; ++i)
#pragma unroll
            for (int j = 0; j < C::FN; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
    }
}

template <int BM, int BN, int WM, int WN, int NS, int ZF>
__global__ void __launch_bounds__(WM * WN * kWave)
__attribute__((amdgpu_waves_per_eu(2, 2)))
w4a16_gemm_kernel(W4Args p) {
    using C = W4GCfg<BM, BN, WM, WN, NS, ZF>;
    constexpr int FM = C::FM, FN = C::FN, TM = C::TM, TN = C::TN;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * C::A_BYTES];
    WMMA_LDS unsigned char* lds = (WMMA_LDS unsigned char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles_m * tiles_n), tiles_m, tiles_n, 4, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int KC = p.K / 64;
    const int kc0 = blockIdx.y * p.kc_per_split;
    const int nk = max(0, min(KC, kc0 + p.kc_per_split) - kc0);

    W4GLane L;
#pragma unroll
    for (int i = 0; i < C::A_DMA; ++i) {
        const int P = 64 * (wave * C::A_DMA + i) + lane;
        const int r = P >> 3, c = (P & 7) ^ swz8(r);
        L.a_off[i] = m0 + r < p.M ? (uint32_t)((r * p.lda + 8 * c) * 2) : kOobOffset;
    }
    L.a_dst = wave * C::A_DMA * 1024;
    L.h = lane >> 5;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int r = wm * TM + 32 * i + (lane & 31);
        L.a_addr[i] = r * 128;
        L.a_sw[i] = swz8(r);
    }
    // The weight resource starts at the workgroup's first column, so weight offsets stay
    // below (BN / 16) * K * 8 bytes whatever the size of the whole matrix.
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n = n0 + wn * TN + 32 * j + (lane & 31);
        const bool ok = n < p.N;
        L.w_off[j] = ok ? (uint32_t)((pk_index(n, 0, L.h, KC) - pk_index(n0, 0, 0, KC)) * 16) : kOobOffset;
        // scale / zero byte offsets at group 0
        L.s_off[j] = ok ? (uint32_t)(s_index<ZF>(p, 0, n) * 2) : kOobOffset;
        if constexpr (ZF != WMMA_ZEROS_U8)
            L.z_off[j] = ok ? (uint32_t)(z_index<ZF>(p, 0, n) * 4) : kOobOffset;
        else
            L.z_off[j] = ok ? (uint32_t)n : kOobOffset;
    }
    const __amdgpu_buffer_rsrc_t ra = make_rsrc(p.A + (int64_t)m0 * p.lda);
    const __amdgpu_buffer_rsrc_t rw = make_rsrc(p.W + pk_index(n0, 0, 0, KC));
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.S);
    const __amdgpu_buffer_rsrc_t rz = make_rsrc(p.Z);

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};
    uint32_t magic = 0x64006400u, magic_hi = 0x54005400u;
    asm volatile("" : "+v"(magic), "+v"(magic_hi));

    W4GSlot<FN> ring[NS];
    if (nk > 0) {
        // Prologue: stages 0 .. NS-2 in flight, in stage order.  The empty asm between the
        // stages keeps the compiler from regrouping their loads (it would otherwise issue
        // every scale and zero load last, and the main loop's first stages would then wait
        // for all but the last few loads -- NS - 2 stages too early).
#pragma unroll
        for (int q = 0; q < NS - 1; ++q) {
            w4g_issue<C, ZF>(p, L, ra, rw, rs, rz, q < nk ? kc0 + q : -1, lds + q * C::A_BYTES, ring[q]);
            asm volatile("" ::: "memory");
        }
        // Main loop, unrolled by NS so every register-ring slot is a static index.  Stage
        // t reads LDS slot t % NS and ring[t % NS]; it issues stage t + NS - 1 into LDS slot
        // (t - 1) % NS and ring[(t - 1) % NS], both free once this stage's barrier passed.
        // The full ring turns run a body with no branch (every stage computes; issues past
        // the end are out-of-range loads, not skipped ones), so the compiler's own vmcnt
        // waits stay exact across the back edge; the last nk % NS stages follow.
        const int full_turns = nk / NS;
        for (int t0 = 0; t0 < full_turns * NS; t0 += NS) {
#pragma unroll
            for (int q = 0; q < NS; ++q) {
                wait_vmcnt<(NS - 2) * C::PER>();
                // lgkmcnt(0): this wave's LDS reads of the previous stage are done before
                // the barrier, after which the stage's DMA overwrites that slot.  Without it
                // the compiler left up to 6 reads in flight across the barrier, and a DMA
                // that won the race fed stale rows to one wave's MFMAs (seen on MI355X with
                // the 128 x 128 tile and a K split: 8-row groups of one wave's columns).
                __builtin_amdgcn_s_waitcnt(0xC07F);
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                const int tn_ = t0 + q + NS - 1;
                w4g_stage<C, ZF>(p, L, ra, rw, rs, rz, lds + q * C::A_BYTES,
                                 lds + ((q + NS - 1) % NS) * C::A_BYTES,
                                 tn_ < nk ? kc0 + tn_ : -1, ring[q], ring[(q + NS - 1) % NS],
                                 true, lane, magic, magic_hi, acc);
            }
        }
        const int t1 = full_turns * NS;
#pragma unroll
        for (int q = 0; q < NS - 1; ++q) {
            if (t1 + q < nk) {  // uniform
                wait_vmcnt<(NS - 2) * C::PER>();
                __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0), as in the loop above
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                w4g_stage<C, ZF>(p, L, ra, rw, rs, rz, lds + q * C::A_BYTES,
                                 lds + ((q + NS - 1) % NS) * C::A_BYTES, -1, ring[q],
                                 ring[(q + NS - 1) % NS], true, lane, magic, magic_hi, acc);
            }
        }
        wait_vmcnt<0>();
    }

    // Epilogue.  D: lane column lane%32, element r -> row 8*(r/4) + 4*(lane/32) + r%4.
    const bool partial = gridDim.y > 1;
    float* out = partial ? p.ws + (size_t)blockIdx.y * (size_t)p.M * (size_t)p.N : p.Y;
    const int64_t ldo = partial ? (int64_t)p.N : p.ldy;
    const int row0 = m0 + wm * TM + 4 * L.h, col0 = n0 + wn * TN + (lane & 31);
    const bool full = m0 + BM <= p.M && n0 + BN <= p.N;
    // Full tiles whose rows take 16-byte (fp32) or 8-byte (fp16) vectors go through the
    // shuffled epilogue; the A ring's LDS holds CH rows of the tile at a time.
    const bool half = !partial && p.y_half;
    const bool vec_ok = full && ldo % 4 == 0 &&
                        (reinterpret_cast<uintptr_t>(out) & (half ? 7u : 15u)) == 0;
    if (vec_ok) {
        constexpr int LDS_ROWS = NS * C::A_BYTES / (BN * 4);
        constexpr int CH = LDS_ROWS >= BM ? BM : (LDS_ROWS >= 128 ? 128 : (LDS_ROWS >= 64 ? 64 : 32));
        static_assert(CH * BN * 4 <= NS * C::A_BYTES, "shuffle chunk exceeds the LDS ring");
        shuffle_epilogue<BM, BN, WM, WN, CH>(
            reinterpret_cast<float*>(smem), acc, wm, wn, lane, [&](int r, int c, float4 v) {
                const int64_t idx = (int64_t)(m0 + r) * ldo + n0 + c;
                if (half) {
                    typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
                    f16x4_t hv = {(f16)v.x, (f16)v.y, (f16)v.z, (f16)v.w};
                    *reinterpret_cast<f16x4_t*>(reinterpret_cast<f16*>(p.Y) + idx) = hv;
                } else {
                    *reinterpret_cast<float4*>(out + idx) = v;
                }
            });
        return;
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = row0 + 32 * i + 8 * (r >> 2) + (r & 3), col = col0 + 32 * j;
                if (full || (row < p.M && col < p.N)) {
                    if (partial)
                        out[(int64_t)row * ldo + col] = acc[i][j][r];
                    else
                        store_y(p, (int64_t)row * ldo + col, acc[i][j][r]);
                }
            }
}

// W4A16 GEMM configurations: BM x BN, all with one row of 4 waves (each weight of a tile
// is dequantised by one wave only; a 2 x 2 grid dequantises every weight in both wave
// rows and measured 4-11% slower at M = 64..256) and a 4-deep ring (6 or 8 stages
// measured no faster).
//   wide   128 x 256, wave tile 128 x 64 (64 KB LDS): grids of at least one tile per CU
//   mid    128 x 128, wave tile 128 x 32 (64 KB LDS)
//   short   64 x 128, wave tile  64 x 32 (32 KB LDS): M <= 128, or tiles within one wave
// (A 256 x 256 tile of 2 x 4 waves spills registers at two waves per SIMD; measured 5-26%
// slower than 128 x 256 at M = 1024 .. 2048.)
enum { W4G_TILE_WIDE = 0, W4G_TILE_MID = 1, W4G_TILE_SHORT = 2 };
constexpr int kW4gTileM[3] = {128, 128, 64};
constexpr int kW4gTileN[3] = {256, 128, 128};

template <int ZF>
void launch_w4g(const W4Args& a, int cfg, dim3 grid, hipStream_t stream) {
    if (cfg == W4G_TILE_WIDE)
        hipLaunchKernelGGL((w4a16_gemm_kernel<128, 256, 1, 4, 4, ZF>), grid, dim3(4 * kWave), 0, stream, a);
    else if (cfg == W4G_TILE_MID)
        hipLaunchKernelGGL((w4a16_gemm_kernel<128, 128, 1, 4, 4, ZF>), grid, dim3(4 * kWave), 0, stream, a);
    else
        hipLaunchKernelGGL((w4a16_gemm_kernel<64, 128, 1, 4, 4, ZF>), grid, dim3(4 * kWave), 0, stream, a);
}

// ------------------------------------------------------------------ MFMA (M > GV_MAXM) --
// D = W^T A^T on MFMA 32x32x16: matrix rows are weight columns n, matrix columns are
// activation rows m.  Workgroup: 4 waves along N, each wave WNT 32-column tiles; the
// activation tile [BM x 64] of each K chunk is staged in LDS (double-buffered) and shared
// by the four waves; each wave streams its own weight blocks from HBM and dequantises
// them in registers.  BM = 32*MT rows per workgroup.
constexpr int WQ_WAVES = 4;

template <int WNT, int MT, int ZF>
__global__ void __launch_bounds__(WQ_WAVES * kWave)
w4a16_mfma_kernel(W4Args p) {
    constexpr int BM = 32 * MT;
    constexpr int A_CH = BM * 8;  // 16-byte chunks per stage
    constexpr int NT = WQ_WAVES * kWave;
    constexpr int A_PER = (A_CH + NT - 1) / NT;
    __shared__ u32x4 sa[2][A_CH];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int KC = p.K / 64;
    const int kc0 = blockIdx.y * p.kc_per_split;
    const int kc1 = min(KC, kc0 + p.kc_per_split);
    const int m0 = blockIdx.z * BM;
    const int ntile0 = (blockIdx.x * WQ_WAVES + wave) * WNT;  // first 32-col tile of wave
    const int ntiles = p.N / 32;
    const int h = lane >> 5;

    f32x16 acc[WNT][MT];
#pragma unroll
    for (int j = 0; j < WNT; ++j)
#pragma unroll
        for (int i = 0; i < MT; ++i) acc[j][i] = f32x16{};

    u32x4 ra[A_PER];
    auto gload_a = [&](int kc) {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(p.A + (int64_t)m0 * p.lda + kc * 64);
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int v = tid + i * NT;
            const int r = v >> 3, c = v & 7;
            const bool ok = (A_CH % NT == 0 || v < A_CH) && (m0 + r < p.M);
            ra[i] = buf_load16(rs, ok ? (uint32_t)((r * p.lda + c * 8) * 2) : kOobOffset);
        }
    };
    auto sstore_a = [&](int buf) {
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int v = tid + i * NT;
            if (A_CH % NT == 0 || v < A_CH) {
                const int r = v >> 3, c = v & 7;
                sa[buf][r * 8 + (c ^ swz8(r))] = ra[i];
            }
        }
    };

    const int nk = kc1 > kc0 ? kc1 - kc0 : 0;
    if (nk > 0) {
        gload_a(kc0);
        sstore_a(0);
    }
    __syncthreads();
    for (int it = 0; it < nk; ++it) {
        const int kc = kc0 + it;
        const int cur = it & 1;
        const bool more = it + 1 < nk;
        if (more) gload_a(kc + 1);
        // weights of this chunk for each of the wave's column tiles
        u32x4 wv[WNT];
        uint32_t zs[WNT], ss[WNT];
#pragma unroll
        for (int j = 0; j < WNT; ++j) {
            const int nt = ntile0 + j;
            if (nt < ntiles) {
                wv[j] = __builtin_nontemporal_load(p.W + pk_index(32 * nt + (lane & 31), kc, h, KC));
                group_params<ZF>(p, (kc * 64 + 32 * h) / p.G, 32 * nt + (lane & 31), &zs[j], &ss[j]);
            } else {
                wv[j] = u32x4{};
                zs[j] = 0x64006400u;
                ss[j] = 0;
            }
        }
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            f16x8 wf[WNT];
#pragma unroll
            for (int j = 0; j < WNT; ++j) {
                uint32_t d[4];
                dequant_word(wv[j][w], zs[j], ss[j], d);
                wf[j] = as_f16x8(u32x4{d[0], d[1], d[2], d[3]});
            }
            // activation operand: row m0 + 32*i + lane%32, k = kc*64 + 32*h + 8*w + 0..7
            const int ch = 4 * h + w;
#pragma unroll
            for (int i = 0; i < MT; ++i) {
                const int r = 32 * i + (lane & 31);
                const f16x8 af = as_f16x8(sa[cur][r * 8 + (ch ^ swz8(r))]);
#pragma unroll
                for (int j = 0; j < WNT; ++j) acc[j][i] = mfma32(wf[j], af, acc[j][i]);
            }
        }
        if (more) sstore_a(cur ^ 1);
        __syncthreads();
    }

    // D: lane column (m) = lane%32; element r -> row (n) 8*(r/4) + 4*(lane/32) + r%4.
    const bool partial = p.split > 1;
#pragma unroll
    for (int j = 0; j < WNT; ++j) {
        const int nt = ntile0 + j;
        if (nt >= ntiles) continue;
#pragma unroll
        for (int i = 0; i < MT; ++i) {
            const int m = m0 + 32 * i + (lane & 31);
            if (m >= p.M) continue;
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int n = 32 * nt + 8 * (r >> 2) + 4 * h + (r & 3);
                if (partial)
                    p.ws[((int64_t)blockIdx.y * p.M + m) * p.N + n] = acc[j][i][r];
                else
                    store_y(p, (int64_t)m * p.ldy + n, acc[j][i][r]);
            }
        }
    }
}

template <int W>
__global__ void __launch_bounds__(256)
w4a16_reduce_kernel(const float* ws, int split, float* Y, int64_t ldy, int M, int N, int y_half) {
    const int64_t total = (int64_t)M * N;
    const int nv = (N + W - 1) / W;
    for (int row = blockIdx.y; row < M; row += gridDim.y) {
        for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < nv; q += gridDim.x * blockDim.x) {
            const int col = q * W;
            float v[W];
            splitk_sum<W>(ws + (int64_t)row * N + col, total, split, v);
#pragma unroll
            for (int e = 0; e < W; ++e) {
                if (y_half)
                    reinterpret_cast<f16*>(Y)[(int64_t)row * ldy + col + e] = (f16)v[e];
                else
                    Y[(int64_t)row * ldy + col + e] = v[e];
            }
        }
    }
}

// Dynamic LDS of the decode kernel: activations plus two fp32 sums per 32-value run.
size_t decode_lds_bytes(int M, int K) { return (size_t)M * K * 2 + (size_t)M * (K / 32) * 8; }

// Dynamic LDS the decode kernels may request without raising the launch limit.
constexpr size_t kDecodeLdsMax = 48 * 1024;

bool w4a16_use_decode(int M, int N, int K, int num_cus) {
    if (num_cus <= 0) num_cus = 256;
    return M >= 1 && M <= GV_MAXM && K % 128 == 0 && decode_lds_bytes(M, K) <= kDecodeLdsMax &&
           N / 16 >= num_cus / 2;
}

int grid_for(int64_t work, int per_block) {
    int64_t b = (work + per_block - 1) / per_block;
    return (int)std::min<int64_t>(std::max<int64_t>(b, 1), 65535);
}

}  // namespace

hipError_t launch_int4_prepack(const int32_t* qweight, int K, int N, int32_t* packed,
                               hipStream_t stream) {
    const int64_t total = (int64_t)(N / 32) * (K / 64) * 64;
    hipLaunchKernelGGL(int4_prepack_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                       qweight, K, N, packed);
    return hipGetLastError();
}

hipError_t launch_int4_unprepack(const int32_t* packed, int K, int N, int32_t* qweight,
                                 hipStream_t stream) {
    const int64_t total = (int64_t)(N / 32) * (K / 64) * 64;
    hipLaunchKernelGGL(int4_unprepack_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                       packed, K, N, qweight);
    return hipGetLastError();
}

hipError_t launch_int4_unpack(const int32_t* qweight, int K, int N, uint8_t* q,
                              hipStream_t stream) {
    const int64_t total = (int64_t)(K / 8) * N;
    hipLaunchKernelGGL(int4_unpack_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                       qweight, K, N, q);
    return hipGetLastError();
}

hipError_t launch_int4_from_awq(const int32_t* qweight_awq, const int32_t* qzeros_awq, int K,
                                int N, int KG, int32_t* qweight, int32_t* zeros,
                                hipStream_t stream) {
    const int64_t total = (int64_t)(K / 8) * N + (int64_t)KG * (N / 8);
    hipLaunchKernelGGL(int4_from_awq_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                       qweight_awq, qzeros_awq, K, N, KG, qweight, zeros);
    return hipGetLastError();
}

hipError_t launch_int4_gptq_zeros(const int32_t* qzeros, int KG, int N, int add, int32_t* zeros,
                                  int32_t* overflow, hipStream_t stream) {
    const int64_t words = (int64_t)KG * (N / 8);
    hipLaunchKernelGGL(int4_gptq_zeros_kernel, dim3(grid_for(words, 256)), dim3(256), 0, stream,
                       qzeros, words, (uint32_t)add, zeros, overflow);
    return hipGetLastError();
}

hipError_t launch_int4_permute_rows(const int32_t* qweight, const int32_t* perm, int K, int N,
                                    int32_t* out, hipStream_t stream) {
    const int64_t total = (int64_t)(K / 8) * N;
    hipLaunchKernelGGL(int4_permute_rows_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                       qweight, perm, K, N, out);
    return hipGetLastError();
}

hipError_t launch_int4_params_slice(const void* scales, const void* zeros, int zeros_format,
                                    int KG, int N, void* scales_out, int32_t* zeros_out,
                                    hipStream_t stream) {
    const int64_t total = (int64_t)(N / 16) * KG;
    const auto* s = static_cast<const uint16_t*>(scales);
    auto* so = static_cast<uint16_t*>(scales_out);
    if (zeros_format == WMMA_ZEROS_PACKED)
        hipLaunchKernelGGL(int4_params_slice_kernel<WMMA_ZEROS_PACKED>, dim3(grid_for(total, 256)),
                           dim3(256), 0, stream, s, zeros, KG, N, so, zeros_out);
    else
        hipLaunchKernelGGL(int4_params_slice_kernel<WMMA_ZEROS_U8>, dim3(grid_for(total, 256)),
                           dim3(256), 0, stream, s, zeros, KG, N, so, zeros_out);
    return hipGetLastError();
}

hipError_t launch_int4_prepack_fused(const int32_t* qweight, const void* scales, const void* zeros,
                                     int zeros_format, int K, int N, int G, int32_t* fused,
                                     hipStream_t stream) {
    const int64_t total = (int64_t)(N / 16) * (fused_slice_bytes(K) / 16);
    const auto* s = static_cast<const uint16_t*>(scales);
    if (zeros_format == WMMA_ZEROS_PACKED)
        hipLaunchKernelGGL(int4_prepack_fused_kernel<WMMA_ZEROS_PACKED>, dim3(grid_for(total, 256)),
                           dim3(256), 0, stream, qweight, s, zeros, K, N, G, fused);
    else
        hipLaunchKernelGGL(int4_prepack_fused_kernel<WMMA_ZEROS_U8>, dim3(grid_for(total, 256)),
                           dim3(256), 0, stream, qweight, s, zeros, K, N, G, fused);
    return hipGetLastError();
}

hipError_t launch_int4_unprepack_fused(const int32_t* fused, int K, int N, int G, int32_t* qweight,
                                       void* scales, int32_t* zeros, hipStream_t stream) {
    const int64_t total = (int64_t)(N / 16) * (K / 128) * 64 + (int64_t)(K / G) * (N / 16);
    hipLaunchKernelGGL(int4_unprepack_fused_kernel, dim3(grid_for(total, 256)), dim3(256), 0,
                       stream, fused, K, N, G, qweight, static_cast<uint16_t*>(scales), zeros);
    return hipGetLastError();
}

// Dynamic LDS the matrix-pipe decode may take: M = 3, 4 past one round stage 49.9 / 66.6 KB
// (two workgroups per CU).  Measured at N = 4096, K = 8192 / 14336: this kernel 7.0 / 10.0
// (M = 3) and 7.0 / 10.7 us (M = 4) against 16.2 / 26.6 and 18.0 / 29.4 us for the split
// GEMV the planner took under a 48 KB limit.
constexpr size_t kDecodeMfmaLdsMax = 96 * 1024;

bool w4a16_fused_decode_ok(int M, int K) {
    return M >= 0 && M <= DM_MAXM && K % 128 == 0 &&
           decode_mfma_lds_bytes(std::max(M, 1), K) <= kDecodeMfmaLdsMax;
}

// Launch model of the W4A16 GEMM for 32 < M <= kW4gModelMaxM: a workgroup streams its
// activation rows (those that exist) and its tile's int4 columns over its K range at a
// per-CU rate, or is held by its MFMA work, plus 1 us; the launch takes that per wave of
// workgroups, plus 2 us and 0.5 us per MB of partial sums with a K split.  Constants set
// by coordinate search on the planning loss over every tile x split 1-8 timed at 128
// shapes (M = 33-1024, N = 1024-14336, K = 2048-14336, graph-replayed): fitted on half the
// K values it takes 1.3% / 0.5% more time than the fastest plan per shape on the other
// half, against 2.5% / 1.4% for the tile-count rule it replaced (up to 1.22x faster:
// 64 x 14336 x 2048 16.1 -> 13.2 us unsplit; 128 x 11008 x 14336 67.3 -> 59.7 us with
// 128 x 256 tiles split 4).
constexpr int kW4gModelMaxM = 1024;
constexpr double kW4gKbPerUs[3] = {40, 35, 35};      // per tile config (W4G_TILE_*)
constexpr double kW4gMflopPerUs[3] = {4, 4, 3};
// The rows kernel (W4_ROWS) in the same model: a workgroup of 16*mb rows x 16*nh columns
// reads its activation rows and int4 columns over all of K at kRowsKbPerUs, plus a fixed
// cost per configuration (the final cross-wave sum grows with the tile), per wave of
// workgroups; no split.  Fitted the same way, on 189 shapes (M = 33-1024, N = 512-14336,
// K = 1024-8192; each configuration below and the LDS-DMA plan timed in one process): the
// model's choices take 0.1% more time than the fastest of them per shape, against 13.3% for
// the LDS-DMA plans alone; each K value held out in turn, the constants fitted on the
// others choose within 0-4% of the fastest on it.  It takes the rows kernel at short K and
// few columns (K = 2048, N = 1024, M = 33-256: 4.6-5.6 us against 7.9-10.4) and the
// LDS-DMA tiles elsewhere.
constexpr double kRowsKbPerUs = 45;
constexpr int kRowsCfg[3][2] = {{1, 2}, {1, 4}, {2, 4}};  // {mb, nh}
constexpr double kRowsWgFixedUs[3] = {0.75, 1.0, 2.0};

// Shapes the rows kernel takes: whole 128-deep pair-steps inside one group, and weights
// addressable with 32-bit byte offsets.
bool rows_shape_ok(int N, int K, int G) {
    return K % 128 == 0 && G % 128 == 0 && ((G / 128) & (G / 128 - 1)) == 0 &&
           (int64_t)N * K < ((int64_t)1 << 32);
}

// Tile config and split of the LDS-DMA GEMM, or (rows_mb > 0) the rows kernel's shape.
void w4g_model_plan(int M, int N, int K, int G, int num_cus, int* cfg_out, int* split_out,
                    int* rows_mb, int* rows_nh) {
    const int KC = K / 64;
    double best_t = 1e300;
    *cfg_out = W4G_TILE_SHORT;
    *split_out = 1;
    *rows_mb = *rows_nh = 0;
    for (int cfg : {W4G_TILE_SHORT, W4G_TILE_MID, W4G_TILE_WIDE}) {
        const int bm = kW4gTileM[cfg], bn = kW4gTileN[cfg];
        for (int sp : {1, 2, 4, 8}) {
            if (sp > 1 && (K <= 1024 || KC < 4 * sp)) continue;
            const int kcps = ceil_div(KC, sp), s = ceil_div(KC, kcps);
            const double kk = kcps * 64.0;
            const int64_t wgs = (int64_t)ceil_div(M, bm) * ceil_div(N, bn) * s;
            const double kb = (std::min(M, bm) * 2.0 + bn / 2.0) * kk / 1000.0;
            const double mflop = 2.0 * bm * bn * kk / 1e6;
            double t = (double)((wgs + num_cus - 1) / num_cus) *
                       (1.0 + std::max(kb / kW4gKbPerUs[cfg], mflop / kW4gMflopPerUs[cfg]));
            if (s > 1) t += 2.0 + 0.5 * (s + 1) * 4.0 * M * N / 1e6;
            if (t < best_t * 0.999) {
                best_t = t;
                *cfg_out = cfg;
                *split_out = sp;
            }
        }
    }
    if (!rows_shape_ok(N, K, G)) return;
    for (int c = 0; c < 3; ++c) {
        const int mb = kRowsCfg[c][0], nh = kRowsCfg[c][1];
        if (N % (16 * nh) != 0) continue;
        const int64_t wgs = (int64_t)(N / (16 * nh)) * ceil_div(M, 16 * mb);
        const double kb = (std::min(M, 16 * mb) * 2.0 + 8.0 * nh) * K / 1000.0;
        const double t =
            (double)((wgs + num_cus - 1) / num_cus) * (kRowsWgFixedUs[c] + kb / kRowsKbPerUs);
        if (t < best_t * 0.999) {
            best_t = t;
            *rows_mb = mb;
            *rows_nh = nh;
        }
    }
}

// 4 < M <= 32: the skinny kernel's plan (skinny_config) against the rows kernel, both in
// the units of the model above.  The skinny launch: slices x K splits workgroups, each
// reading its rows' activations and its columns' int4 weights over its K range at
// kW4SkKbPerUs plus kW4SkWgFixedUs, per wave of workgroups, plus kW4SkSplitUs and
// kW4SkPartialUsPerMB per MB of partial sums with a split.  The rows kernel here also has
// a 16 x 16 configuration.  Fitted on 120 shapes (M = 5-32, N = 1024-14336,
// K = 2048-14336; the skinny plan and four rows configurations timed in one process): the
// model's choices take 0.4% more time than the fastest per shape, against 6.3% for the
// skinny plans alone (M = 32, K = 2048, N = 1024-2048: 4.4 us against 6.3-6.4; M = 32,
// N = K = 4096: 7.3 against 9.4; M = 5-16 keep the skinny kernel except at long K and wide
// N).
constexpr double kW4SkKbPerUs = 60, kW4SkWgFixedUs = 0.25, kW4SkSplitUs = 3.0,
                 kW4SkPartialUsPerMB = 0.5, kRowsSmallFixedUs = 0.5;

bool rows_beats_skinny(int M, int N, int K, int G, int num_cus, int nh, int u, int* mb_out,
                       int* nh_out) {
    if (!rows_shape_ok(N, K, G)) return false;
    const int kps = SK_NW * u * 128, sp = ceil_div(K, kps);
    const int skmb = M <= 16 ? 1 : 2;
    const int64_t sk_wgs = (int64_t)(N / (16 * nh)) * sp;
    const double sk_kb = (std::min(M, 16 * skmb) * 2.0 + 8.0 * nh) * std::min(K, kps) / 1000.0;
    double best = (double)((sk_wgs + num_cus - 1) / num_cus) * (kW4SkWgFixedUs + sk_kb / kW4SkKbPerUs);
    if (sp > 1) best += kW4SkSplitUs + kW4SkPartialUsPerMB * (sp + 1) * 4.0 * M * N / 1e6;
    bool rows = false;
    for (int c = -1; c < 3; ++c) {
        const int mb = c < 0 ? 1 : kRowsCfg[c][0], rnh = c < 0 ? 1 : kRowsCfg[c][1];
        const double fixed = c < 0 ? kRowsSmallFixedUs : kRowsWgFixedUs[c];
        if (N % (16 * rnh) != 0) continue;
        const int64_t wgs = (int64_t)(N / (16 * rnh)) * ceil_div(M, 16 * mb);
        const double kb = (std::min(M, 16 * mb) * 2.0 + 8.0 * rnh) * K / 1000.0;
        const double t = (double)((wgs + num_cus - 1) / num_cus) * (fixed + kb / kRowsKbPerUs);
        if (t < best * 0.999) {
            best = t;
            rows = true;
            *mb_out = mb;
            *nh_out = rnh;
        }
    }
    return rows;
}

// M <= 4 rows against few columns and a long K: the decode gives one workgroup per
// 16-column slice, each walking all of K, so with under num_cus / 4 slices a K-split skinny
// launch finishes first.  Measured on MI355X (256 CUs), decode against skinny, us:
//   K = 8192,  N = 128 / 256: M = 3 5.1 / 5.3 vs 4.6 / 4.7; M = 2 4.4 / 4.6 vs 4.6 / 4.6;
//   K = 11008, N = 512: M = 2 5.7 vs 5.3, M = 4 7.1 vs 5.6; N = 1024: M = 2 6.0 vs 6.7,
//              M = 3 7.1 vs 6.7;
//   K = 14336, N = 256: M = 4 7.6 vs 5.5; N = 1024: M = 4 7.9 vs 7.3; N = 1536: M = 4 8.1
//              vs 9.0;
//   K <= 6144 the decode at every N <= 1024, M <= 4 (N = 1024, M = 4: 4.8 vs 6.7).
bool w4a16_narrow_skinny(int M, int N, int K, int num_cus) {
    const int slices = N / 16;
    int min_m = DM_MAXM + 1;
    if (8 * slices <= num_cus)
        min_m = K >= 10240 ? 2 : (K >= 8192 ? 3 : DM_MAXM + 1);
    else if (4 * slices <= num_cus)
        min_m = K >= 10240 ? 3 : DM_MAXM + 1;
    return M >= min_m && M <= DM_MAXM;
}

// Host-only: choose the kernel and K split.
//   decode-mfma  M <= 4, G = 128 * 2^j, K % 128 == 0 and the staged activations fit LDS, at
//                any N (narrow N included: at N = 256..1536, K = 1024..14336 it runs
//                1.2-2.5x faster than the split GEMV), except the narrow, long-K shapes
//                above, which take the skinny kernel.
//   decode       M <= 4 where the 16-column slices give at least half a workgroup per CU,
//                other group sizes.
//   gemv-split   other M <= 4 shapes: one workgroup per 32 columns, K split (plus a reduce
//                pass) only when fewer than 2*CUs workgroups would exist.
//   skinny       4 < M <= 32 (and the narrow, long-K M <= 4 shapes) with G = 128 * 2^j: 16,
//                32 or 64 columns per workgroup, K split (plus a reduce pass) only when the
//                tiles alone give under half a workgroup per CU.
//   gemm         M > 32 with G a power of two: LDS-DMA MFMA GEMM (tile below), K split
//                (plus a reduce pass) only when the tiles cannot fill the chip.
//   rows         4 < M <= 1024 with G = 128 * 2^j where the launch model prefers it to
//                the skinny plan (M <= 32) or to every LDS-DMA plan (short K, few
//                columns): no ring, no split.
//   mfma         everything else (the shapes the kernels above do not take).
W4A16Plan w4a16_plan(int M, int N, int K, int G, int num_cus, bool aligned) {
    if (num_cus <= 0) num_cus = 256;
    W4A16Plan pl{};
    pl.split = 1;
    pl.k_per_split = K;
    (void)aligned;
    const bool g_ok = G % 128 == 0 && ((G / 128) & (G / 128 - 1)) == 0;
    const bool narrow_skinny = K % 128 == 0 && g_ok && w4a16_narrow_skinny(M, N, K, num_cus);
    if (M >= 1 && M <= DM_MAXM && K % 128 == 0 && g_ok && !narrow_skinny &&
        decode_mfma_lds_bytes(M, K) <= kDecodeMfmaLdsMax) {
        pl.kind = W4_DECODE_MFMA;
        return pl;
    }
    if (!narrow_skinny && w4a16_use_decode(M, N, K, num_cus)) {
        pl.kind = W4_DECODE;
        return pl;
    }
    if ((M > DM_MAXM || narrow_skinny) && M <= 32 && K % 128 == 0 && g_ok) {
        int nh = 2, u = 1;
        skinny_config(M, N, K, num_cus, &nh, &u);
        int mb, rnh;
        if (M > DM_MAXM && rows_beats_skinny(M, N, K, G, num_cus, nh, u, &mb, &rnh)) {
            pl.kind = W4_ROWS;
            pl.mb = mb;
            pl.big = rnh;
            pl.k_per_split = K;
            return pl;
        }
        pl.big = nh;
        pl.kind = W4_SKINNY;
        pl.k_per_split = SK_NW * u * 128;
        pl.split = ceil_div(K, pl.k_per_split);
        return pl;
    }
    const int KC = K / 64;
    if (M > 32 && (G & (G - 1)) == 0) {
        // LDS-DMA W4A16 GEMM.  M <= 1024: the tile (64 x 128, 128 x 128, 128 x 256) and the
        // K split (1, 2, 4, 8) with the shortest modelled time (w4g_model_plan).  Larger M
        // (measured at K = 4096, N in {4096, 11008, 14336}): 64 x 128 while its tiles fit
        // one wave of the CUs; 128 x 256 when those tiles give at least one per CU, in whole
        // multiples of the CU count or 1.7 of them (M = 2048: 5-26% faster than 128 x 128;
        // M = 1024, N = 11008, 1.34 tiles per CU: 4% slower); else 128 x 128.
        int cfg, s = 1;
        if (M <= kW4gModelMaxM) {
            int mb, nh;
            w4g_model_plan(M, N, K, G, num_cus, &cfg, &s, &mb, &nh);
            if (mb > 0) {
                pl.kind = W4_ROWS;
                pl.mb = mb;
                pl.big = nh;
                pl.k_per_split = K;
                return pl;
            }
        } else {
            const int64_t wide_tiles = (int64_t)ceil_div(M, 128) * ceil_div(N, 256);
            const int64_t short_tiles = (int64_t)ceil_div(M, 64) * ceil_div(N, 128);
            cfg = W4G_TILE_MID;
            if (short_tiles <= num_cus)
                cfg = W4G_TILE_SHORT;
            else if (wide_tiles >= num_cus &&
                     (wide_tiles % num_cus == 0 || 10 * wide_tiles >= 17 * (int64_t)num_cus))
                cfg = W4G_TILE_WIDE;
            // Split while the tiles do not give one per CU: num_cus / tiles ways, at most 8,
            // never at K <= 1024.
            const int64_t tiles = (int64_t)ceil_div(M, kW4gTileM[cfg]) * ceil_div(N, kW4gTileN[cfg]);
            if (tiles < num_cus && K > 1024)
                s = (int)std::min<int64_t>(std::max<int64_t>(num_cus / tiles, 1), 8);
            s = std::max(1, std::min(s, KC / 4));
        }
        pl.big = cfg;
        const int kcps = ceil_div(KC, s);
        pl.kind = W4_GEMM;
        pl.split = ceil_div(KC, kcps);
        pl.k_per_split = kcps * 64;
        return pl;
    }
    const bool use_mfma = M > GV_MAXM;
    int64_t blocks;
    if (!use_mfma) {
        blocks = N / 32;
    } else {
        const int wnt = M >= 256 ? 2 : 1;
        const int mt = M > 32 ? 4 : 1;
        blocks = (int64_t)ceil_div(N / 32, WQ_WAVES * wnt) * ceil_div(M, 32 * mt);
    }
    int s = 1;
    const int64_t target = use_mfma ? num_cus : 2 * num_cus;
    if (blocks < target) s = (int)std::min<int64_t>((target + blocks - 1) / blocks, 16);
    // each split is whole 64-deep chunks; a lane's 32 K values stay inside one group
    // whenever G % 32 == 0.
    int kcps = ceil_div(KC, s);
    s = ceil_div(KC, kcps);
    pl.kind = use_mfma ? W4_MFMA : W4_GEMV_SPLIT;
    pl.split = s;
    pl.k_per_split = kcps * 64;
    return pl;
}

namespace {

template <int ZF>
hipError_t launch_w4a16_zf(const W4Args& a, const W4A16Launch& w, hipStream_t stream) {
    const int ntiles = w.N / 32;
    const W4A16Plan& pl = w.plan;
    if (pl.kind == W4_DECODE_MFMA) {
        const size_t lds = decode_mfma_lds_bytes(w.M, w.K);
        const dim3 grid(w.N / 16), block(DM_NW * kWave);
        if (decode_mfma_one(w.K))
            launch_decode_mfma<ZF, true>(a, w.M, grid, block, lds, stream);
        else
            launch_decode_mfma<ZF, false>(a, w.M, grid, block, lds, stream);
        return hipGetLastError();
    }
    if (pl.kind == W4_DECODE) {
        const size_t lds = decode_lds_bytes(w.M, w.K);
        const dim3 grid(w.N / 16), block(DV_NW * kWave);
        if (w.K <= DV_NW * DV_U * 128) {
            switch (w.M) {
                case 1: hipLaunchKernelGGL((w4a16_decode_kernel<1, ZF, true>), grid, block, lds, stream, a); break;
                case 2: hipLaunchKernelGGL((w4a16_decode_kernel<2, ZF, true>), grid, block, lds, stream, a); break;
                case 3: hipLaunchKernelGGL((w4a16_decode_kernel<3, ZF, true>), grid, block, lds, stream, a); break;
                default: hipLaunchKernelGGL((w4a16_decode_kernel<4, ZF, true>), grid, block, lds, stream, a); break;
            }
        } else {
            switch (w.M) {
                case 1: hipLaunchKernelGGL((w4a16_decode_kernel<1, ZF, false>), grid, block, lds, stream, a); break;
                case 2: hipLaunchKernelGGL((w4a16_decode_kernel<2, ZF, false>), grid, block, lds, stream, a); break;
                case 3: hipLaunchKernelGGL((w4a16_decode_kernel<3, ZF, false>), grid, block, lds, stream, a); break;
                default: hipLaunchKernelGGL((w4a16_decode_kernel<4, ZF, false>), grid, block, lds, stream, a); break;
            }
        }
        return hipGetLastError();
    }
    if (pl.kind == W4_GEMM) {
        const int bm = kW4gTileM[pl.big], bn = kW4gTileN[pl.big];
        const dim3 grid(ceil_div(w.M, bm) * ceil_div(w.N, bn), pl.split);
        launch_w4g<ZF>(a, pl.big, grid, stream);
    } else if (pl.kind == W4_ROWS) {
        const dim3 grid(w.N / (16 * pl.big), 1, ceil_div(w.M, 16 * pl.mb));
        if (pl.mb == 1 && pl.big == 1)
            launch_rows<ZF, 1, 1>(a, grid, stream);
        else if (pl.mb == 1 && pl.big == 2)
            launch_rows<ZF, 1, 2>(a, grid, stream);
        else if (pl.mb == 1)
            launch_rows<ZF, 1, 4>(a, grid, stream);
        else
            launch_rows<ZF, 2, 4>(a, grid, stream);
    } else if (pl.kind == W4_SKINNY) {
        const int U = pl.k_per_split / (SK_NW * 128);
        const dim3 grid(w.N / (16 * pl.big), pl.split);
        if (w.M <= 16) {
            if (pl.big == 4)
                launch_skinny_mb<ZF, 1, 4>(a, U, grid, stream);
            else if (pl.big == 2)
                launch_skinny_mb<ZF, 1, 2>(a, U, grid, stream);
            else
                launch_skinny_mb<ZF, 1, 1>(a, U, grid, stream);
        } else {
            if (pl.big == 4)
                launch_skinny_mb<ZF, 2, 4>(a, U, grid, stream);
            else
                launch_skinny_mb<ZF, 2, 2>(a, U, grid, stream);
        }
    } else if (pl.kind == W4_GEMV_SPLIT) {
        hipLaunchKernelGGL((w4a16_gemv_kernel<ZF>), dim3(ntiles, pl.split), dim3(GV_NW * kWave), 0,
                           stream, a);
    } else {
        const int wnt = w.M >= 256 ? 2 : 1;
        const int mt = w.M > 32 ? 4 : 1;
        dim3 grid(ceil_div(ntiles, WQ_WAVES * wnt), pl.split, ceil_div(w.M, 32 * mt));
        if (wnt == 2)
            hipLaunchKernelGGL((w4a16_mfma_kernel<2, 4, ZF>), grid, dim3(WQ_WAVES * kWave), 0, stream, a);
        else if (mt == 4)
            hipLaunchKernelGGL((w4a16_mfma_kernel<1, 4, ZF>), grid, dim3(WQ_WAVES * kWave), 0, stream, a);
        else
            hipLaunchKernelGGL((w4a16_mfma_kernel<1, 1, ZF>), grid, dim3(WQ_WAVES * kWave), 0, stream, a);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pl.split <= 1) return e;
    const bool vec4 = w.N % 4 == 0 && (reinterpret_cast<uintptr_t>(w.workspace) & 15u) == 0;
    const int nv = vec4 ? w.N / 4 : w.N;
    const dim3 grid(std::min(ceil_div(nv, 256), 64), std::min(w.M, 65535));
    const float* ws = static_cast<const float*>(w.workspace);
    if (vec4)
        hipLaunchKernelGGL(w4a16_reduce_kernel<4>, grid, dim3(256), 0, stream, ws, pl.split, w.Y,
                           w.ldy, w.M, w.N, w.y_half ? 1 : 0);
    else
        hipLaunchKernelGGL(w4a16_reduce_kernel<1>, grid, dim3(256), 0, stream, ws, pl.split, w.Y,
                           w.ldy, w.M, w.N, w.y_half ? 1 : 0);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_w4a16(const W4A16Launch& w, hipStream_t stream) {
    W4Args a{};
    a.A = static_cast<const f16*>(w.A);
    a.lda = w.lda;
    a.W = reinterpret_cast<const u32x4*>(w.packed);
    a.S = static_cast<const f16*>(w.scales);
    a.Z = w.zeros;
    a.zfmt = w.zeros_format;
    a.M = w.M;
    a.N = w.N;
    a.K = w.K;
    a.G = w.G;
    a.Y = w.Y;
    a.ldy = w.ldy;
    a.ws = static_cast<float*>(w.workspace);
    a.split = w.plan.split;
    a.kc_per_split = w.plan.k_per_split / 64;
    a.kg = w.K / w.G;
    a.y_half = w.y_half ? 1 : 0;
    a.pp_shift = 0;
    while (w.G >= 128 && (128 << (a.pp_shift + 1)) <= w.G) ++a.pp_shift;
    a.g_shift = 0;
    while ((2 << a.g_shift) <= w.G) ++a.g_shift;
    if (w.zeros_format == WMMA_W4_FUSED) {
        // The fused layout is read by the matrix-pipe decode kernel only (the planner gives
        // it every shape the C-ABI accepts in this layout).
        if (w.plan.kind != W4_DECODE_MFMA) return hipErrorInvalidValue;
        const size_t lds = decode_mfma_lds_bytes(w.M, w.K);
        const dim3 grid(w.N / 16), block(DM_NW * kWave);
        if (decode_mfma_one(w.K))
            launch_decode_mfma<WMMA_W4_FUSED, true>(a, w.M, grid, block, lds, stream);
        else
            launch_decode_mfma<WMMA_W4_FUSED, false>(a, w.M, grid, block, lds, stream);
        return hipGetLastError();
    }
    if (w.zeros_format == WMMA_ZEROS_PACKED) return launch_w4a16_zf<WMMA_ZEROS_PACKED>(a, w, stream);
    if (w.zeros_format == WMMA_ZEROS_SLICED) return launch_w4a16_zf<WMMA_ZEROS_SLICED>(a, w, stream);
    return launch_w4a16_zf<WMMA_ZEROS_U8>(a, w, stream);
}

}  // namespace wmma_amd
