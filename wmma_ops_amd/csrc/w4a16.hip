// INT4 weight layout kernels and W4A16 dequant-GEMM kernels for gfx950.
//
// The reference has no INT4 code; the W4A16 path is defined by its task statement:
//   Y[M,N] (fp32) = A[M,K] (fp16) @ W,  W[k][n] = fp16((q[k][n] - z[g][n]) * s[g][n]),
//   g = k / G, q and z 4-bit unsigned, s fp16, the dequantised weight rounded once to fp16.
//
// Layouts
//   GPTQ qweight   int32 [K/8, N]: q[k][n] in bits 4*(k%8).. of qweight[k/8][n].
//   prepacked      int32 [N/32][K/64][64 lanes][4 words]: lane l of block (nt, kc) holds
//                  column n = 32*nt + l%32, words w = 0..3 for k-group
//                  kg = 8*kc + 4*(l/32) + w (k = 8*kg .. 8*kg+7).  Inside a prepacked word
//                  nibble p holds k-offset kPerm[p] = {0,2,4,6,1,3,5,7}[p], so that
//                  (word >> 4i) & 0x000F000F yields the pair (k 2i, k 2i+1) as two 16-bit
//                  lanes.  One wave reading one block issues a single contiguous 1 KB load,
//                  and each lane's 16 bytes are exactly the K-contiguous operand of four
//                  32x32x16 MFMAs for its column.
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

// Nibble position -> k offset inside a prepacked word (and its inverse).
__constant__ int kPermDev[8] = {0, 2, 4, 6, 1, 3, 5, 7};

// ---------------------------------------------------------------- layout conversions --
// One thread per (block, lane): reads four GPTQ words (coalesced along n), reorders each
// word's nibbles, writes 16 bytes.
__global__ void __launch_bounds__(256)
int4_prepack_kernel(const int32_t* __restrict__ qw, int K, int N, int32_t* __restrict__ out) {
    const int KC = K / 64;
    const int64_t total = (int64_t)(N / 32) * KC * 64;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int l = (int)(t & 63);
        const int64_t blk = t >> 6;
        const int kc = (int)(blk % KC);
        const int nt = (int)(blk / KC);
        const int n = 32 * nt + (l & 31);
        const int kg0 = 8 * kc + 4 * (l >> 5);
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
    const int64_t total = (int64_t)(N / 32) * KC * 64;
    for (int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; t < total;
         t += (int64_t)gridDim.x * blockDim.x) {
        const int l = (int)(t & 63);
        const int64_t blk = t >> 6;
        const int kc = (int)(blk % KC);
        const int nt = (int)(blk / KC);
        const int n = 32 * nt + (l & 31);
        const int kg0 = 8 * kc + 4 * (l >> 5);
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
};

// Per-lane group parameters: zs = (1024 + z, 1024 + z), ss = (s, s) as packed fp16 pairs.
__device__ __forceinline__ void group_params(const W4Args& p, int g, int n, uint32_t* zs,
                                             uint32_t* ss) {
    const uint16_t s = __builtin_bit_cast(uint16_t, p.S[(int64_t)g * p.N + n]);
    uint32_t z;
    if (p.zfmt == WMMA_ZEROS_PACKED) {
        const uint32_t zw = (uint32_t)static_cast<const int32_t*>(p.Z)[(int64_t)g * (p.N / 8) + n / 8];
        z = (zw >> (4 * (n & 7))) & 0xFu;
    } else {
        z = static_cast<const uint8_t*>(p.Z)[(int64_t)g * p.N + n] & 0xFu;
    }
    const uint32_t zh = 0x6400u | z;
    *zs = zh | (zh << 16);
    *ss = (uint32_t)s | ((uint32_t)s << 16);
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

    const u32x4* wbase = p.W + (int64_t)nt * KC * 64 + lane;
    for (int kcb = kc0 + wave; kcb < kc1; kcb += GV_NW * GV_UNROLL) {
        u32x4 wv[GV_UNROLL];
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int kc = kcb + u * GV_NW;
            if (kc < kc1) wv[u] = __builtin_nontemporal_load(wbase + (int64_t)kc * 64);
        }
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int kc = kcb + u * GV_NW;
            if (kc < kc1) {
                const int k0 = kc * 64 + 32 * h;
                uint32_t zs, ss;
                group_params(p, k0 / p.G, n, &zs, &ss);
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
                p.Y[(int64_t)m * p.ldy + col] = v;
        }
    }
}

// ------------------------------------------------------------------ MFMA (M > GV_MAXM) --
// D = W^T A^T on MFMA 32x32x16: matrix rows are weight columns n, matrix columns are
// activation rows m.  Workgroup: 4 waves along N, each wave WNT 32-column tiles; the
// activation tile [BM x 64] of each K chunk is staged in LDS (double-buffered) and shared
// by the four waves; each wave streams its own weight blocks from HBM and dequantises
// them in registers.  BM = 32*MT rows per workgroup.
constexpr int WQ_WAVES = 4;

template <int WNT, int MT>
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
                wv[j] = __builtin_nontemporal_load(p.W + ((int64_t)nt * KC + kc) * 64 + lane);
                group_params(p, (kc * 64 + 32 * h) / p.G, 32 * nt + (lane & 31), &zs[j], &ss[j]);
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
                    p.Y[(int64_t)m * p.ldy + n] = acc[j][i][r];
            }
        }
    }
}

__global__ void __launch_bounds__(256)
w4a16_reduce_kernel(const float* ws, int split, float* Y, int64_t ldy, int M, int N) {
    const int64_t total = (int64_t)M * N;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < total;
         i += (int64_t)gridDim.x * blockDim.x) {
        float v = ws[i];
        for (int s = 1; s < split; ++s) v += ws[(int64_t)s * total + i];
        Y[(i / N) * ldy + i % N] = v;
    }
}

int grid_for(int64_t work, int per_block) {
    int64_t b = (work + per_block - 1) / per_block;
    return (int)std::min<int64_t>(std::max<int64_t>(b, 1), 65535);
}

// MFMA kernel variants: (WNT, MT).
constexpr int kWqVariants[][2] = {{1, 1}, {1, 4}, {2, 4}};

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

// Host-only: choose the kernel and K split.  GEMV for M <= 4 (one workgroup per 32
// columns, K split only when fewer than 2*CUs workgroups would exist); MFMA otherwise.
void w4a16_plan(int M, int N, int K, int G, int num_cus, int* split, int* k_per_split,
                bool* mfma) {
    const int KC = K / 64;
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
    // each split must be whole chunks and, for G >= 64, whole groups are not required:
    // a lane's 32 K values stay inside one group whenever G % 32 == 0.
    int kcps = ceil_div(KC, s);
    s = ceil_div(KC, kcps);
    *split = s;
    *k_per_split = kcps * 64;
    *mfma = use_mfma;
}

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
    a.split = w.split;
    a.kc_per_split = w.k_per_split / 64;
    const int ntiles = w.N / 32;
    if (!w.mfma) {
        hipLaunchKernelGGL(w4a16_gemv_kernel, dim3(ntiles, w.split), dim3(GV_NW * kWave), 0,
                           stream, a);
    } else {
        const int wnt = w.M >= 256 ? 2 : 1;
        const int mt = w.M > 32 ? 4 : 1;
        dim3 grid(ceil_div(ntiles, WQ_WAVES * wnt), w.split, ceil_div(w.M, 32 * mt));
        if (wnt == 2)
            hipLaunchKernelGGL((w4a16_mfma_kernel<2, 4>), grid, dim3(WQ_WAVES * kWave), 0, stream, a);
        else if (mt == 4)
            hipLaunchKernelGGL((w4a16_mfma_kernel<1, 4>), grid, dim3(WQ_WAVES * kWave), 0, stream, a);
        else
            hipLaunchKernelGGL((w4a16_mfma_kernel<1, 1>), grid, dim3(WQ_WAVES * kWave), 0, stream, a);
    }
    (void)kWqVariants;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || w.split <= 1) return e;
    const int64_t total = (int64_t)w.M * w.N;
    hipLaunchKernelGGL(w4a16_reduce_kernel, dim3(grid_for(total, 256)), dim3(256), 0, stream,
                       static_cast<const float*>(w.workspace), w.split, w.Y, w.ldy, w.M, w.N);
    return hipGetLastError();
}

}  // namespace wmma_amd
