// Calibration kernels: what the hardware itself sustains, for the roofline figures that the
// benchmarks quote.  Not part of the wmma_ops path (no reference counterpart); built into a
// library of their own (libwmma_calib.so, declared in include/wmma_calib.h).
//
//  * mfma_ceiling_kernel -- every wave issues v_mfma_f32_32x32x16_f16 back to back on eight
//    independent accumulators from fp16 operands held in registers: no memory traffic, no
//    LDS, no dependent chains.  Its rate is the matrix pipe's sustained throughput on this
//    board (clock and power limits included), the ceiling a GEMM main loop can approach;
//    with random operands the operand bits switch as in a GEMM on random data.
//  * read_stream_kernel -- streams a buffer once with 16-byte nontemporal loads (each
//    workgroup a contiguous run of THREADS x LOADS 16-byte units, every lane LOADS loads in
//    flight) and folds the words into one value per wave, the floor of an HBM-bound kernel
//    that reads the same bytes with the same launch shape.
//  * lds_read_kernel -- eight waves per workgroup read a 64 KB LDS buffer over and over, in
//    one of three patterns: ds_read_b128 (1 KB contiguous per instruction, the K rows of
//    the flash kernels and the A rows of the GEMM), ds_read_b64_tr_b16 on 512 contiguous
//    bytes, and ds_read_b64_tr_b16 in the flash forward's V-fragment pattern at D = 128
//    (eight 256-byte rows, 64 bytes each, chunk swizzle 4 * (row % 4)).  The LDS read rate
//    the MFMA kernels' fragment reads share with their matrix instructions.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/wmma_calib.h"
#include "common.hpp"

using namespace wmma_amd;

namespace {

template <int ACC>
__global__ void __launch_bounds__(256) mfma_ceiling_kernel(int iters, const u32x4* operands,
                                                           float* sink) {
    f32x16 acc[ACC];
#pragma unroll
    for (int i = 0; i < ACC; ++i) acc[i] = f32x16{};
    // ACC A fragments and ACC B fragments per lane.  From `operands` (random data, so the
    // operand bits toggle from one MFMA to the next as in a GEMM on random inputs), or, with
    // operands == NULL, constants from the thread index.  The switching activity of the
    // operands moves the power draw, and with it the clock, so the two differ.
    f16x8 a[ACC], b[ACC];
#pragma unroll
    for (int i = 0; i < ACC; ++i) {
        if (operands) {
            const int64_t base = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) * 2 * ACC;
            a[i] = as_f16x8(operands[base + i]);
            b[i] = as_f16x8(operands[base + ACC + i]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                a[i][e] = (f16)(float)((threadIdx.x + i) & 7);
                b[i][e] = (f16)(float)e;
            }
        }
    }
    for (int it = 0; it < iters; it += 2) {
        // every MFMA of the pair of rounds takes a different (A, B) pair
#pragma unroll
        for (int i = 0; i < ACC; ++i) acc[i] = mfma32(a[i], b[(i + 1) % ACC], acc[i]);
#pragma unroll
        for (int i = 0; i < ACC; ++i) acc[i] = mfma32(a[(i + 3) % ACC], b[i], acc[i]);
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < ACC; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) s += acc[i][r];
    if (s == 1234.5f) sink[blockIdx.x] = s;  // never true; keeps the work alive
}

template <int THREADS, int LOADS>
__global__ void __launch_bounds__(THREADS) read_stream_kernel(const u32x4* src, int64_t units,
                                                              float* sink) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int64_t per_wg = (int64_t)THREADS * LOADS;  // 16-byte units per workgroup
    const int64_t base = (int64_t)blockIdx.x * per_wg;
    u32x4 w[LOADS];
#pragma unroll
    for (int u = 0; u < LOADS; ++u) {
        const int64_t i = base + (int64_t)(wave * LOADS + u) * 64 + lane;
        w[u] = __builtin_nontemporal_load(src + (i < units ? i : units - 1));
    }
    uint32_t x = 0;
#pragma unroll
    for (int u = 0; u < LOADS; ++u) x ^= w[u][0] ^ w[u][1] ^ w[u][2] ^ w[u][3];
    // every lane's words feed the result (a per-wave reduction), so no load is dead
    x ^= __shfl_xor(x, 1);
    x ^= __shfl_xor(x, 2);
    x ^= __shfl_xor(x, 4);
    x ^= __shfl_xor(x, 8);
    x ^= __shfl_xor(x, 16);
    x ^= __shfl_xor(x, 32);
    if (x == 0x9E3779B9u && lane == 0) sink[blockIdx.x] = (float)wave;
}

// Every wave reads 8 KB per iteration (eight ds_read_b128, or eight pairs of
// ds_read_b64_tr_b16); addresses are fixed per lane, offsets per iteration wave-uniform.
template <int MODE>
__global__ void __launch_bounds__(512) lds_read_kernel(int iters, float* sink) {
    __shared__ __attribute__((aligned(1024))) unsigned char smem[65536];
    for (int i = threadIdx.x; i < 65536 / 4; i += 512)
        reinterpret_cast<uint32_t*>(smem)[i] = (uint32_t)i * 2654435761u;
    __syncthreads();
    const WMMA_LDS unsigned char* lds = (const WMMA_LDS unsigned char*)smem;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    int vbase[4];
    {
        // flash forward V fragments (D = 128): lane 4j + a of 16-lane group g reads row
        // 4 (g / 2) + j, columns 32 db + 16 (g % 2) + 4 a .. +3 of a 256-byte-row tile
        const int g = lane >> 4, jj = (lane & 15) >> 2, aa = lane & 3;
        const int row = 4 * (g >> 1) + jj, sw = 4 * (row & 3);
#pragma unroll
        for (int db = 0; db < 4; ++db) {
            const int col = 32 * db + 16 * (g & 1) + 4 * aa;
            vbase[db] = row * 256 + (((col >> 3) ^ sw) << 4) + ((col & 7) << 1);
        }
    }
    uint32_t x = 0;
    for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int blk = (it * 64 + u * 8 + wave) & 63;  // wave-uniform 1 KB block
            if constexpr (MODE == 0) {
                const u32x4 v = *(const volatile WMMA_LDS u32x4*)(lds + blk * 1024 + lane * 16);
                x ^= v[0] ^ v[1] ^ v[2] ^ v[3];
            } else {
                const int a0 = MODE == 1 ? blk * 1024 + lane * 8
                                         : vbase[u & 3] + 16 * ((it + (u >> 2) + wave) & 3) * 256;
                const u32x2 lo = __builtin_bit_cast(u32x2, lds_read_tr16(lds + a0));
                const u32x2 hi = __builtin_bit_cast(u32x2, lds_read_tr16(lds + a0 + (MODE == 1 ? 512 : 2048)));
                x ^= lo[0] ^ lo[1] ^ hi[0] ^ hi[1];
            }
        }
    }
    if (x == 0x9E3779B9u) sink[blockIdx.x] = 1.0f;  // keeps the reads observable
}

// The activation stage of the small-M LDS-DMA GEMMs: every iteration a workgroup copies a
// 64-row x 128-byte block (rows `row_bytes` apart, block column it % (row_bytes / 128);
// workgroups alternate between two 64-row blocks like two M tiles) from an L2-resident
// buffer into LDS by buffer_load ... lds, NW waves of 8 / NW 1 KB loads each, with
// DEPTH - 1 stages in flight (DEPTH = 1: each stage waited for before the next is
// issued).  strided = 0 reads the same bytes as contiguous 8 KB blocks instead.
template <int NW, int DEPTH>
__global__ void __launch_bounds__(NW * 64) l2_stage_kernel(const u32x4* src, uint32_t bytes,
                                                           uint32_t row_bytes, int iters,
                                                           int strided, float* sink) {
    constexpr int U = 8 / NW;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[DEPTH * 8192];
    const __amdgpu_buffer_rsrc_t r = make_rsrc(src);
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t cols = row_bytes / 128u;
    const uint32_t base = (blockIdx.x & 1u) * 64u * row_bytes;
    for (int it = 0; it < iters; ++it) {
        const uint32_t kc = (uint32_t)it % cols;
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t row = (uint32_t)((wave * U + u) * 8 + (lane >> 3));
            const uint32_t off = strided ? base + row * row_bytes + kc * 128u + (uint32_t)(lane & 7) * 16u
                                         : base + (kc * 64u + row) * 128u + (uint32_t)(lane & 7) * 16u;
            lds_dma16(r, off % bytes,
                      (WMMA_LDS unsigned char*)smem + (it % DEPTH) * 8192 + (wave * U + u) * 1024);
        }
        wait_vmcnt<(DEPTH - 1) * U>();
        __builtin_amdgcn_s_barrier();
    }
    wait_vmcnt<0>();
    __syncthreads();
    if (smem[threadIdx.x] == 0xAB && smem[threadIdx.x + 1] == 0xCD) sink[blockIdx.x] = 1.0f;
}

}  // namespace

extern "C" {

int wmma_calib_l2_stage(int waves, int depth, int strided, const void* src, size_t bytes,
                        size_t row_bytes, int workgroups, int iters, float* sink, void* stream) {
    if (!src || !sink || workgroups <= 0 || iters <= 0 || row_bytes < 128 || row_bytes % 128 != 0 ||
        bytes < 128 * row_bytes || bytes > 0x7FFFFFFFu || (reinterpret_cast<uintptr_t>(src) & 15u) != 0)
        return 1;
    hipStream_t st = static_cast<hipStream_t>(stream);
    const auto s = static_cast<const u32x4*>(src);
    const uint32_t b = (uint32_t)bytes, rb = (uint32_t)row_bytes;
#define WMMA_CALIB_L2(W, D)                                                                     \
    if (waves == (W) && depth == (D)) {                                                         \
        hipLaunchKernelGGL((l2_stage_kernel<W, D>), dim3(workgroups), dim3((W) * 64), 0, st, s,   \
                           b, rb, iters, strided, sink);                                         \
        return hipGetLastError() == hipSuccess ? 0 : 5;                                         \
    }
    WMMA_CALIB_L2(4, 1) WMMA_CALIB_L2(4, 4) WMMA_CALIB_L2(4, 8) WMMA_CALIB_L2(8, 1) WMMA_CALIB_L2(8, 4)
    WMMA_CALIB_L2(8, 8)
#undef WMMA_CALIB_L2
    return 2;
}

double wmma_calib_l2_stage_bytes(int workgroups, int iters) {
    return (double)workgroups * (double)iters * 8192.0;
}

int wmma_calib_mfma_ceiling(int workgroups, int iters, const void* operands, float* sink,
                            void* stream) {
    if (workgroups <= 0 || iters <= 0 || iters % 2 != 0 || !sink) return 1;
    if ((reinterpret_cast<uintptr_t>(operands) & 15u) != 0) return 1;
    hipLaunchKernelGGL((mfma_ceiling_kernel<8>), dim3(workgroups), dim3(256), 0,
                       static_cast<hipStream_t>(stream), iters,
                       static_cast<const u32x4*>(operands), sink);
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

double wmma_calib_mfma_ceiling_flops(int workgroups, int iters) {
    // 4 waves x 8 accumulators x iters MFMAs of 32 x 32 x 16 (2 FLOP per multiply-add)
    return (double)workgroups * 4 * 8 * iters * (2.0 * 32 * 32 * 16);
}

int wmma_calib_read_stream_shape(const void* src, size_t bytes, int threads, int loads_per_lane,
                                 float* sink, void* stream) {
    if (!src || !sink || bytes < 16 || (reinterpret_cast<uintptr_t>(src) & 15u) != 0) return 1;
    const int64_t units = (int64_t)(bytes / 16);
    hipStream_t st = static_cast<hipStream_t>(stream);
    const int64_t per_wg = (int64_t)threads * loads_per_lane;
    const dim3 grid(per_wg > 0 ? (unsigned)((units + per_wg - 1) / per_wg) : 0u);
#define WMMA_CALIB_RS(T, L)                                                                      \
    if (threads == (T) && loads_per_lane == (L)) {                                               \
        hipLaunchKernelGGL((read_stream_kernel<T, L>), grid, dim3(T), 0, st, (const u32x4*)src,   \
                           units, sink);                                                          \
        return hipGetLastError() == hipSuccess ? 0 : 5;                                          \
    }
    WMMA_CALIB_RS(64, 16) WMMA_CALIB_RS(256, 2) WMMA_CALIB_RS(256, 4) WMMA_CALIB_RS(256, 8)
    WMMA_CALIB_RS(512, 2) WMMA_CALIB_RS(512, 4) WMMA_CALIB_RS(512, 8) WMMA_CALIB_RS(1024, 2)
    WMMA_CALIB_RS(1024, 4)
#undef WMMA_CALIB_RS
    return 2;
}

int wmma_calib_lds_read(int mode, int workgroups, int iters, float* sink, void* stream) {
    if (workgroups <= 0 || iters <= 0 || !sink) return 1;
    hipStream_t st = static_cast<hipStream_t>(stream);
    switch (mode) {
        case 0: hipLaunchKernelGGL(lds_read_kernel<0>, dim3(workgroups), dim3(512), 0, st, iters, sink); break;
        case 1: hipLaunchKernelGGL(lds_read_kernel<1>, dim3(workgroups), dim3(512), 0, st, iters, sink); break;
        case 2: hipLaunchKernelGGL(lds_read_kernel<2>, dim3(workgroups), dim3(512), 0, st, iters, sink); break;
        default: return 2;
    }
    return hipGetLastError() == hipSuccess ? 0 : 5;
}

double wmma_calib_lds_read_bytes(int workgroups, int iters) {
    return (double)workgroups * 8.0 * (double)iters * 8192.0;
}

int wmma_calib_read_stream(const void* src, size_t bytes, int loads_per_wave, float* sink,
                           void* stream) {
    return wmma_calib_read_stream_shape(src, bytes, 512, loads_per_wave, sink, stream);
}

}  // extern "C"
