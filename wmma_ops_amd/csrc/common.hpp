// Device-side building blocks shared by every gfx950 kernel in this library.
//
// Everything here is CDNA4-specific: 64-lane wavefronts, MFMA matrix instructions,
// buffer-resource loads whose hardware range check supplies zero-fill for masked lanes,
// and the workgroup-to-XCD placement of a 256-CU, 8-XCD part.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace wmma_amd {

typedef _Float16 f16;
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;
constexpr int kNumXcd = 8;

// Offset that lies outside every buffer resource built below: a masked lane loads 0.
constexpr uint32_t kOobOffset = 0x80000000u;
// num_records for resources whose validity is expressed per lane through kOobOffset.
constexpr int32_t kRecordsAll = 0x7fffffff;
// Third descriptor word for gfx9-family raw buffers (byte-addressed, no stride).
constexpr int32_t kRsrcFlags = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base,
                                                            int32_t records = kRecordsAll) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, records,
                                             kRsrcFlags);
}

// 16-byte load through a buffer resource; offset kOobOffset yields zeros.
__device__ __forceinline__ u32x4 buf_load16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 0);
}
// The same with the nontemporal hint (streamed data read once).
__device__ __forceinline__ u32x4 buf_load16_nt(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b128(r, byte_off, 0, 2);
}
__device__ __forceinline__ u32x2 buf_load8(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b64(r, byte_off, 0, 0);
}
__device__ __forceinline__ uint32_t buf_load4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b32(r, byte_off, 0, 0);
}
__device__ __forceinline__ uint16_t buf_load2(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b16(r, byte_off, 0, 0);
}
__device__ __forceinline__ uint8_t buf_load1(__amdgpu_buffer_rsrc_t r, uint32_t byte_off) {
    return __builtin_amdgcn_raw_buffer_load_b8(r, byte_off, 0, 0);
}

// v_mfma_f32_32x32x16_f16: D(32x32 fp32) += A(32x16) * B(16x32).
// Lane l supplies row l%32 of A and column l%32 of B, eight K values each (the K half is
// selected by l/32; A and B use the same K assignment, so any consistent permutation of
// K within a lane is harmless).  D: lane l holds column l%32, element r holds row
// 8*(r/4) + 4*(l/32) + r%4.
__device__ __forceinline__ f32x16 mfma32(f16x8 a, f16x8 b, f32x16 c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(a, b, c, 0, 0, 0);
}
// v_mfma_f32_16x16x32_f16: D(16x16) += A(16x32) * B(32x16).  Lane l supplies row l%16
// of A / column l%16 of B with eight K values (K quarter l/16).  D: lane l holds column
// l%16, element r holds row 4*(l/16) + r.
__device__ __forceinline__ f32x4 mfma16(f16x8 a, f16x8 b, f32x4 c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
}

// ---- LDS access (address space 3) -------------------------------------------------------
#define WMMA_LDS __attribute__((address_space(3)))
typedef short s16x4 __attribute__((ext_vector_type(4)));

// Direct global -> LDS copy of 16 bytes per lane (buffer_load_dwordx4 ... lds).  The LDS
// destination is `dst` (wave-uniform) + 16 * lane; lanes whose offset lies outside the
// resource write zeros.  The copy is tracked by vmcnt, not by any VGPR.
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                          WMMA_LDS void* dst) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 16, byte_off, 0, 0, 0);
}

// ds_read_b64_tr_b16.  Inside each group of 16 lanes, the 8-byte rows the lanes address
// form a 16x4 matrix R (row = source lane); lane i = 4a + b of the group receives
// R[4j + a][b] for j = 0..3.  So when source lane 4j + a points at row k0 + j, columns
// c0 + 4a .. c0 + 4a + 3 of a row-major 16-bit tile, lane i receives the column c0 + i,
// rows k0 .. k0 + 3: a K-contiguous MFMA operand read out of N-contiguous storage.
__device__ __forceinline__ f16x4 lds_read_tr16(const WMMA_LDS void* p) {
    return __builtin_bit_cast(
        f16x4, __builtin_amdgcn_ds_read_tr16_b64_v4i16((WMMA_LDS s16x4*)p));
}

// s_waitcnt on vmcnt only (expcnt and lgkmcnt left at their maxima).  gfx9 encoding:
// vmcnt[3:0] in bits 3:0 and vmcnt[5:4] in bits 15:14.
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__device__ __forceinline__ f16x8 as_f16x8(u32x4 v) { return __builtin_bit_cast(f16x8, v); }
__device__ __forceinline__ u32x4 as_u32x4(f16x8 v) { return __builtin_bit_cast(u32x4, v); }

// v_perm_b32 selectors: pack the low (resp. high) 16-bit halves of two words, first
// argument's half in the high half of the result.
constexpr uint32_t kPermLo = 0x05040100u;
constexpr uint32_t kPermHi = 0x07060302u;

// Transpose an 8x8 block of 16-bit values held as 8 rows of 16 bytes: out[c] holds
// column c (eight values, row 0 lowest).  32 v_perm_b32.
__device__ __forceinline__ void transpose8x8(const u32x4 in[8], u32x4 out[8]) {
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const uint32_t sel = (c & 1) ? kPermHi : kPermLo;
        const int w = c >> 1;
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            out[c][d] = __builtin_amdgcn_perm(in[2 * d + 1][w], in[2 * d][w], sel);
        }
    }
}

// LDS chunk swizzle for 128-byte rows of eight 16-byte chunks.  Eight consecutive rows
// read at one chunk position land on eight distinct chunks (conflict-free 16-byte
// reads), and rows 8 apart also differ, so the transposing B store (rows 8*i + j) is
// conflict-free as well.
__device__ __forceinline__ int swz8(int row) { return (row ^ (row >> 3)) & 7; }

// Workgroups are dispatched to the 8 XCDs round-robin (id % 8).  Re-map the linear id
// so that each XCD receives a contiguous run of tile ids: the tiles sharing one XCD's
// 4 MB L2 are then neighbours in the grouped order below.
__device__ __forceinline__ int xcd_remap(int pid, int total) {
    if (total % kNumXcd != 0) return pid;
    const int per = total / kNumXcd;
    return (pid % kNumXcd) * per + pid / kNumXcd;
}

// Grouped tile order: walk `group` tile rows at a time, column-major inside the group,
// so consecutive ids share A rows and B columns.
__device__ __forceinline__ void grouped_tile(int pid, int tiles_m, int tiles_n, int group,
                                             int* tm, int* tn) {
    const int per_group = group * tiles_n;
    const int g = pid / per_group;
    const int first_m = g * group;
    const int gsize = min(tiles_m - first_m, group);
    const int in = pid - g * per_group;
    *tm = first_m + in % gsize;
    *tn = in / gsize;
}

// Shuffled epilogue of a BM x BN fp32 tile held in 32x32 MFMA accumulators: wave (wm, wn)
// owns the TM x TN sub-tile at (wm*TM, wn*TN) as FM x FN blocks, lane l holding column l%32
// and element r row 8*(r/4) + 4*(l/32) + r%4 of each block.  Written to global memory
// directly, every store instruction writes two rows of 128 bytes; staged row-major in LDS
// first (CH rows at a time, CH*BN*4 bytes of `lds`), every wave then writes whole 16-byte
// vectors of contiguous row runs -- measured on MI355X, 3.8 -> 1.3 us for the 64 KB output
// of a 128 x 128 tile.  emit(r, c, v) stores the four values of tile row r, columns c..c+3.
// Every thread of the workgroup must call it (it synchronises); the caller's LDS use must be
// complete except for the barrier this function starts with.
template <int BM, int BN, int WM, int WN, int CH, class Emit>
__device__ __forceinline__ void shuffle_epilogue(float* lds,
                                                 const f32x16 (&acc)[BM / WM / 32][BN / WN / 32],
                                                 int wm, int wn, int lane, Emit&& emit) {
    constexpr int TM = BM / WM, TN = BN / WN, FM = TM / 32, FN = TN / 32;
    constexpr int NT = WM * WN * kWave, V = BN / 4;
    static_assert(CH % 32 == 0 && BM % CH == 0, "chunks of whole 32-row blocks");
    const int h = lane >> 5;
#pragma unroll
    for (int c = 0; c < BM / CH; ++c) {
        __syncthreads();  // earlier readers of the LDS are done
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const int rb = wm * TM + 32 * i - c * CH;  // block's first row in the chunk (uniform)
            if (rb >= 0 && rb < CH) {
#pragma unroll
                for (int j = 0; j < FN; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        lds[(rb + 8 * (r >> 2) + 4 * h + (r & 3)) * BN + wn * TN + 32 * j + (lane & 31)] =
                            acc[i][j][r];
            }
        }
        __syncthreads();
        for (int e = (int)threadIdx.x; e < CH * V; e += NT) {
            const int lr = e / V, lv = e - lr * V;
            emit(c * CH + lr, 4 * lv, *reinterpret_cast<const float4*>(lds + lr * BN + 4 * lv));
        }
    }
}

// Sum of split-K partials p[s * stride + 0 .. W-1] over s = 0, 1, ..., split-1, added in
// that order (the fixed order every split-K path shares, so results do not depend on
// scheduling).  The loads of eight splits are issued before any is waited on: a split-K
// reduction is one memory round trip per eight splits, not one per split.
template <int W>
struct FVec;
template <>
struct FVec<1> {
    using T = float;
};
template <>
struct FVec<4> {
    using T = f32x4;
};
template <int W>
__device__ __forceinline__ void splitk_sum(const float* p, int64_t stride, int split,
                                           float (&v)[W]) {
    using T = typename FVec<W>::T;
    constexpr int B = 8;
    T acc{};
    for (int s0 = 0; s0 < split; s0 += B) {
        T t[B];
#pragma unroll
        for (int u = 0; u < B; ++u)  // clamped index: every load unconditional
            t[u] = *reinterpret_cast<const T*>(p + (int64_t)min(s0 + u, split - 1) * stride);
#pragma unroll
        for (int u = 0; u < B; ++u)
            if (s0 + u < split) acc += t[u];
    }
    if constexpr (W == 1) {
        v[0] = acc;
    } else {
#pragma unroll
        for (int e = 0; e < W; ++e) v[e] = acc[e];
    }
}

}  // namespace wmma_amd
