// Flash-attention backward for gfx950: dQ, dK, dV of O = softmax(scale * Q K^T [+ mask]) V
// given dO and the forward's per-row log-sum-exp L (natural log).
//
// With P = exp(scale * S - L) (S = Q K^T), dP = dO V^T and Delta = rowsum(dO o O):
//     dV = P^T dO,    dS = P o (dP - Delta),    dQ = scale * dS K,    dK = scale * dS^T Q.
// Two kernels, both deterministic (every output element is written once, by one wave,
// from FP32 registers; no atomics):
//
//  * dQ kernel (runs first): built like the forward kernel -- a workgroup owns 256 queries
//    of one (batch, head), 8 waves x 32 queries, and streams 64-key K/V tiles through a
//    4-deep LDS ring by buffer_load ... lds DMA.  The wave keeps its Q and dO fragments in
//    registers, recomputes S^T = K Q^T and dP^T = V dO^T on v_mfma_f32_32x32x16_f16 (K and
//    V rows by ds_read_b128), forms dS^T in registers and accumulates dQ^T += K^T dS^T with
//    K^T read by the transposing ds_read_b64_tr_b16.  It also computes Delta from its own
//    dO and O fragments and writes Delta and L / scale (the log-sum-exp in raw-score units)
//    to the workspace for the second kernel.
//  * dK/dV kernel: a workgroup owns the keys of one (batch, key/value head) -- 4 waves, one
//    per SIMD with the whole 512-register file, x 64 keys for D = 64 and x 32 keys for
//    D = 128 -- with the wave's K and V fragments in registers and dK^T, dV^T accumulated in
//    registers.  It streams 64-query tiles of Q, dO and the two row statistics through the
//    LDS ring -- for grouped-query attention, the tiles of every query head of the group in
//    turn, which makes dK and dV the sum over the group without a second pass.  Per 32-query
//    block: S = Q K^T and dP = dO V^T (Q, dO rows by ds_read_b128; the accumulators start at
//    -L/scale and -Delta, so P = exp2(scale*log2e * acc) and dS = P o acc need no further
//    row terms), then dV^T += dO^T P and dK^T += Q^T dS with dO^T, Q^T read by the
//    transposing read.
//  * Tiles read both row-wise and transposed (K in the dQ kernel, Q and dO in the dK/dV
//    kernel) use a 16-byte-chunk swizzle that is conflict-free for both access patterns
//    (checked at compile time below).
//  * Causal (key j <= query i, top-left aligned as in the forward): the dQ kernel stops at
//    the workgroup's last query and waves skip tiles past their own; the dK/dV kernel
//    starts at the tile holding its first key and waves skip tiles before their own keys;
//    only tiles crossing the diagonal are masked.  Heaviest workgroups are dispatched first.
//  * Query rows past the end of a sequence load as zeros (dO = 0, Delta = 0), so they add
//    nothing to dK, dV without a mask; key rows past the end are never stored.
//  * Head dims: as in the forward, any multiple of 8 up to 128 runs on the D = 64 or D = 128
//    kernels with the d columns past the head dim loaded as zeros and never stored.
#include <type_traits>

#include "common.hpp"
#include "kernels.hpp"
#include "plan.hpp"

namespace wmma_amd {

namespace {

constexpr int FB_WAVES_KV = 4;            // dK/dV kernel: one wave per SIMD (see below)
constexpr int FB_ROWS = 32;               // queries per dQ wave
// dQ kernel waves per workgroup and LDS ring depth (both kernels) per head dim: D <= 128
// runs 8 dQ waves (two per SIMD) and a 4-deep ring; D = 256 -- Q, dO fragments and dQ
// accumulators alone take 256 registers a lane -- 4 dQ waves (one per SIMD) and a 2-deep
// ring of 64 KB stages.
template <int D>
struct FbGeom {
    static constexpr int WQ = D > 128 ? 4 : 8;
    static constexpr int NS = D > 128 ? 2 : 4;
    static constexpr int BLOCK_Q = WQ * FB_ROWS;  // queries owned by a dQ workgroup
};
// dK/dV wave: KB 32-key blocks (each LDS read of Q or dO feeds KB matrix instructions).  Two
// for D = 64; for D = 128 the resident K, V, dK and dV of two blocks (384 registers) leave
// too few for the rest and the kernel spills.
// D = 256 splits the dK/dV output columns over DSPLIT = 2 workgroups (blockIdx.z): each
// recomputes S and dP over the whole head dim but accumulates dK, dV for half of it, so
// the resident K, V fragments (128 registers a lane) and the dK, dV accumulators (128)
// fit one wave's register file.
template <int D>
struct FbKv {
    static constexpr int KB = D == 64 ? 2 : 1;
    static constexpr int ROWS = 32 * KB;              // keys per wave
    static constexpr int BLOCK = FB_WAVES_KV * ROWS;  // keys per workgroup
    static constexpr int DSPLIT = D > 128 ? 2 : 1;    // workgroups over the dK/dV columns
    static constexpr int NDB_OUT = D / 32 / DSPLIT;   // 32-wide d blocks of dK, dV per workgroup
};
constexpr int FB_T = 64;                  // rows per streamed tile
constexpr float kNegInfB = -__builtin_huge_valf();
constexpr float kLog2e = 1.4426950408889634f;

template <int D>
struct FbDim {
    static constexpr int RB = D * 2;                    // bytes per row
    static constexpr int DCH = D / 8;                   // 16-byte chunks per row
    static constexpr int NDS = D / 16;                  // 16-wide d steps
    static constexpr int NDB = D / 32;                  // 32-wide d blocks of an accumulator
    static constexpr int TILE = FB_T * RB;              // bytes of one 64-row tile
    static constexpr int STAT = 256;                    // one 64-float row-statistic slot
};

// Per-wave DMA split and ring stage layout of a W-wave workgroup.  dQ kernel stage: K tile,
// V tile.  dK/dV kernel stage: Q tile, dO tile, one statistic slot per wave (slot 0:
// -L / scale, slot 1: -Delta; the others receive zeros).
template <int D, int W>
struct FbCfg : FbDim<D> {
    using B = FbDim<D>;
    static constexpr int DMA = B::TILE / 1024 / W;      // 1 KB DMA instructions per wave per tile
    static constexpr int STAGE_Q = 2 * B::TILE;
    static constexpr int STAGE_KV = 2 * B::TILE + W * B::STAT;
    static constexpr int PER_STAGE_Q = 2 * DMA;
    static constexpr int PER_STAGE_KV = 2 * DMA + 1;
    static_assert(B::TILE % (1024 * W) == 0, "DMA split");
};

// 16-byte-chunk swizzle of a tile row.  Required: (a) 16 consecutive rows (aligned) read at
// one logical chunk by ds_read_b128 hit 16 distinct 16-byte slots of the 256-byte bank
// window, and (b) the 4 x 4 block of rows 4i..4i+3, chunks 4j..4j+3 that half a wave's
// ds_read_b64_tr_b16 touches also hits 16 distinct slots.  The swizzle depends on row % 16
// only, so offsets of 16 rows are plain additions.
template <int D>
__host__ __device__ constexpr int swz2(int row) {
    return D >= 128 ? (((row & 3) << 2) | ((row >> 2) & 3))
                    : ((((row >> 1) & 1) << 2) | ((row >> 2) & 3));
}

template <int D>
constexpr bool swz2_conflict_free() {
    constexpr int CH = D / 8;
    for (int m = 0; m < 4; ++m)
        for (int c = 0; c < CH; ++c) {
            bool seen[16] = {};
            for (int r = 16 * m; r < 16 * m + 16; ++r) {
                if ((c ^ swz2<D>(r)) >= CH) return false;
                const int slot = (r * CH + (c ^ swz2<D>(r))) & 15;
                if (seen[slot]) return false;
                seen[slot] = true;
            }
        }
    for (int i = 0; i < 16; ++i)
        for (int j = 0; j < CH / 4; ++j) {
            bool seen[16] = {};
            for (int r = 4 * i; r < 4 * i + 4; ++r)
                for (int c = 4 * j; c < 4 * j + 4; ++c) {
                    const int slot = (r * CH + (c ^ swz2<D>(r))) & 15;
                    if (seen[slot]) return false;
                    seen[slot] = true;
                }
        }
    for (int r = 0; r < 64; ++r)
        if (swz2<D>(r) != swz2<D>(r & 15)) return false;
    return true;
}
static_assert(swz2_conflict_free<256>() && swz2_conflict_free<128>() && swz2_conflict_free<64>(),
              "swizzle");

struct BwdArgs {
    const f16* Q;
    const f16* K;
    const f16* V;
    const f16* O;
    const f16* dO;
    const float* lse;  // natural log, per query row
    f16* dQ;
    f16* dK;
    f16* dV;
    float* ws;         // [2][rows]: -Delta, then -L / scale
    int64_t rows;      // query rows of lse: B*H*Sq dense, H*total_q variable length
    int Sq, Sk;
    int nqb;           // 256-query blocks (dQ kernel)
    float c;           // scale * log2(e)
    float scale;
    int group;         // query heads per key/value head
    int dr;            // head dim of the tensors: a multiple of 8, at most the kernel's D
                       // (d columns dr .. D-1 load as zeros and are not stored)
    const int* cu_q;   // variable length (nullptr: dense), as in the forward
    const int* cu_k;
    int H, Hkv;
    int total_q, total_k;
    // Grouped-query split of the dK/dV kernel (dense layout; gsplit = 1: none): part gp of
    // blockIdx.z / DSPLIT takes query heads [gp gper, (gp + 1) gper) of the group and
    // writes fp32 partial dK, dV (scaled as the final ones) to kv_part[gp] and
    // kv_part[gsplit + gp], each laid out like K; flash_bwd_kv_sum_kernel adds the parts.
    int gsplit, gper;
    float* kv_part;
    int64_t kv_elems;  // elements of K (B * Hkv * Sk * dr)
};

// Geometry of one (batch entry, query head): lengths, row strides (elements) and bases.
struct SeqGeo {
    int Sq, Sk, qs, ks;
    int64_t q_base, k_base, r_base;  // Q/O/dO element base, K/V element base, lse row base
};

template <int D>
__device__ __forceinline__ SeqGeo seq_geo(const BwdArgs& p, int b, int hq) {
    SeqGeo g;
    if (p.cu_q) {
        const int qa = min(max(p.cu_q[b], 0), p.total_q);
        const int qe = min(max(p.cu_q[b + 1], qa), p.total_q);
        const int ka = min(max(p.cu_k[b], 0), p.total_k);
        const int ke = min(max(p.cu_k[b + 1], ka), p.total_k);
        g.Sq = min(qe - qa, p.Sq);
        g.Sk = min(ke - ka, p.Sk);
        g.qs = p.H * p.dr;
        g.ks = p.Hkv * p.dr;
        g.q_base = (int64_t)qa * g.qs + (int64_t)hq * p.dr;
        g.k_base = (int64_t)ka * g.ks + (int64_t)(hq / p.group) * p.dr;
        g.r_base = (int64_t)hq * p.total_q + qa;
    } else {
        g.Sq = p.Sq;
        g.Sk = p.Sk;
        g.qs = p.dr;
        g.ks = p.dr;
        g.q_base = ((int64_t)b * p.H + hq) * p.Sq * p.dr;
        g.k_base = ((int64_t)b * p.Hkv + hq / p.group) * p.Sk * p.dr;
        g.r_base = ((int64_t)b * p.H + hq) * p.Sq;
    }
    return g;
}

// Per-lane LDS addresses shared by both kernels.
template <int D, int W>
struct FbLane {
    uint32_t dma_off[FbCfg<D, W>::DMA];  // DMA source offset (bytes) inside a tile
    int dma_row[FbCfg<D, W>::DMA];       // tile row of each DMA chunk
    int dma_dst;                      // this wave's DMA slice of a tile (uniform)
    int row_addr;                     // ds_read_b128 row base: row lane%32 of a 32-row block
    int row_sw;                       // its swizzle
    int tr;                           // transposing-read address of d block 0, rows 0..7
    int h;                            // lane / 32
};

// stride: row stride of the streamed tensor (elements); dr: its head dim.  LDS chunk pc of a
// row receives global chunk pc ^ swizzle; chunks at d >= dr load zeros.
template <int D, int W>
__device__ __forceinline__ void fb_lane_init(FbLane<D, W>& L, int wave, int lane, int stride,
                                             int dr) {
    using C = FbCfg<D, W>;
    L.h = lane >> 5;
    L.dma_dst = wave * (C::DMA * 1024);
#pragma unroll
    for (int i = 0; i < C::DMA; ++i) {
        const int P = 64 * (wave * C::DMA + i) + lane;
        const int row = P / C::DCH, pc = P % C::DCH;
        const int gc = pc ^ swz2<D>(row);
        L.dma_row[i] = row;
        L.dma_off[i] = 8 * gc < dr ? (uint32_t)((row * stride + 8 * gc) * 2) : kOobOffset;
    }
    L.row_addr = (lane & 31) * C::RB;
    L.row_sw = swz2<D>(lane & 31);
    // Transposing read: source lane 4 jj + aa of 16-lane group g reads row 4 (g / 2) + jj
    // (+8 for the upper half of a 16-row step), columns 32 db + 16 (g % 2) + 4 aa .. +3.
    // Lane l then receives column 32 db + l % 32, rows 4 (l / 32) + 0..3 (and +8): the
    // K-contiguous MFMA A operand of the transposed tile.  Only d block 0's address is
    // kept: d block db is 4 db chunks further, i.e. chunk bits 2.. XOR db (the swizzle keeps
    // rows aligned to 64-byte groups), and rows +8 flip swizzle bit 1 (fb_tr_addr).
    const int g = lane >> 4, s16 = lane & 15, jj = s16 >> 2, aa = s16 & 3;
    const int r0 = 4 * (g >> 1) + jj;
    const int col = 16 * (g & 1) + 4 * aa;
    L.tr = r0 * C::RB + (((col >> 3) ^ swz2<D>(r0)) << 4) + ((col & 7) << 1);
}

// Byte address (inside a tile, before the 16-row step offset) of the transposing read of d
// block db, rows 0..7 (hi = false) or 8..15 (hi = true) of the step.
template <int D, int W>
__device__ __forceinline__ int fb_tr_addr(const FbLane<D, W>& L, int db, bool hi) {
    return (L.tr ^ (64 * db) ^ (hi ? 32 : 0)) + (hi ? 8 * FbCfg<D, W>::RB : 0);
}
template <int D>
constexpr bool tr_addr_identity() {
    // The XOR forms of fb_tr_addr equal the direct address for every lane and d block.
    constexpr int RB = D * 2;
    for (int lane = 0; lane < 64; ++lane) {
        const int g = lane >> 4, jj = (lane & 15) >> 2, aa = lane & 3;
        const int r0 = 4 * (g >> 1) + jj;
        const int col0 = 16 * (g & 1) + 4 * aa;
        const int t = r0 * RB + (((col0 >> 3) ^ swz2<D>(r0)) << 4) + ((col0 & 7) << 1);
        for (int db = 0; db < D / 32; ++db)
            for (int hi = 0; hi < 2; ++hi) {
                const int r = r0 + 8 * hi, col = 32 * db + col0;
                const int direct = r * RB + (((col >> 3) ^ swz2<D>(r)) << 4) + ((col & 7) << 1);
                const int viaxor = (t ^ (64 * db) ^ (hi ? 32 : 0)) + (hi ? 8 * RB : 0);
                if (direct != viaxor) return false;
            }
    }
    return true;
}
static_assert(tr_addr_identity<256>() && tr_addr_identity<128>() && tr_addr_identity<64>(),
              "transposing-read addresses");

// DMA of one 64-row tile (rows >= left load zeros).
template <int D, int W>
__device__ __forceinline__ void fb_dma_tile(WMMA_LDS unsigned char* dst, const FbLane<D, W>& L,
                                            __amdgpu_buffer_rsrc_t r, int left) {
#pragma unroll
    for (int i = 0; i < FbCfg<D, W>::DMA; ++i)
        lds_dma16(r, L.dma_row[i] < left ? L.dma_off[i] : kOobOffset, dst + L.dma_dst + i * 1024);
}

// Direct global -> LDS copy of 4 bytes per lane (64 floats per wave).
__device__ __forceinline__ void lds_dma4(__amdgpu_buffer_rsrc_t r, uint32_t byte_off,
                                         WMMA_LDS void* dst) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, dst, 4, byte_off, 0, 0, 0);
}

// acc += A B^T over all d steps, where A is 32 rows of an LDS tile (row block `rb`, read
// row-wise) and the register fragments f hold the other operand (lane%32 = its row).
template <int D, int W>
__device__ __forceinline__ f32x16 fb_rows_x_frag(const WMMA_LDS unsigned char* tile,
                                                 const FbLane<D, W>& L, int rb,
                                                 const f16x8 (&f)[FbCfg<D, W>::NDS], f32x16 acc) {
    const WMMA_LDS unsigned char* base = tile + rb * 32 * FbCfg<D, W>::RB + L.row_addr;
#pragma unroll
    for (int ds = 0; ds < FbCfg<D, W>::NDS; ++ds) {
        const int c = (2 * ds + L.h) ^ L.row_sw;
        acc = mfma32(as_f16x8(*(const WMMA_LDS u32x4*)(base + (c << 4))), f[ds], acc);
    }
    return acc;
}

// acc[db] += T^T B over the 16-row step `step` of an LDS tile T (transposing read), for
// every 32-wide d block.
template <int D, int W>
__device__ __forceinline__ void fb_tr_x(const WMMA_LDS unsigned char* tile, const FbLane<D, W>& L,
                                        int step, f16x8 b, f32x16 (&acc)[FbCfg<D, W>::NDB]) {
    const int off = 16 * step * FbCfg<D, W>::RB;
#pragma unroll
    for (int db = 0; db < FbCfg<D, W>::NDB; ++db) {
        const f16x4 lo = lds_read_tr16(tile + fb_tr_addr<D, W>(L, db, false) + off);
        const f16x4 hi = lds_read_tr16(tile + fb_tr_addr<D, W>(L, db, true) + off);
        acc[db] = mfma32(__builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7), b, acc[db]);
    }
}

// Register fragments of one row per lane: row `row` (valid if < n), d = 16 ds + 8 h + 0..7
// (zeros for d >= dr).
template <int D>
__device__ __forceinline__ void fb_load_frag(const f16* base, int stride, int dr, int row, int n,
                                             int h, f16x8 (&f)[FbDim<D>::NDS]) {
    const __amdgpu_buffer_rsrc_t rs = make_rsrc(base);
#pragma unroll
    for (int ds = 0; ds < FbDim<D>::NDS; ++ds)
        f[ds] = as_f16x8(buf_load16(
            rs, row < n && 16 * ds + 8 * h < dr
                    ? (uint32_t)(((int64_t)row * stride + 16 * ds + 8 * h) * 2)
                    : kOobOffset));
}

// Store a transposed accumulator (lane%32 = row, element r = d d0 + 32 db + 8 (r/4) + 4 h +
// r%4) as fp16 rows of the output, scaled by s; columns d >= dr are not stored.
template <int NDB>
__device__ __forceinline__ void fb_store_rows(f16* base, int stride, int dr, int row, int n, int h,
                                              const f32x16 (&acc)[NDB], float s, int d0 = 0) {
    if (row >= n) return;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            f16x4 v;
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] = (f16)(acc[db][4 * g + e] * s);
            const int d = d0 + 32 * db + 8 * g + 4 * h;
            if (d < dr) *reinterpret_cast<f16x4*>(base + (int64_t)row * stride + d) = v;
        }
}

// The same rows as fp32 partial sums (the grouped-query split of the dK/dV kernel).
template <int NDB>
__device__ __forceinline__ void fb_store_rows_f32(float* base, int stride, int dr, int row, int n,
                                                  int h, const f32x16 (&acc)[NDB], float s,
                                                  int d0) {
    if (row >= n) return;
#pragma unroll
    for (int db = 0; db < NDB; ++db)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = d0 + 32 * db + 8 * g + 4 * h;
            if (d < dr)
                *reinterpret_cast<float4*>(base + (int64_t)row * stride + d) =
                    make_float4(acc[db][4 * g] * s, acc[db][4 * g + 1] * s, acc[db][4 * g + 2] * s,
                                acc[db][4 * g + 3] * s);
        }
}

// ---------------------------------------------------------------------------- dQ kernel --
// One tile (64 keys) of the dQ kernel: barrier, DMA of tile t+3, then two 32-key blocks of
// S^T, dP^T, dS^T and dQ^T += K^T dS^T.  masked: the tile reaches past Sk or (causal) past
// this wave's first query.
template <int D, bool CAUSAL>
__device__ __forceinline__ void fb_dq_iter(const WMMA_LDS unsigned char* __restrict__ cur,
                                           WMMA_LDS unsigned char* __restrict__ dst,
                                           const FbLane<D, FbGeom<D>::WQ>& L, __amdgpu_buffer_rsrc_t rk,
                                           __amdgpu_buffer_rsrc_t rv, int kleft_dma,
                                           const f16x8 (&qf)[FbCfg<D, FbGeom<D>::WQ>::NDS],
                                           const f16x8 (&dof)[FbCfg<D, FbGeom<D>::WQ>::NDS],
                                           f32x16 (&dq)[FbCfg<D, FbGeom<D>::WQ>::NDB], float c, float lse2,
                                           float delta, int kv0, int qrow, int Sk, bool live,
                                           bool masked) {
    using C = FbCfg<D, FbGeom<D>::WQ>;
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads are done
    wait_vmcnt<(FbGeom<D>::NS - 2) * C::PER_STAGE_Q>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    fb_dma_tile<D>(dst, L, rk, kleft_dma);
    fb_dma_tile<D>(dst + C::TILE, L, rv, kleft_dma);
    if (!live) return;
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        // S^T, dP^T: lane%32 = query, element r = key 32 kb + 8 (r/4) + 4 h + r%4.
        f32x16 S = fb_rows_x_frag<D>(cur, L, kb, qf, f32x16{});
        const f32x16 dP = fb_rows_x_frag<D>(cur + C::TILE, L, kb, dof, f32x16{});
        // On masked tiles only: S = -inf for keys at row offset 8 (r/4) + r%4 >= lim (past
        // Sk or, causal, past this lane's query).  The empty asm keeps this a real
        // (wave-uniform) branch instead of selects executed on every tile (two waves per
        // SIMD hide the split scheduling region; peeling the masked tiles into a loop of
        // their own, as the dK/dV kernel does, measured no faster here).
        if (masked) {
            asm volatile("" ::: "memory");
            const int lim = (CAUSAL ? min(Sk, qrow + 1) : Sk) - (kv0 + 32 * kb + 4 * L.h);
#pragma unroll
            for (int r = 0; r < 16; ++r) S[r] = 8 * (r >> 2) + (r & 3) < lim ? S[r] : kNegInfB;
        }
        f16x8 dS[2];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(S[r], c, -lse2));
            dS[r >> 3][r & 7] = (f16)(pv * (dP[r] - delta));
        }
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) fb_tr_x<D>(cur, L, 2 * kb + hh, dS[hh], dq);
    }
}

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(FbGeom<D>::WQ * kWave)
__attribute__((amdgpu_waves_per_eu(FbGeom<D>::WQ / 4, FbGeom<D>::WQ / 4)))
flash_bwd_dq_kernel(BwdArgs p) {
    using C = FbCfg<D, FbGeom<D>::WQ>;
    constexpr int NS = FbGeom<D>::NS;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * C::STAGE_Q];
    WMMA_LDS unsigned char* lds = (WMMA_LDS unsigned char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5, c32 = lane & 31;
    const int bh = blockIdx.x;
    const int qb_idx = CAUSAL ? (p.nqb - 1 - (int)blockIdx.y) : (int)blockIdx.y;
    const int q0 = qb_idx * FbGeom<D>::BLOCK_Q;
    const int qw = q0 + wave * FB_ROWS;
    const SeqGeo G = seq_geo<D>(p, bh / p.H, bh % p.H);
    if (q0 >= G.Sq) return;
    const int Sq = G.Sq, Sk = G.Sk;
    const int qrow = qw + c32;

    f16x8 qf[C::NDS], dof[C::NDS];
    fb_load_frag<D>(p.Q + G.q_base, G.qs, p.dr, qrow, Sq, h, qf);
    fb_load_frag<D>(p.dO + G.q_base, G.qs, p.dr, qrow, Sq, h, dof);
    // Delta = rowsum(dO o O): this lane's 64 d values, then the other half of the row.
    float delta;
    {
        f16x8 of[C::NDS];
        fb_load_frag<D>(p.O + G.q_base, G.qs, p.dr, qrow, Sq, h, of);
        float acc[2] = {0.0f, 0.0f};
#pragma unroll
        for (int ds = 0; ds < C::NDS; ++ds)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
                const f16x2 a = {dof[ds][2 * e], dof[ds][2 * e + 1]};
                const f16x2 o = {of[ds][2 * e], of[ds][2 * e + 1]};
                acc[e & 1] = __builtin_amdgcn_fdot2(a, o, acc[e & 1], false);
            }
        delta = acc[0] + acc[1];
        delta += __shfl_xor(delta, 32);
    }
    const float lse = qrow < Sq ? p.lse[G.r_base + qrow] : 0.0f;
    const float c = p.c;
    const float lse2 = lse * kLog2e;
    if (h == 0 && qrow < Sq) {
        p.ws[G.r_base + qrow] = -delta;
        p.ws[p.rows + G.r_base + qrow] = -lse / p.scale;
    }

    FbLane<D, FbGeom<D>::WQ> L;
    fb_lane_init<D>(L, wave, lane, G.ks, p.dr);
    const f16* Kb = p.K + G.k_base;
    const f16* Vb = p.V + G.k_base;
    const int kv_end = CAUSAL ? min(Sk, q0 + FbGeom<D>::BLOCK_Q) : Sk;
    const int T = (kv_end + FB_T - 1) / FB_T;
    const int Tw = CAUSAL ? min(T, (qw + FB_ROWS - 1) / FB_T + 1) : T;
    auto rk_of = [&](int t) { return make_rsrc(Kb + (int64_t)min(t, T - 1) * FB_T * G.ks); };
    auto rv_of = [&](int t) { return make_rsrc(Vb + (int64_t)min(t, T - 1) * FB_T * G.ks); };
    auto kleft = [&](int t) { return t < T ? Sk - t * FB_T : 0; };
    auto masked = [&](int t) {
        const int kv0 = t * FB_T;
        return kv0 + FB_T > Sk || (CAUSAL && kv0 + FB_T - 1 > qw);
    };

    f32x16 dq[C::NDB];
#pragma unroll
    for (int db = 0; db < C::NDB; ++db) dq[db] = f32x16{};

    if (T > 0) {
#pragma unroll
        for (int s = 0; s < NS - 1; ++s) {
            fb_dma_tile<D>(lds + s * C::STAGE_Q, L, rk_of(s), kleft(s));
            fb_dma_tile<D>(lds + s * C::STAGE_Q + C::TILE, L, rv_of(s), kleft(s));
        }
        for (int t = 0; t < T; ++t) {
            const int tf = t + NS - 1;
            fb_dq_iter<D, CAUSAL>(lds + (t % NS) * C::STAGE_Q, lds + (tf % NS) * C::STAGE_Q, L,
                                  rk_of(tf), rv_of(tf), kleft(tf), qf, dof, dq, c, lse2, delta,
                                  t * FB_T, qrow, Sk, t < Tw, masked(t));
        }
        wait_vmcnt<0>();
    }
    fb_store_rows<C::NDB>(p.dQ + G.q_base, G.qs, p.dr, qrow, Sq, h, dq, p.scale);
}

// ------------------------------------------------------------------------- dK/dV kernel --
// acc[kb] += A B_kb^T over all d steps for KB register fragment sets: each row-wise LDS read
// of A (32 rows of block `rb`) feeds KB matrix instructions.
template <int D, int W, int KB>
__device__ __forceinline__ void fb_rows_x_frags(const WMMA_LDS unsigned char* tile,
                                                const FbLane<D, W>& L, int rb,
                                                const f16x8 (&f)[KB][FbDim<D>::NDS],
                                                f32x16 (&acc)[KB]) {
    const WMMA_LDS unsigned char* base = tile + rb * 32 * FbDim<D>::RB + L.row_addr;
#pragma unroll
    for (int ds = 0; ds < FbDim<D>::NDS; ++ds) {
        const int c = (2 * ds + L.h) ^ L.row_sw;
        const f16x8 a = as_f16x8(*(const WMMA_LDS u32x4*)(base + (c << 4)));
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) acc[kb] = mfma32(a, f[kb][ds], acc[kb]);
    }
}

// acc[kb][db] += T^T B_kb over the 16-row step `step` of tile T for the NDBO d blocks from
// db0: each transposing read feeds KB matrix instructions.
template <int D, int W, int KB, int NDBO>
__device__ __forceinline__ void fb_tr_x_multi(const WMMA_LDS unsigned char* tile,
                                              const FbLane<D, W>& L, int step, const f16x8 (&b)[KB],
                                              f32x16 (&acc)[KB][NDBO], int db0) {
    const int off = 16 * step * FbDim<D>::RB;
#pragma unroll
    for (int db = 0; db < NDBO; ++db) {
        const f16x4 lo = lds_read_tr16(tile + fb_tr_addr<D, W>(L, db0 + db, false) + off);
        const f16x4 hi = lds_read_tr16(tile + fb_tr_addr<D, W>(L, db0 + db, true) + off);
        const f16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
        for (int kb = 0; kb < KB; ++kb) acc[kb][db] = mfma32(a, b[kb], acc[kb][db]);
    }
}

// One tile (64 queries of one query head) of the dK/dV kernel; the wave owns KB 32-key
// blocks starting at key `key0` (this lane: key0 + 32 kb + lane%32).  MASK (causal tiles
// that cross the workgroup's diagonal): zero P where key > query.  A compile-time choice: the
// diagonal tiles run in a loop of their own, so the main loop body is one branch-free block
// the scheduler can interleave across its two query blocks.
template <int D, bool MASK>
__device__ __forceinline__ void fb_kv_iter(const WMMA_LDS unsigned char* __restrict__ cur,
                                           WMMA_LDS unsigned char* __restrict__ dst,
                                           const FbLane<D, FB_WAVES_KV>& L, int wave,
                                           __amdgpu_buffer_rsrc_t rq, __amdgpu_buffer_rsrc_t rdo,
                                           __amdgpu_buffer_rsrc_t rst, int qleft_dma,
                                           const f16x8 (&kf)[FbKv<D>::KB][FbDim<D>::NDS],
                                           const f16x8 (&vf)[FbKv<D>::KB][FbDim<D>::NDS],
                                           f32x16 (&dk)[FbKv<D>::KB][FbKv<D>::NDB_OUT],
                                           f32x16 (&dv)[FbKv<D>::KB][FbKv<D>::NDB_OUT], float c, int q0,
                                           int key0, int db0) {
    using C = FbCfg<D, FB_WAVES_KV>;
    __builtin_amdgcn_s_waitcnt(0xC07F);
    wait_vmcnt<(FbGeom<D>::NS - 2) * C::PER_STAGE_KV>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    fb_dma_tile<D>(dst, L, rq, qleft_dma);
    fb_dma_tile<D>(dst + C::TILE, L, rdo, qleft_dma);
    {
        const int lane = threadIdx.x & 63;
        lds_dma4(rst, wave < 2 && lane < qleft_dma ? (uint32_t)(4 * lane) : kOobOffset,
                 dst + 2 * C::TILE + wave * C::STAT);
    }
    // No early exit for tiles wholly before this wave's keys: they take the masked path
    // (all of P is zero).  A skip would give the loop two paths that the register allocator
    // joins by moving the dK/dV accumulators between register files.
    const WMMA_LDS unsigned char* st = cur + 2 * C::TILE;
#pragma unroll
    for (int qb = 0; qb < 2; ++qb) {
        // Accumulators start at -L/scale and -Delta of their query rows 32 qb + 8 g + 4 h + 0..3:
        // S = Q K^T - L/scale, dP = dO V^T - Delta, lane%32 = key, element r = query
        // 32 qb + 8 (r/4) + 4 h + r%4.
        f32x16 S[FbKv<D>::KB];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 l4 = *(const WMMA_LDS f32x4*)(st + 4 * (32 * qb + 8 * g + 4 * L.h));
#pragma unroll
            for (int kb = 0; kb < FbKv<D>::KB; ++kb)
#pragma unroll
                for (int e = 0; e < 4; ++e) S[kb][4 * g + e] = l4[e];
        }
        // Diagonal tiles: S starts at -inf (and stays there) where key > query, i.e. where
        // the row offset 8 (r/4) + r%4 is below `lim` (a no-op for waves whose keys all
        // precede the tile's queries).
        if (MASK) {
#pragma unroll
            for (int kb = 0; kb < FbKv<D>::KB; ++kb) {
                const int lim = key0 + 32 * kb - (q0 + 32 * qb + 4 * L.h);
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    S[kb][r] = 8 * (r >> 2) + (r & 3) >= lim ? S[kb][r] : kNegInfB;
            }
        }
        fb_rows_x_frags<D, FB_WAVES_KV, FbKv<D>::KB>(cur, L, qb, kf, S);
        // P = exp2(c S) (in place)
        f16x8 P[2][FbKv<D>::KB];
#pragma unroll
        for (int kb = 0; kb < FbKv<D>::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const float pv = __builtin_amdgcn_exp2f(S[kb][r] * c);
                S[kb][r] = pv;
                P[r >> 3][kb][r & 7] = (f16)pv;
            }
        f32x16 dP[FbKv<D>::KB];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const f32x4 d4 = *(const WMMA_LDS f32x4*)(st + C::STAT + 4 * (32 * qb + 8 * g + 4 * L.h));
#pragma unroll
            for (int kb = 0; kb < FbKv<D>::KB; ++kb)
#pragma unroll
                for (int e = 0; e < 4; ++e) dP[kb][4 * g + e] = d4[e];
        }
        fb_rows_x_frags<D, FB_WAVES_KV, FbKv<D>::KB>(cur + C::TILE, L, qb, vf, dP);
        f16x8 dS[2][FbKv<D>::KB];
#pragma unroll
        for (int kb = 0; kb < FbKv<D>::KB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) dS[r >> 3][kb][r & 7] = (f16)(S[kb][r] * dP[kb][r]);
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
            fb_tr_x_multi<D, FB_WAVES_KV, FbKv<D>::KB, FbKv<D>::NDB_OUT>(cur + C::TILE, L, 2 * qb + hh,
                                                                         P[hh], dv, db0);
            fb_tr_x_multi<D, FB_WAVES_KV, FbKv<D>::KB, FbKv<D>::NDB_OUT>(cur, L, 2 * qb + hh, dS[hh],
                                                                         dk, db0);
        }
    }
    if constexpr (D == 64) {
        // One wave per SIMD has no other wave to fill its stalls: ask the scheduler to
        // interleave each matrix instruction with LDS reads and VALU work (measured +11% at
        // D = 64; every pattern tried at D = 128 was slower than the default schedule).
#pragma unroll
        for (int i = 0; i < 64 * FbKv<D>::KB; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // 1 MFMA
            __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);  // 3 LDS reads
            __builtin_amdgcn_sched_group_barrier(0x002, 6, 0);  // 6 VALU
        }
    }
}

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(FB_WAVES_KV * kWave)
__attribute__((amdgpu_waves_per_eu(FB_WAVES_KV / 4, FB_WAVES_KV / 4)))
flash_bwd_dkdv_kernel(BwdArgs p) {
    using C = FbCfg<D, FB_WAVES_KV>;
    constexpr int NS = FbGeom<D>::NS;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * C::STAGE_KV];
    WMMA_LDS unsigned char* lds = (WMMA_LDS unsigned char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5, c32 = lane & 31;
    const int bkv = blockIdx.x;
    const int b = bkv / p.Hkv, j = bkv % p.Hkv;
    const int k0 = (int)blockIdx.y * FbKv<D>::BLOCK;  // causal: lower key blocks are heavier, and first
    const int kw = k0 + wave * FbKv<D>::ROWS;
    const SeqGeo G0 = seq_geo<D>(p, b, j * p.group);
    if (k0 >= G0.Sk) return;
    const int Sq = G0.Sq, Sk = G0.Sk;

    f16x8 kf[FbKv<D>::KB][C::NDS], vf[FbKv<D>::KB][C::NDS];
#pragma unroll
    for (int kb = 0; kb < FbKv<D>::KB; ++kb) {
        fb_load_frag<D>(p.K + G0.k_base, G0.ks, p.dr, kw + 32 * kb + c32, Sk, h, kf[kb]);
        fb_load_frag<D>(p.V + G0.k_base, G0.ks, p.dr, kw + 32 * kb + c32, Sk, h, vf[kb]);
    }

    FbLane<D, FB_WAVES_KV> L;
    fb_lane_init<D>(L, wave, lane, G0.qs, p.dr);
    // Query tiles: t0 .. Tq-1 of each of this workgroup's query heads of the group in turn
    // (heads g_lo .. g_lo + ng - 1: the whole group, or one part of a grouped-query split).
    // Head gi's rows start at q_base0 + gi * qh (Q/dO elements) and r_base0 + gi * rh
    // (statistics).
    const int gp = (int)blockIdx.z / FbKv<D>::DSPLIT;
    const int g_lo = gp * p.gper;
    const int ng = max(0, min(p.group, g_lo + p.gper) - g_lo);
    const int Tq = (Sq + FB_T - 1) / FB_T;
    const int t0 = CAUSAL ? min(k0 / FB_T, Tq) : 0;
    const int nT = Tq - t0;
    const int U = ng * nT;
    const int64_t qh = p.cu_q ? (int64_t)p.dr : (int64_t)Sq * p.dr;
    const int64_t rh = p.cu_q ? (int64_t)p.total_q : (int64_t)Sq;
    const float* ws_lse = p.ws + p.rows;
    const float* ws_delta = p.ws;
    // Statistic slot source of this wave: wave 0 -L/scale, wave 1 -Delta, others nothing.
    const float* st_src = wave == 0 ? ws_lse : ws_delta;
    auto tile_of = [&](int u, int& gi, int& t) {
        const int uu = min(u, U - 1);
        const int gr = uu / nT;
        gi = g_lo + gr;
        t = t0 + (uu - gr * nT);
    };
    auto qleft = [&](int u, int t) { return u < U ? Sq - t * FB_T : 0; };

    constexpr int NDBO = FbKv<D>::NDB_OUT;
    // first d block of this workgroup's dK, dV columns
    const int db0 = ((int)blockIdx.z % FbKv<D>::DSPLIT) * NDBO;
    f32x16 dk[FbKv<D>::KB][NDBO], dv[FbKv<D>::KB][NDBO];
#pragma unroll
    for (int kb = 0; kb < FbKv<D>::KB; ++kb)
#pragma unroll
        for (int db = 0; db < NDBO; ++db) {
            dk[kb][db] = f32x16{};
            dv[kb][db] = f32x16{};
        }
    const float c = p.c;

    if (U > 0) {
        auto issue = [&](WMMA_LDS unsigned char* dst, int u) {
            int gi, t;
            tile_of(u, gi, t);
            const int64_t qoff = G0.q_base + gi * qh + (int64_t)t * FB_T * G0.qs;
            const int left = qleft(u, t);
            fb_dma_tile<D>(dst, L, make_rsrc(p.Q + qoff), left);
            fb_dma_tile<D>(dst + C::TILE, L, make_rsrc(p.dO + qoff), left);
            lds_dma4(make_rsrc(st_src + G0.r_base + gi * rh + (int64_t)t * FB_T),
                     wave < 2 && lane < left ? (uint32_t)(4 * lane) : kOobOffset,
                     dst + 2 * C::TILE + wave * C::STAT);
        };
#pragma unroll
        for (int s = 0; s < NS - 1; ++s) issue(lds + s * C::STAGE_KV, s);
        auto step = [&](auto mask_tag, int u) {
            const int uf = u + NS - 1;
            int gi, t, gf, tf;
            tile_of(u, gi, t);
            tile_of(uf, gf, tf);
            const int64_t qoff = G0.q_base + gf * qh + (int64_t)tf * FB_T * G0.qs;
            fb_kv_iter<D, decltype(mask_tag)::value>(
                lds + (u % NS) * C::STAGE_KV, lds + (uf % NS) * C::STAGE_KV, L, wave,
                make_rsrc(p.Q + qoff), make_rsrc(p.dO + qoff),
                make_rsrc(st_src + G0.r_base + gf * rh + (int64_t)tf * FB_T), qleft(uf, tf), kf, vf,
                dk, dv, c, t * FB_T, kw + c32, db0);
        };
        // Causal: the first BLOCK/64 tiles of each query head hold queries below the
        // workgroup's last key (k0 is a multiple of the tile, so exactly these).
        const int nmask = CAUSAL ? min(nT, FbKv<D>::BLOCK / FB_T) : 0;
        for (int gr = 0, u = 0; gr < ng; ++gr) {
            for (const int e = u + nmask; u < e; ++u) step(std::true_type{}, u);
            for (const int e = (gr + 1) * nT; u < e; ++u) step(std::false_type{}, u);
        }
        wait_vmcnt<0>();
    }
    if (p.gsplit > 1) {
        float* pk = p.kv_part + (int64_t)gp * p.kv_elems + G0.k_base;
        float* pv = p.kv_part + (int64_t)(p.gsplit + gp) * p.kv_elems + G0.k_base;
#pragma unroll
        for (int kb = 0; kb < FbKv<D>::KB; ++kb) {
            fb_store_rows_f32<NDBO>(pk, G0.ks, p.dr, kw + 32 * kb + c32, Sk, h, dk[kb], p.scale,
                                    32 * db0);
            fb_store_rows_f32<NDBO>(pv, G0.ks, p.dr, kw + 32 * kb + c32, Sk, h, dv[kb], 1.0f,
                                    32 * db0);
        }
        return;
    }
#pragma unroll
    for (int kb = 0; kb < FbKv<D>::KB; ++kb) {
        fb_store_rows<NDBO>(p.dK + G0.k_base, G0.ks, p.dr, kw + 32 * kb + c32, Sk, h, dk[kb], p.scale,
                            32 * db0);
        fb_store_rows<NDBO>(p.dV + G0.k_base, G0.ks, p.dr, kw + 32 * kb + c32, Sk, h, dv[kb], 1.0f,
                            32 * db0);
    }
}

// dK, dV of a grouped-query split: the gsplit fp32 parts of each element added in part
// order (deterministic) and rounded once to fp16.  Four elements per thread.
__global__ void __launch_bounds__(256)
flash_bwd_kv_sum_kernel(const float* kv_part, int gsplit, int64_t n, f16* dK, f16* dV) {
    const int64_t n4 = n / 4;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < 2 * n4;
         i += (int64_t)gridDim.x * blockDim.x) {
        const bool v = i >= n4;
        const int64_t e = 4 * (v ? i - n4 : i);
        const float* src = kv_part + (v ? (int64_t)gsplit * n : 0) + e;
        float4 a = *reinterpret_cast<const float4*>(src);
        for (int g = 1; g < gsplit; ++g) {
            const float4 b = *reinterpret_cast<const float4*>(src + (int64_t)g * n);
            a.x += b.x;
            a.y += b.y;
            a.z += b.z;
            a.w += b.w;
        }
        f16x4 o;
        o[0] = (f16)a.x;
        o[1] = (f16)a.y;
        o[2] = (f16)a.z;
        o[3] = (f16)a.w;
        *reinterpret_cast<f16x4*>((v ? dV : dK) + e) = o;
    }
}

template <int D>
void launch_bwd_d(BwdArgs a, int B, bool causal, hipStream_t stream) {
    a.nqb = ceil_div(a.Sq, FbGeom<D>::BLOCK_Q);
    const dim3 bq(FbGeom<D>::WQ * kWave), bk(FB_WAVES_KV * kWave);
    const dim3 gq(B * a.H, a.nqb);
    const dim3 gk(B * a.Hkv, ceil_div(a.Sk, FbKv<D>::BLOCK), FbKv<D>::DSPLIT * a.gsplit);
    // The dQ kernel writes the row statistics the dK/dV kernel reads: same stream, in order.
    // An empty side (no query or no key rows) launches nothing for it; with no query rows
    // the dK/dV kernel still runs and stores zeros.
    if (gq.x > 0 && gq.y > 0) {
        if (causal)
            hipLaunchKernelGGL((flash_bwd_dq_kernel<D, true>), gq, bq, 0, stream, a);
        else
            hipLaunchKernelGGL((flash_bwd_dq_kernel<D, false>), gq, bq, 0, stream, a);
    }
    if (gk.x > 0 && gk.y > 0) {
        if (causal)
            hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, true>), gk, bk, 0, stream, a);
        else
            hipLaunchKernelGGL((flash_bwd_dkdv_kernel<D, false>), gk, bk, 0, stream, a);
        if (a.gsplit > 1 && a.kv_elems > 0) {
            const int grid = (int)std::min<int64_t>(ceil_div64(2 * (a.kv_elems / 4), 256), 8192);
            hipLaunchKernelGGL(flash_bwd_kv_sum_kernel, dim3(grid), dim3(256), 0, stream,
                               a.kv_part, a.gsplit, a.kv_elems, a.dK, a.dV);
        }
    }
}

// dK/dV workgroups of a dense shape without a grouped-query split.
template <int D>
int64_t dkdv_workgroups(int B, int Hkv, int Sk) {
    return (int64_t)B * Hkv * ceil_div(Sk, FbKv<D>::BLOCK) * FbKv<D>::DSPLIT;
}

}  // namespace

int64_t flash_bwd_workspace_rows(const FlashBwdLaunch& f) {
    return f.cu_q ? (int64_t)f.H * f.total_q : (int64_t)f.B * f.H * f.Sq;
}

int flash_bwd_group_split(int B, int H, int Hkv, int Sq, int Sk, int D, bool causal,
                          int num_cus) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || H % Hkv != 0 || Sq <= 0 || Sk <= 0 || num_cus <= 0)
        return 1;
    const int group = H / Hkv;
    if (group == 1) return 1;
    const int64_t wgs = D > 128 ? dkdv_workgroups<256>(B, Hkv, Sk)
                                : D > 64 ? dkdv_workgroups<128>(B, Hkv, Sk)
                                         : dkdv_workgroups<64>(B, Hkv, Sk);
    // Parts enough to fill one wave of the CUs when the workgroups fill less than half of
    // it.  With a causal mask, a grid of at most one wave is split in two even when it
    // fills the wave: its first key blocks carry twice the average work and a single wave
    // lasts as long as they do, while two waves dispatched heaviest first even out (measured
    // on MI355X, 32 query / 8 key-value heads, 4096 tokens: 635 -> 508 us; splitting small
    // grids into two waves instead of one cost 3-13%).
    int64_t s = 2 * wgs > num_cus ? 1 : ceil_div64(num_cus, wgs);
    if (causal && s == 1 && wgs <= num_cus) s = 2;
    s = std::min<int64_t>(s, group);
    if (s <= 1) return 1;
    // whole heads per part, no empty part
    const int gper = ceil_div(group, (int)s);
    return ceil_div(group, gper);
}

size_t flash_bwd_split_bytes(int B, int Hkv, int Sk, int D, int gsplit) {
    if (gsplit <= 1) return 0;
    return (size_t)2 * gsplit * (size_t)B * Hkv * Sk * D * sizeof(float);
}

hipError_t launch_flash_bwd(const FlashBwdLaunch& f, hipStream_t stream) {
    BwdArgs a{};
    a.Q = static_cast<const f16*>(f.Q);
    a.K = static_cast<const f16*>(f.K);
    a.V = static_cast<const f16*>(f.V);
    a.O = static_cast<const f16*>(f.O);
    a.dO = static_cast<const f16*>(f.dO);
    a.lse = f.lse;
    a.dQ = static_cast<f16*>(f.dQ);
    a.dK = static_cast<f16*>(f.dK);
    a.dV = static_cast<f16*>(f.dV);
    a.ws = f.ws;
    a.rows = flash_bwd_workspace_rows(f);
    a.Sq = f.Sq;
    a.Sk = f.Sk;
    a.c = f.scale * kLog2e;
    a.scale = f.scale;
    a.group = f.H / f.Hkv;
    a.dr = f.D;
    a.cu_q = f.cu_q;
    a.cu_k = f.cu_k;
    a.H = f.H;
    a.Hkv = f.Hkv;
    a.total_q = f.total_q;
    a.total_k = f.total_k;
    a.gsplit = 1;
    a.gper = a.group;
    if (!f.cu_q && f.gsplit > 1 && f.kv_part) {
        a.gsplit = f.gsplit;
        a.gper = ceil_div(a.group, f.gsplit);
        a.kv_part = f.kv_part;
        a.kv_elems = (int64_t)f.B * f.Hkv * f.Sk * f.D;
    }
    if (f.D > 128)
        launch_bwd_d<256>(a, f.B, f.causal, stream);
    else if (f.D > 64)
        launch_bwd_d<128>(a, f.B, f.causal, stream);
    else
        launch_bwd_d<64>(a, f.B, f.causal, stream);
    return hipGetLastError();
}

}  // namespace wmma_amd
