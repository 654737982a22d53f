// Flash-attention forward for gfx950:  O = softmax(scale * Q K^T [+ causal mask]) V.
//
// The reference documents flash_attention(Q, K, V, causal=False, scale=-1.0) on
// [B, H, N, D] fp16 tensors with default scale 1/sqrt(D) (README.md:221-251); its kernel
// was removed.  This is a new MFMA design for CDNA4:
//
//  * A workgroup owns 256 queries of one (batch, head): 8 waves x 32 queries, two waves
//    per SIMD, so one wave's softmax (VALU) overlaps the other's matrix work (MFMA).
//  * K/V tiles of 64 keys travel global -> LDS by buffer_load ... lds DMA into a 4-deep
//    ring shared by the 8 waves (no VGPR staging); out-of-range keys arrive as zeros.  K
//    rows and V rows are stored as in memory, XOR-swizzled by 16-byte chunk.
//  * Scores are computed transposed, S^T = K Q^T, on v_mfma_f32_32x32x16_f16 with K as the
//    A operand (ds_read_b128) and the wave's Q fragments as the B operand (registers for
//    the whole kernel): every lane owns one query and 16 keys of each 32-key block (the
//    other 16 sit in lane ^ 32), so row max and row sum are lane-local plus one exchange.
//  * The probabilities stay in registers: a lane's score elements are exactly the B operand
//    it must supply for O^T = V^T P^T.  The matching A operand -- V^T, i.e. 8 keys of one
//    d column -- comes straight out of the row-major V tile with the gfx950 transposing
//    read ds_read_b64_tr_b16 (4 keys per read).
//  * One barrier per tile; the DMA of tile j+3 is issued right after it.
//  * FP32 online softmax in base 2 (scale * log2 e folded into one FMA per score) against a
//    stale running max: no per-tile row max; the running max is only moved (and O and the
//    row sum rescaled, the tile recomputed) when some probability could reach 2^15, which
//    the lane's partial sum shows, so P stays below 2^15 in fp16.
//  * Causal (key j <= query i, top-left aligned as torch SDPA's is_causal): key tiles past
//    the workgroup's last query are never loaded, tiles past a wave's own last query are
//    skipped by that wave, masks are applied only on tiles that cross the diagonal or the
//    end of K, and the heaviest query blocks are dispatched first.
//  * Head dims: kernels are built for D = 64, 128 and 256; any multiple of 8 up to 256 runs
//    on the smallest that holds it, the d columns past the tensors' head dim arriving as
//    zeros (no score or output contribution) and never stored.  D = 256 runs 4 waves of
//    the whole register file each and a 2-deep ring (see FaCfg).
#include "common.hpp"
#include "kernels.hpp"
#include "plan.hpp"

namespace wmma_amd {

namespace {

struct FlashArgs {
    const f16* Q;
    const f16* K;
    const f16* V;
    f16* O;
    int Sq, Sk;
    int nqb;           // query blocks
    float scale_log2;  // scale * log2(e)
    int group;         // query heads per key/value head (1: multi-head attention)
    int dr;            // head dim of the tensors: a multiple of 8, at most the kernel's D
                       // (d columns dr .. D-1 load as zeros and are not stored)
    // Variable length (cu_q != nullptr): Q/O packed [total_q][H][D], K/V [total_k][Hkv][D];
    // sequence b spans rows cu_q[b] .. cu_q[b+1] (and cu_k likewise).  Sq/Sk then hold the
    // longest lengths; every row index is clamped into [0, total) so inconsistent offsets
    // cannot send a load or store outside the tensors.
    const int* cu_q;
    const int* cu_k;
    int H, Hkv;
    int total_q, total_k;
    // Optional per-row log-sum-exp of the scaled scores (natural log; +inf for a row with
    // no key): [B*H][Sq] dense, [H][total_q] variable length.
    float* lse;
    // Split key range (dense layout only; kv_chunk = 0: one pass).  Workgroup z of the grid
    // takes keys [z kv_chunk, (z + 1) kv_chunk) and writes, for each of its query rows r =
    // bh Sq + q, the unnormalised O (o_part[z][r][dr]) and its running max (base-2 scaled
    // scores) and row sum (ml_part[z][r][2]); flash_combine_kernel merges the chunks.
    int kv_chunk;
    float* o_part;
    float* ml_part;
};

constexpr int FA_WQ = 32;                   // queries per wave
constexpr int FA_NQB = FA_WQ / 32;          // 32-query MFMA blocks per wave
constexpr int FA_BKV = 64;                  // keys per tile
constexpr float kNegInf = -__builtin_huge_valf();

// Per head dim: D <= 128 runs 8 waves (two per SIMD, so one wave's softmax overlaps the
// other's matrix work) and a 4-deep ring; D = 256 -- whose O accumulators and Q fragments
// alone take 192 registers a lane -- runs 4 waves (one per SIMD, the whole register file)
// and a 2-deep ring of 64 KB stages (the DMA of tile t + 1 overlaps tile t).
template <int D>
struct FaCfg {
    static constexpr int WAVES = D > 128 ? 4 : 8;      // waves per workgroup
    static constexpr int NS = D > 128 ? 2 : 4;         // LDS ring depth
    static constexpr int BQ = WAVES * FA_WQ;           // queries per workgroup
    static constexpr int DCH = D / 8;                  // 16-byte chunks per row
    static constexpr int NDS = D / 16;                 // d-steps of S^T
    static constexpr int NDB = D / 32;                 // 32-wide d blocks of O
    static constexpr int TILE = FA_BKV * D * 2;        // bytes of one K (or V) tile
    static constexpr int STAGE = 2 * TILE;             // K then V
    static constexpr int DMA = TILE / 1024 / WAVES;    // 1 KB DMA instructions per wave per tile
    static constexpr int PER_STAGE = 2 * DMA;          // vmcnt per stage
    static_assert(TILE % (1024 * WAVES) == 0, "DMA split");
    static_assert(NS * STAGE <= 160 * 1024, "LDS ring");
};

// Row swizzles (16-byte chunk index XOR).  K rows are read by ds_read_b128 with 32 lanes
// on 32 consecutive rows at one chunk; V rows by the transposing read, four consecutive
// rows at one chunk pair.
template <int D>
__device__ __forceinline__ int swz_k(int row) {
    return D >= 128 ? (row & 15) : ((row ^ (row >> 3)) & 7);
}
template <int D>
__device__ __forceinline__ int swz_v(int row) {
    return D >= 128 ? 4 * (row & 3) : 2 * (row & 3);
}

template <int D>
struct FaLane {
    uint32_t k_off[FaCfg<D>::DMA], v_off[FaCfg<D>::DMA];  // DMA source offsets in a tile
    int k_row[FaCfg<D>::DMA], v_row[FaCfg<D>::DMA];       // key row of each DMA chunk
    int dma_k, dma_v;                                     // this wave's DMA slice (uniform)
    int k_addr[2];        // K fragment row base (bytes) for key blocks 0, 1
    int k_sw[2];          // K swizzle of this lane's row in key blocks 0, 1
    int v_addr[FaCfg<D>::NDB];  // first transposing-read address per d block
    int h;                // lane / 32
};

// DMA of one K/V tile (kleft = valid keys in it; <= 0 loads zeros).
template <int D>
__device__ __forceinline__ void fa_dma(WMMA_LDS unsigned char* dst, const FaLane<D>& L,
                                       __amdgpu_buffer_rsrc_t rk, __amdgpu_buffer_rsrc_t rv,
                                       int kleft) {
    constexpr int DMA = FaCfg<D>::DMA;
#pragma unroll
    for (int i = 0; i < DMA; ++i)
        lds_dma16(rk, L.k_row[i] < kleft ? L.k_off[i] : kOobOffset, dst + L.dma_k + i * 1024);
#pragma unroll
    for (int i = 0; i < DMA; ++i)
        lds_dma16(rv, L.v_row[i] < kleft ? L.v_off[i] : kOobOffset,
                  dst + FaCfg<D>::TILE + L.dma_v + i * 1024);
}

// S^T = K Q^T for NKB 32-key blocks of one tile, starting at key block kb0, and every
// query block of the wave.
template <int D, int NKB>
__device__ __forceinline__ void fa_scores(const WMMA_LDS unsigned char* s, const FaLane<D>& L,
                                          const f16x8 (&qf)[FA_NQB][FaCfg<D>::NDS], int kb0,
                                          f32x16 (&S)[NKB][FA_NQB]) {
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int qb = 0; qb < FA_NQB; ++qb) S[kb][qb] = f32x16{};
#pragma unroll
    for (int ds = 0; ds < FaCfg<D>::NDS; ++ds) {
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb) {
            const int c = (2 * ds + L.h) ^ L.k_sw[kb0 + kb];
            const f16x8 kf =
                as_f16x8(*(const WMMA_LDS u32x4*)(s + L.k_addr[kb0 + kb] + (c << 4)));
#pragma unroll
            for (int qb = 0; qb < FA_NQB; ++qb) S[kb][qb] = mfma32(kf, qf[qb][ds], S[kb][qb]);
        }
    }
}

// Sets masked scores (keys past Sk or, causal, past the query) to -inf; kv0 is the first
// key of S's first block.
template <int NKB>
__device__ __forceinline__ void fa_mask(f32x16 (&S)[NKB][FA_NQB], int kv0, int qrow0, int Sk,
                                        bool causal, int h) {
#pragma unroll
    for (int qb = 0; qb < FA_NQB; ++qb) {
        const int q = qrow0 + 32 * qb;
#pragma unroll
        for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int key = kv0 + 32 * kb + 8 * (r >> 2) + 4 * h + (r & 3);
                const bool ok = key < Sk && (!causal || key <= q);
                S[kb][qb][r] = ok ? S[kb][qb][r] : kNegInf;
            }
    }
}

// Online softmax of one softmax step (NKB key blocks), every query block (base 2, FP32),
// with a stale running max.
// Returns (through `resc`) whether O must be rescaled by `alpha` before this tile's PV.  The probabilities
// are computed straight against the running max m_run, p = exp2(c*s - m_run), with no
// per-tile max: that max is only needed when some p could leave fp16's range, and every
// such case shows in the lane's partial sum (p <= sum), so a wave-uniform check of
// "sum > 2^15 or no key seen yet" decides.  Only then is the tile's max taken (one
// cross-lane exchange), m_run raised, O and l rescaled by alpha = exp2(m_old - m_new) and
// the tile recomputed -- on the first tile, and after that only when a row's max grows by
// more than 2^15.  Otherwise every p < 2^15 < 65504, so P converts to fp16 safely.  The
// row sum uses four independent partial sums (short dependency chains).
template <int NKB>
__device__ __forceinline__ void fa_exp_tile(const f32x16 (&S)[NKB][FA_NQB], int qb, float c,
                                            float m, f16x8 (&P)[NKB][2][FA_NQB], float& sum) {
    float s4[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float pv = __builtin_amdgcn_exp2f(__builtin_fmaf(S[kb][qb][8 * hh + e], c, -m));
                s4[e & 3] += pv;
                P[kb][hh][qb][e] = (f16)pv;
            }
    sum = (s4[0] + s4[1]) + (s4[2] + s4[3]);
}

template <int NKB>
__device__ __forceinline__ void fa_softmax(f32x16 (&S)[NKB][FA_NQB], float c,
                                           float (&m_run)[FA_NQB], float (&l_run)[FA_NQB],
                                           float (&alpha)[FA_NQB], bool& resc,
                                           f16x8 (&P)[NKB][2][FA_NQB]) {
    constexpr float kSumMax = 32768.0f;  // 2^15
    float sum[FA_NQB];
    bool need = false;
#pragma unroll
    for (int qb = 0; qb < FA_NQB; ++qb) {
        const bool fresh = m_run[qb] == kNegInf;
        fa_exp_tile(S, qb, c, fresh ? 0.0f : m_run[qb], P, sum[qb]);
        need |= fresh || !(sum[qb] <= kSumMax);  // also catches inf / NaN
    }
    resc = __builtin_amdgcn_ballot_w64(need) != 0;
    if (resc) {  // wave-uniform, rare
#pragma unroll
        for (int qb = 0; qb < FA_NQB; ++qb) {
            float mx = kNegInf;
#pragma unroll
            for (int kb = 0; kb < NKB; ++kb)
#pragma unroll
                for (int r = 0; r < 16; ++r) mx = fmaxf(mx, S[kb][qb][r]);
            mx = fmaxf(mx, __shfl_xor(mx, 32));
            const float mn = fmaxf(m_run[qb], mx * c);  // c > 0: max of the scaled scores
            // A running max of -inf (no key seen yet) gives alpha = 0 and keeps exp2's
            // argument finite.
            alpha[qb] = m_run[qb] == kNegInf ? 0.0f : __builtin_amdgcn_exp2f(m_run[qb] - mn);
            m_run[qb] = mn;
            l_run[qb] *= alpha[qb];
            fa_exp_tile(S, qb, c, mn == kNegInf ? 0.0f : mn, P, sum[qb]);
        }
    } else {
#pragma unroll
        for (int qb = 0; qb < FA_NQB; ++qb) alpha[qb] = 1.0f;
    }
#pragma unroll
    for (int qb = 0; qb < FA_NQB; ++qb) l_run[qb] += sum[qb];
}

// O^T += V^T P^T over the 16-key steps of NKB key blocks starting at key block kb0.
template <int D, int NKB>
__device__ __forceinline__ void fa_pv(const WMMA_LDS unsigned char* s, const FaLane<D>& L,
                                      const f16x8 (&P)[NKB][2][FA_NQB], int kb0,
                                      f32x16 (&O)[FaCfg<D>::NDB][FA_NQB]) {
    constexpr int RB = D * 2;  // bytes per V row
#pragma unroll
    for (int ks = 0; ks < 2 * NKB; ++ks) {
#pragma unroll
        for (int db = 0; db < FaCfg<D>::NDB; ++db) {
            const WMMA_LDS unsigned char* pv =
                s + FaCfg<D>::TILE + L.v_addr[db] + 16 * (2 * kb0 + ks) * RB;
            const f16x4 lo = lds_read_tr16(pv);
            const f16x4 hi = lds_read_tr16(pv + 8 * RB);
            const f16x8 vf = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
#pragma unroll
            for (int qb = 0; qb < FA_NQB; ++qb) O[db][qb] = mfma32(vf, P[ks >> 1][ks & 1][qb], O[db][qb]);
        }
    }
}

// One main-loop iteration (tile j): barrier (tile j resident and visible in every wave,
// tile j-1's buffer free), DMA of tile j+3 into that buffer, then S^T, softmax and PV of
// tile j in 2/NKB softmax steps.  The two buffers are distinct and passed as __restrict__
// so the compiler keeps the DMA in flight across the LDS reads; the true DMA -> read
// ordering is the explicit vmcnt wait + barrier.
//
// The causal kernel takes the tile in two 32-key steps (NKB = 1): S and P of one step need
// half the registers, and with the diagonal tiles' extra mask work the shorter
// S -> softmax -> PV chains interleave better between the two waves of a SIMD (measured
// +9% at S = 4096, D = 128); the non-causal kernel is as fast either way and keeps the
// whole tile per step (NKB = 2, half as many rescale checks).
template <int D, bool CAUSAL>
__device__ __forceinline__ void fa_iter(const WMMA_LDS unsigned char* __restrict__ cur,
                                        WMMA_LDS unsigned char* __restrict__ dst,
                                        const FaLane<D>& L, __amdgpu_buffer_rsrc_t rk,
                                        __amdgpu_buffer_rsrc_t rv, int kleft_dma,
                                        const f16x8 (&qf)[FA_NQB][FaCfg<D>::NDS],
                                        f32x16 (&O)[FaCfg<D>::NDB][FA_NQB], float (&m_run)[FA_NQB],
                                        float (&l_run)[FA_NQB], float c, int kv0, int qrow0, int Sk,
                                        bool live, bool masked) {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads are done
    wait_vmcnt<(FaCfg<D>::NS - 2) * FaCfg<D>::PER_STAGE>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    fa_dma<D>(dst, L, rk, rv, kleft_dma);
    if (!live) return;  // causal: every key of this tile is past this wave's queries

    constexpr int NKB = CAUSAL ? 1 : 2;  // 32-key blocks per softmax step
#pragma unroll
    for (int kb0 = 0; kb0 < 2; kb0 += NKB) {
        f32x16 S[NKB][FA_NQB];
        fa_scores<D, NKB>(cur, L, qf, kb0, S);
        if (masked) fa_mask<NKB>(S, kv0 + 32 * kb0, qrow0, Sk, CAUSAL, L.h);
        float alpha[FA_NQB];
        bool resc;
        f16x8 P[NKB][2][FA_NQB];
        fa_softmax<NKB>(S, c, m_run, l_run, alpha, resc, P);
        if (resc) {
#pragma unroll
            for (int db = 0; db < FaCfg<D>::NDB; ++db)
#pragma unroll
                for (int qb = 0; qb < FA_NQB; ++qb) O[db][qb] *= alpha[qb];
        }
        fa_pv<D, NKB>(cur, L, P, kb0, O);
    }
}

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(FaCfg<D>::WAVES * kWave)
__attribute__((amdgpu_waves_per_eu(FaCfg<D>::WAVES / 4, FaCfg<D>::WAVES / 4)))
flash_fwd_kernel(FlashArgs p) {
    using C = FaCfg<D>;
    __shared__ __attribute__((aligned(1024))) unsigned char smem[C::NS * C::STAGE];
    WMMA_LDS unsigned char* lds = (WMMA_LDS unsigned char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int h = lane >> 5, c32 = lane & 31;
    const int bh = blockIdx.x;
    const int qb_idx = CAUSAL ? (p.nqb - 1 - (int)blockIdx.y) : (int)blockIdx.y;
    const int q0 = qb_idx * C::BQ;
    const int qw = q0 + wave * FA_WQ;
    const float c = p.scale_log2;

    // Rows of this (batch, head): base offsets and row strides (elements).  Grouped-query
    // attention: query heads of one batch entry come in runs of `group` that share one
    // key/value head (heads are the inner index of both layouts).
    int Sq, Sk, qs, ks;
    int64_t q_base, k_base, lse_base;
    if (p.cu_q) {
        const int b = bh / p.H, hq = bh % p.H;
        const int qa = min(max(p.cu_q[b], 0), p.total_q);
        const int qe = min(max(p.cu_q[b + 1], qa), p.total_q);
        const int ka = min(max(p.cu_k[b], 0), p.total_k);
        const int ke = min(max(p.cu_k[b + 1], ka), p.total_k);
        Sq = min(qe - qa, p.Sq);
        Sk = min(ke - ka, p.Sk);
        qs = p.H * p.dr;
        ks = p.Hkv * p.dr;
        q_base = (int64_t)qa * qs + (int64_t)hq * p.dr;
        k_base = (int64_t)ka * ks + (int64_t)(hq / p.group) * p.dr;
        lse_base = (int64_t)hq * p.total_q + qa;
    } else {
        Sq = p.Sq;
        Sk = p.Sk;
        qs = p.dr;
        ks = p.dr;
        q_base = (int64_t)bh * Sq * p.dr;
        k_base = (int64_t)(bh / p.group) * Sk * p.dr;
        lse_base = (int64_t)bh * Sq;
    }
    if (q0 >= Sq) return;  // a query block past this sequence (variable length): no work
    const f16* Qb = p.Q + q_base;
    const f16* Kb = p.K + k_base;
    const f16* Vb = p.V + k_base;
    f16* Ob = p.O + q_base;

    // Q fragments (B operand of S^T): query qw + 32 qb + lane%32, d = 16 ds + 8 h + 0..7
    // (zeros for d >= dr, so padded d columns add nothing to the scores).
    f16x8 qf[FA_NQB][C::NDS];
    {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(Qb);
#pragma unroll
        for (int qb = 0; qb < FA_NQB; ++qb) {
            const int q = qw + 32 * qb + c32;
#pragma unroll
            for (int ds = 0; ds < C::NDS; ++ds)
                qf[qb][ds] = as_f16x8(buf_load16(
                    rs, q < Sq && 16 * ds + 8 * h < p.dr
                            ? (uint32_t)(((int64_t)q * qs + 16 * ds + 8 * h) * 2)
                            : kOobOffset));
        }
    }

    FaLane<D> L;
    L.h = h;
    L.dma_k = wave * (C::DMA * 1024);
    L.dma_v = wave * (C::DMA * 1024);
    // LDS chunk pc of a row receives global chunk pc ^ swizzle; chunks at d >= dr load zeros.
#pragma unroll
    for (int i = 0; i < C::DMA; ++i) {
        const int P = 64 * (wave * C::DMA + i) + lane;
        const int row = P / C::DCH, pc = P % C::DCH;
        const int gk = pc ^ swz_k<D>(row), gv = pc ^ swz_v<D>(row);
        L.k_row[i] = row;
        L.k_off[i] = 8 * gk < p.dr ? (uint32_t)((row * ks + 8 * gk) * 2) : kOobOffset;
        L.v_row[i] = row;
        L.v_off[i] = 8 * gv < p.dr ? (uint32_t)((row * ks + 8 * gv) * 2) : kOobOffset;
    }
#pragma unroll
    for (int kb = 0; kb < 2; ++kb) {
        L.k_addr[kb] = (32 * kb + c32) * (D * 2);
        L.k_sw[kb] = swz_k<D>(32 * kb + c32);
    }
    {
        // transposing-read source lane s = 4 jj + aa of 16-lane group g: V row
        // 4 (g / 2) + jj (+8 for the upper half, +16 per key step), columns
        // 32 db + 16 (g % 2) + 4 aa .. +3.
        const int g = lane >> 4, s16 = lane & 15, jj = s16 >> 2, aa = s16 & 3;
        const int row = 4 * (g >> 1) + jj;
        const int sw = swz_v<D>(row);
#pragma unroll
        for (int db = 0; db < C::NDB; ++db) {
            const int col = 32 * db + 16 * (g & 1) + 4 * aa;
            L.v_addr[db] = row * (D * 2) + (((col >> 3) ^ sw) << 4) + ((col & 7) << 1);
        }
    }

    const int kv_end = CAUSAL ? min(Sk, q0 + C::BQ) : Sk;
    const int T = (kv_end + FA_BKV - 1) / FA_BKV;
    // Key tiles [tb, te) of this workgroup: all of them, or one chunk of a split key range.
    int tb = 0, te = T;
    if (p.kv_chunk) {
        const int per = p.kv_chunk / FA_BKV;
        tb = min(T, (int)blockIdx.z * per);
        te = min(T, tb + per);
    }
    // Tiles this wave needs (causal: keys <= its last query); none for a wave whose queries
    // all lie past Sq (it still loads its share of every tile).
    const int Tw = qw >= Sq ? 0 : CAUSAL ? min(T, (qw + FA_WQ - 1) / FA_BKV + 1) : T;
    auto rk_of = [&](int t) { return make_rsrc(Kb + (int64_t)min(t, te - 1) * FA_BKV * ks); };
    auto rv_of = [&](int t) { return make_rsrc(Vb + (int64_t)min(t, te - 1) * FA_BKV * ks); };
    auto kleft = [&](int t) { return t < te ? Sk - t * FA_BKV : 0; };
    // A tile needs masking if it reaches past Sk or (causal) past this wave's first query.
    auto masked = [&](int t) {
        const int kv0 = t * FA_BKV;
        return kv0 + FA_BKV > Sk || (CAUSAL && kv0 + FA_BKV - 1 > qw);
    };

    f32x16 O[C::NDB][FA_NQB];
#pragma unroll
    for (int db = 0; db < C::NDB; ++db)
#pragma unroll
        for (int qb = 0; qb < FA_NQB; ++qb) O[db][qb] = f32x16{};
    float m_run[FA_NQB], l_run[FA_NQB];
#pragma unroll
    for (int qb = 0; qb < FA_NQB; ++qb) {
        m_run[qb] = kNegInf;
        l_run[qb] = 0.0f;
    }
    const int qrow0 = qw + c32;

    if (te > tb) {
        // Prologue: tiles tb .. tb+NS-2 in flight (tiles past te load zeros).
#pragma unroll
        for (int s = 0; s < C::NS - 1; ++s)
            fa_dma<D>(lds + s * C::STAGE, L, rk_of(tb + s), rv_of(tb + s), kleft(tb + s));
        for (int t = tb; t < te; ++t) {
            const int tf = t + C::NS - 1;
            fa_iter<D, CAUSAL>(lds + ((t - tb) % C::NS) * C::STAGE,
                               lds + ((tf - tb) % C::NS) * C::STAGE, L, rk_of(tf), rv_of(tf),
                               kleft(tf), qf, O, m_run, l_run, c, t * FA_BKV, qrow0, Sk, t < Tw,
                               masked(t));
        }
        wait_vmcnt<0>();
    }

    if (p.kv_chunk) {
        // One chunk of a split key range: unnormalised O, running max and row sum of each
        // query row (a chunk with no live key leaves O = 0, max = -inf, sum = 0).
        const int64_t rows = (int64_t)gridDim.x * Sq;
#pragma unroll
        for (int qb = 0; qb < FA_NQB; ++qb) {
            const int q = qrow0 + 32 * qb;
            const float l_tot = l_run[qb] + __shfl_xor(l_run[qb], 32);
            if (q >= Sq) continue;
            const int64_t r = (int64_t)blockIdx.z * rows + (int64_t)bh * Sq + q;
            if (h == 0) {
                p.ml_part[2 * r] = m_run[qb];
                p.ml_part[2 * r + 1] = l_tot;
            }
            float* op = p.o_part + r * p.dr;
#pragma unroll
            for (int db = 0; db < C::NDB; ++db)
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * db + 8 * g + 4 * h;
                    if (d < p.dr)
                        *reinterpret_cast<float4*>(op + d) =
                            make_float4(O[db][qb][4 * g], O[db][qb][4 * g + 1],
                                        O[db][qb][4 * g + 2], O[db][qb][4 * g + 3]);
                }
        }
        return;
    }

    // Normalise and store: lane owns query qw + 32 qb + lane%32, d = 32 db + 8 (r/4) +
    // 4 h + r%4.
#pragma unroll
    for (int qb = 0; qb < FA_NQB; ++qb) {
        const int q = qrow0 + 32 * qb;
        const float l_tot = l_run[qb] + __shfl_xor(l_run[qb], 32);
        const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
        // log-sum-exp: m_run is the running max of the base-2 scaled scores, l_tot the sum
        // of exp2(score - m_run), so ln(sum exp) = (m_run + log2 l_tot) * ln 2.
        if (p.lse && h == 0 && q < Sq)
            p.lse[lse_base + q] = l_tot > 0.0f
                                      ? (m_run[qb] + __builtin_amdgcn_logf(l_tot)) * 0.6931471805599453f
                                      : __builtin_huge_valf();
        if (q < Sq) {
#pragma unroll
            for (int db = 0; db < C::NDB; ++db) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    f16x4 v;
#pragma unroll
                    for (int e = 0; e < 4; ++e) v[e] = (f16)(O[db][qb][4 * g + e] * inv);
                    const int d = 32 * db + 8 * g + 4 * h;
                    if (d < p.dr) *reinterpret_cast<f16x4*>(Ob + (int64_t)q * qs + d) = v;
                }
            }
        }
    }
}

// Merges the chunks of a split key range: O = sum_z w_z O_z / sum_z w_z l_z with chunk
// weights w_z = exp2(m_z - m), m the largest running max (0 for a row with no key), and
// lse = (m + log2 l) ln 2 (+inf for a row with no key).  One thread per 4 d columns of a
// query row.  The chunks are read 8 at a time -- all 8 loads issued before any is used, so
// a batch costs one memory round trip -- and folded in order with an online rescale.
constexpr int FA_ZB = 8;

__global__ void __launch_bounds__(256)
flash_combine_kernel(const float* o_part, const float* ml_part, int split, int64_t rows, int dr,
                     f16* O, float* lse) {
    const int dq = dr / 4;
    const int64_t n = rows * dq;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
         i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / dq;
        const int d = (int)(i - r * dq) * 4;
        float m = kNegInf, l = 0.0f;
        float4 acc = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (int z0 = 0; z0 < split; z0 += FA_ZB) {
            float mz[FA_ZB], lz[FA_ZB];
            float4 oz[FA_ZB];
#pragma unroll
            for (int j = 0; j < FA_ZB; ++j) {
                const int64_t zr = (int64_t)(z0 + j) * rows + r;
                const bool in = z0 + j < split;
                mz[j] = in ? ml_part[2 * zr] : kNegInf;
                lz[j] = in ? ml_part[2 * zr + 1] : 0.0f;
                oz[j] = in ? *reinterpret_cast<const float4*>(o_part + zr * dr + d)
                           : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
#pragma unroll
            for (int j = 0; j < FA_ZB; ++j) {
                if (mz[j] == kNegInf) continue;  // a chunk with no live key
                const float mn = fmaxf(m, mz[j]);
                const float a = __builtin_amdgcn_exp2f(m - mn);  // 0 while m is -inf
                const float w = __builtin_amdgcn_exp2f(mz[j] - mn);
                l = l * a + w * lz[j];
                acc.x = acc.x * a + w * oz[j].x;
                acc.y = acc.y * a + w * oz[j].y;
                acc.z = acc.z * a + w * oz[j].z;
                acc.w = acc.w * a + w * oz[j].w;
                m = mn;
            }
        }
        const float inv = l > 0.0f ? 1.0f / l : 0.0f;
        f16x4 v;
        v[0] = (f16)(acc.x * inv);
        v[1] = (f16)(acc.y * inv);
        v[2] = (f16)(acc.z * inv);
        v[3] = (f16)(acc.w * inv);
        *reinterpret_cast<f16x4*>(O + r * dr + d) = v;
        if (lse && d == 0)
            lse[r] = l > 0.0f ? (m + __builtin_amdgcn_logf(l)) * 0.6931471805599453f
                              : __builtin_huge_valf();
    }
}

template <int D>
void launch_d(FlashArgs a, int BH, bool causal, hipStream_t stream) {
    a.nqb = ceil_div(a.Sq, FaCfg<D>::BQ);
    dim3 grid(BH, a.nqb, a.kv_chunk ? ceil_div(a.Sk, a.kv_chunk) : 1);
    const dim3 block(FaCfg<D>::WAVES * kWave);
    if (causal)
        hipLaunchKernelGGL((flash_fwd_kernel<D, true>), grid, block, 0, stream, a);
    else
        hipLaunchKernelGGL((flash_fwd_kernel<D, false>), grid, block, 0, stream, a);
}

}  // namespace

hipError_t launch_flash_fwd(const FlashLaunch& f, hipStream_t stream) {
    FlashArgs a{};
    a.Q = static_cast<const f16*>(f.Q);
    a.K = static_cast<const f16*>(f.K);
    a.V = static_cast<const f16*>(f.V);
    a.O = static_cast<f16*>(f.O);
    a.Sq = f.Sq;
    a.Sk = f.Sk;
    a.group = f.H / f.Hkv;
    a.dr = f.D;
    a.cu_q = f.cu_q;
    a.cu_k = f.cu_k;
    a.H = f.H;
    a.Hkv = f.Hkv;
    a.total_q = f.total_q;
    a.total_k = f.total_k;
    a.lse = f.lse;
    a.scale_log2 = f.scale * 1.4426950408889634f;
    const int BH = f.B * f.H;
    const int split = f.cu_q ? 1 : f.kv_split;
    if (split > 1) {
        // chunks of whole 64-key tiles; the partial sums sit at the start of the workspace
        a.kv_chunk = ceil_div(ceil_div(f.Sk, split), FA_BKV) * FA_BKV;
        const int64_t rows = (int64_t)BH * f.Sq;
        const int nz = ceil_div(f.Sk, a.kv_chunk);
        a.o_part = static_cast<float*>(f.workspace);
        a.ml_part = a.o_part + (int64_t)nz * rows * f.D;
    }
    // head dims up to 64 run the D = 64 kernel, up to 128 the D = 128 kernel, up to 256 the
    // D = 256 kernel
    if (f.D > 128)
        launch_d<256>(a, BH, f.causal, stream);
    else if (f.D > 64)
        launch_d<128>(a, BH, f.causal, stream);
    else
        launch_d<64>(a, BH, f.causal, stream);
    if (a.kv_chunk == 0) return hipGetLastError();
    if (hipError_t e = hipGetLastError(); e != hipSuccess) return e;
    const int64_t rows = (int64_t)BH * f.Sq;
    const int64_t threads = rows * (f.D / 4);
    const int grid = (int)std::min<int64_t>(ceil_div64(threads, 256), 8192);
    hipLaunchKernelGGL(flash_combine_kernel, dim3(grid), dim3(256), 0, stream, a.o_part, a.ml_part,
                       ceil_div(f.Sk, a.kv_chunk), rows, f.D, a.O, f.lse);
    return hipGetLastError();
}

int flash_kv_split(int B, int H, int Hkv, int Sq, int Sk, int D, int num_cus) {
    if (B <= 0 || H <= 0 || Hkv <= 0 || Sq <= 0 || Sk <= 0 || num_cus <= 0) return 1;
    const int bq = D > 128 ? FaCfg<256>::BQ : FaCfg<128>::BQ;
    const int64_t wgs = (int64_t)B * H * ceil_div(Sq, bq);
    if (wgs * 2 > num_cus) return 1;  // at least half the CUs busy without a split
    // chunks of at least 4 tiles, enough of them to fill the CUs, while the partial sums
    // (written and read back: 8 bytes per query row and d column per chunk) stay within a
    // quarter of the K/V bytes read (4 per key and d column of each K/V head)
    int s = (int)std::min<int64_t>(ceil_div64(num_cus, wgs), ceil_div(Sk, FA_BKV) / 4);
    const int64_t group = H / Hkv;
    while (s > 1 && (int64_t)s * Sq * group * 8 > Sk) --s;
    return std::max(s, 1);
}

size_t flash_fwd_workspace_bytes(int B, int H, int Sq, int Sk, int D, int split) {
    if (split <= 1) return 0;
    const int64_t kv_chunk = ceil_div(ceil_div(Sk, split), FA_BKV) * FA_BKV;
    const int64_t nz = ceil_div64(Sk, kv_chunk);
    return (size_t)(nz * B * H * Sq) * (size_t)(D + 2) * sizeof(float);
}

}  // namespace wmma_amd
