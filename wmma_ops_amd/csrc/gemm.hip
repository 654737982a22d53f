// FP16 x FP16 -> FP32 GEMM kernels for gfx950 (MI355X).
//
//   C_out = alpha * A[M,K] @ B[K,N] + beta * C_in        (A, B row-major fp16; C fp32)
//
// Kernels:
//  * gemm_mfma_kernel    -- the main path (A, B 16-byte aligned; K, N, lda, ldb multiples
//                           of 8).  MFMA 32x32x16 on K-stages that travel global -> LDS by
//                           buffer_load ... lds DMA (no VGPR staging) into an NS-deep LDS
//                           ring.  A fragments are read with ds_read_b128, B fragments with
//                           the gfx950 transposing read ds_read_b64_tr_b16 straight out of
//                           row-major [K][N] storage.  One barrier per stage, placed before
//                           the stage's last k-step so the next stage's first fragments are
//                           read while the last MFMAs of this one run.  Workgroup ids are
//                           re-mapped per XCD and walked in grouped order so each XCD's L2
//                           sees neighbouring tiles.
//  * gemm_tiled_kernel   -- generic path for unaligned shapes (any M, N, K): element-wise
//                           masked loads, B transposed in registers (8x8 blocks, v_perm) on
//                           its way into a double-buffered LDS stage.
//  * gemm_skinny_kernel  -- M <= 16.  Streams B once from HBM with coalesced 16-byte
//                           loads, computes C^T = B^T A^T with MFMA 16x16x32 so the wide
//                           N dimension fills the matrix rows, reduces its four waves'
//                           K slices in LDS.
//  * splitk_reduce_kernel-- sums split-K partials in a fixed order and applies the
//                           alpha/beta epilogue (reading C_in once).
//
// Reference semantics followed: the epilogue r = alpha*acc; if (beta != 0 && C_in)
// r += beta*C_in (wmma_gemm.hip:636-666); in-place when C_in == C_out
// (wmma_gemm.hip:1988-1991) -- each output element is read and then written by the same
// thread, and no pointer here is declared __restrict__.  Split-K partitions K into
// k_per_split ranges (wmma_xor_swizzle.hpp:293-332) and reduces with a separate kernel
// (wmma_xor_swizzle.hpp:334-353).
#include "common.hpp"
#include "kernels.hpp"
#include "plan.hpp"

namespace wmma_amd {

namespace {

constexpr int BK = kBlockK;  // 64

struct GemmArgs {
    const f16* A;
    const f16* B;
    const float* Cin;
    float* Cout;
    float* ws;  // split-K partials [split][M][N] (dense), used when split > 1
    int64_t lda, ldb, ldcin, ldc;
    int M, N, K;
    float alpha, beta;
    int tiles_m, tiles_n;
    int k_per_split;
    int split;
};

// ------------------------------------------------------------------------------------
// LDS-DMA MFMA kernel (A and B 16-byte aligned, K and N multiples of 8)
//
// One workgroup owns a BMxBN output tile and walks its K range in BK-deep stages held in
// an NS-deep LDS ring.  Every 16-byte chunk of a stage travels global -> LDS by
// buffer_load ... lds: no VGPR staging, no transpose instructions.  Lanes of one DMA
// instruction write 1 KB of LDS contiguously, so the swizzled LDS layout is produced by
// choosing which global chunk each lane fetches.  Out-of-range chunks (M, N and K tails)
// come back as zeros from the buffer range check.
//   A stage: [BM][BK] fp16, rows of KCH 16-byte chunks, chunk c of row r stored at
//            c ^ swz_a(r).  Fragments: ds_read_b128 (row = lane%32, K half = lane/32).
//   B stage: [BK][BN] fp16 (row-major as in memory), chunk c of row k stored at
//            c ^ swz_b(k).  Fragments: two ds_read_b64_tr_b16 per 32x32x16 operand, which
//            deliver column lane%32 with four consecutive K values each.
// Both operands therefore present K-contiguous MFMA fragments with the same K order.
// Wave (wm, wn) owns a TMxTN sub-tile of (TM/32)x(TN/32) 32x32 accumulators.
// ------------------------------------------------------------------------------------
template <int KCH>
__device__ __forceinline__ int swz_a(int r) {
    // Chunk XOR of row r for the fragment reads (ds_read_b128 of 32 consecutive rows at
    // one logical chunk per half-wave).  Both forms measured conflict-free on gfx950
    // (SQ_LDS_BANK_CONFLICT = 0 in a probe of this exact access pattern); for 64-byte rows
    // ((r >> 1) ^ (r >> 3)) & 3 measured 4 conflict cycles per read.
    if constexpr (KCH == 8)
        return (r ^ (r >> 3)) & 7;
    else
        return (r >> 2) & 3;
}

template <int BNC>
__device__ __forceinline__ int swz_b(int k) {
    // The transposing read touches four consecutive rows k..k+3 at one chunk pair; the
    // XOR spreads them over distinct banks.
    if constexpr (BNC >= 16)
        return 4 * (k & 3);
    else
        return 2 * (k & 3);
}

// Per-lane constants of the LDS-DMA kernel.
template <int A_DMA, int B_DMA, int FM, int FN>
struct MfmaLane {
    uint32_t a_off[A_DMA], b_off[B_DMA];  // DMA source offsets (kOobOffset when masked)
    int a_k[A_DMA], b_k[B_DMA];           // K offset of each DMA chunk inside a stage
    int a_addr[FM];                       // byte offset of the lane's A row in a stage
    int a_sw[FM];                         // swizzle of that row
    int b_addr[FN];                       // byte offset of the lane's first tr-read
    int h;                                // lane / 32
    int dma_a, dma_b;                     // this wave's DMA slice of a stage (uniform)
};

// Fragment reads of one 16-deep k-step of a stage (A via ds_read_b128, B via two
// ds_read_b64_tr_b16 per 32x32x16 operand).
template <int BN, int FM, int FN, class Lane>
__device__ __forceinline__ void mfma_read(const WMMA_LDS unsigned char* s, const Lane& L, int ks,
                                          f16x8 (&a)[FM], f16x8 (&b)[FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int c = (2 * ks + L.h) ^ L.a_sw[i];
        a[i] = as_f16x8(*(const WMMA_LDS u32x4*)(s + L.a_addr[i] + (c << 4)));
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const WMMA_LDS unsigned char* pb = s + L.b_addr[j] + ks * 16 * (BN * 2);
        const f16x4 lo = lds_read_tr16(pb);
        const f16x4 hi = lds_read_tr16(pb + 4 * (BN * 2));
        b[j] = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
    }
}

template <int FM, int FN>
__device__ __forceinline__ void mfma_block(const f16x8 (&a)[FM], const f16x8 (&b)[FN],
                                           f32x16 (&acc)[FM][FN]) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma32(a[i], b[j], acc[i][j]);
}

// Scheduling hint for one k-step: MF MFMAs interleaved one-for-one with RD LDS reads,
// optionally preceded by `lead` VMEM (DMA) instructions spread over the first MFMAs.
template <int MF, int RD, int DMA>
__device__ __forceinline__ void mfma_sched() {
    constexpr int X = RD < MF ? RD : MF;
#pragma unroll
    for (int x = 0; x < X; ++x) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
        if (x < DMA) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);
    }
    if constexpr (DMA > X) __builtin_amdgcn_sched_group_barrier(0x020, DMA - X, 0);
    if constexpr (MF > X) __builtin_amdgcn_sched_group_barrier(0x008, MF - X, 0);
    if constexpr (RD > X) __builtin_amdgcn_sched_group_barrier(0x100, RD - X, 0);
}

// One main-loop iteration of the LDS-DMA kernel (stage t):
//   (a) k-steps 0..KS-2 of stage t, each interleaved with the reads of the next k-step;
//   (b) this wave's DMA of stage t+1 complete (vmcnt), LDS reads drained, barrier: from
//       here every wave's copy of stage t+1 is visible, and every wave has finished
//       reading stage t-1;
//   (c) DMA of stage t+NS-1 into the buffer stage t-1 used;
//   (d) the last k-step of stage t, interleaved with the first reads of stage t+1.
// The three buffers are distinct (NS >= 3), so they are passed as __restrict__
// pointers: that lets the compiler keep the DMA in flight across the reads.  Ordering
// between a DMA and later reads of the same buffer is the vmcnt wait + barrier of (b).
template <int BM, int BN, int BK, int WM, int WN, int NS, int A_DMA, int B_DMA, class Lane>
__device__ __forceinline__ void mfma_iter(const WMMA_LDS unsigned char* __restrict__ cur,
                                          const WMMA_LDS unsigned char* __restrict__ nxt,
                                          WMMA_LDS unsigned char* __restrict__ dma_dst,
                                          const Lane& L, __amdgpu_buffer_rsrc_t ra,
                                          __amdgpu_buffer_rsrc_t rb, int kleft,
                                          f16x8 (&af)[2][BM / WM / 32], f16x8 (&bf)[2][BN / WN / 32],
                                          f32x16 (&acc)[BM / WM / 32][BN / WN / 32]) {
    constexpr int FM = BM / WM / 32, FN = BN / WN / 32;
    constexpr int KS = BK / 16;
    constexpr int PER_STAGE = A_DMA + B_DMA;
    constexpr int RD = FM + 2 * FN, MF = FM * FN;
    static_assert(KS % 2 == 0, "fragment double buffer assumes an even k-step count");
    // (a)
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
        mfma_read<BN>(cur, L, ks + 1, af[(ks + 1) & 1], bf[(ks + 1) & 1]);
        mfma_block(af[ks & 1], bf[ks & 1], acc);
        mfma_sched<MF, RD, 0>();
    }
    // (b)
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads are done
    wait_vmcnt<(NS - 3) * PER_STAGE>();
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    // (c)
    const bool full = kleft >= BK;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i)
        lds_dma16(ra, (full || L.a_k[i] < kleft) ? L.a_off[i] : kOobOffset,
                  dma_dst + L.dma_a + i * 1024);
#pragma unroll
    for (int i = 0; i < B_DMA; ++i)
        lds_dma16(rb, (full || L.b_k[i] < kleft) ? L.b_off[i] : kOobOffset,
                  dma_dst + L.dma_b + i * 1024);
    // (d)
    mfma_read<BN>(nxt, L, 0, af[0], bf[0]);
    mfma_block(af[1], bf[1], acc);
    mfma_sched<MF, RD, PER_STAGE>();
}

template <int BM, int BN, int BK, int WM, int WN, int NS>
__global__ void __launch_bounds__(WM * WN * kWave)
__attribute__((amdgpu_waves_per_eu(WM * WN / 4, WM * WN / 4)))
gemm_mfma_kernel(GemmArgs p) {
    constexpr int NW = WM * WN;
    constexpr int TM = BM / WM, TN = BN / WN;
    constexpr int FM = TM / 32, FN = TN / 32;
    constexpr int KCH = BK / 8, BNC = BN / 8;
    constexpr int A_BYTES = BM * BK * 2, B_BYTES = BK * BN * 2;
    constexpr int STAGE = A_BYTES + B_BYTES;
    constexpr int A_DMA = A_BYTES / (1024 * NW);  // 1 KB DMA instructions per wave
    constexpr int B_DMA = B_BYTES / (1024 * NW);
    constexpr int PER_STAGE = A_DMA + B_DMA;      // vmcnt increments per stage
    static_assert(A_BYTES % (1024 * NW) == 0 && B_BYTES % (1024 * NW) == 0, "DMA split");
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");
    static_assert(NS >= 3 && (NS - 2) * PER_STAGE < 64, "vmcnt range");

    __shared__ __attribute__((aligned(1024))) unsigned char smem[NS * STAGE];
    WMMA_LDS unsigned char* lds = (WMMA_LDS unsigned char*)smem;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wm = wave / WN, wn = wave % WN;

    const int tiles = p.tiles_m * p.tiles_n;
    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles), p.tiles_m, p.tiles_n, 4, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = blockIdx.y * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;
    const int M = p.M, N = p.N;
    const int64_t lda = p.lda, ldb = p.ldb;

    MfmaLane<A_DMA, B_DMA, FM, FN> L;
#pragma unroll
    for (int i = 0; i < A_DMA; ++i) {
        const int P = 64 * (wave * A_DMA + i) + lane;
        const int r = P / KCH, c = (P % KCH) ^ swz_a<KCH>(r);
        L.a_off[i] = m0 + r < M ? (uint32_t)((r * lda + 8 * c) * 2) : kOobOffset;
        L.a_k[i] = 8 * c;
    }
#pragma unroll
    for (int i = 0; i < B_DMA; ++i) {
        const int P = 64 * (wave * B_DMA + i) + lane;
        const int k = P / BNC, c = (P % BNC) ^ swz_b<BNC>(k);
        L.b_off[i] = n0 + 8 * c < N ? (uint32_t)((k * ldb + 8 * c) * 2) : kOobOffset;
        L.b_k[i] = k;
    }
    L.h = lane >> 5;
    L.dma_a = wave * (A_DMA * 1024);
    L.dma_b = A_BYTES + wave * (B_DMA * 1024);
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int r = wm * TM + i * 32 + (lane & 31);
        L.a_addr[i] = r * (BK * 2);
        L.a_sw[i] = swz_a<KCH>(r);
    }
    {
        // tr-read source lane s = 4*jj + aa of 16-lane group g: row 8*(g/2) + jj (+4 for
        // the upper half), columns 16*(g%2) + 4*aa .. +3 of the wave's 32-column tile.
        const int g = lane >> 4, s16 = lane & 15, jj = s16 >> 2, aa = s16 & 3;
        const int krow = 8 * (g >> 1) + jj;
        const int sw = swz_b<BNC>(jj);
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int n = wn * TN + j * 32 + 16 * (g & 1) + 4 * aa;
            L.b_addr[j] = A_BYTES + krow * (BN * 2) + (((n >> 3) ^ sw) << 4) + ((n & 7) << 1);
        }
    }

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

    const f16* Ablk = p.A + (int64_t)m0 * lda;
    const f16* Bblk = p.B + n0;
    auto rsrc_a = [&](int kt) { return make_rsrc(Ablk + kbeg + (int64_t)min(kt, nk - 1) * BK); };
    auto rsrc_b = [&](int kt) {
        return make_rsrc(Bblk + (int64_t)(kbeg + (int64_t)min(kt, nk - 1) * BK) * ldb);
    };
    auto kleft = [&](int kt) { return kt < nk ? kend - (kbeg + kt * BK) : 0; };

    if (nk > 0) {
        // Prologue: stages 0 .. NS-2 in flight (stages past the end load zeros), stage 0
        // landed and visible, the first k-step of stage 0 read.
#pragma unroll
        for (int s = 0; s < NS - 1; ++s) {
            WMMA_LDS unsigned char* dst = lds + s * STAGE;
            const int kl = kleft(s);
            const bool full = kl >= BK;
            const __amdgpu_buffer_rsrc_t ra = rsrc_a(s), rb = rsrc_b(s);
#pragma unroll
            for (int i = 0; i < A_DMA; ++i)
                lds_dma16(ra, (full || L.a_k[i] < kl) ? L.a_off[i] : kOobOffset,
                          dst + L.dma_a + i * 1024);
#pragma unroll
            for (int i = 0; i < B_DMA; ++i)
                lds_dma16(rb, (full || L.b_k[i] < kl) ? L.b_off[i] : kOobOffset,
                          dst + L.dma_b + i * 1024);
        }
        wait_vmcnt<(NS - 2) * PER_STAGE>();
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        f16x8 af[2][FM], bf[2][FN];
        mfma_read<BN>(lds, L, 0, af[0], bf[0]);

        for (int t = 0; t < nk; ++t) {
            const int tf = t + NS - 1;  // stage whose DMA is issued in this iteration
            mfma_iter<BM, BN, BK, WM, WN, NS, A_DMA, B_DMA>(
                lds + (t % NS) * STAGE, lds + ((t + 1) % NS) * STAGE, lds + (tf % NS) * STAGE, L,
                rsrc_a(tf), rsrc_b(tf), kleft(tf), af, bf, acc);
        }
        wait_vmcnt<0>();
    }

    // Epilogue.  D layout: lane column lane%32, element r -> row 8*(r/4)+4*(lane/32)+r%4.
    const bool partial = p.split > 1;
    float* out = partial ? p.ws + (size_t)blockIdx.y * (size_t)M * (size_t)N : p.Cout;
    const int64_t ldo = partial ? (int64_t)N : p.ldc;
    const float alpha = partial ? 1.0f : p.alpha;
    const bool use_c = !partial && p.beta != 0.0f && p.Cin != nullptr;
    const int h = lane >> 5;
    const int row0 = m0 + wm * TM + 4 * h, col0 = n0 + wn * TN + (lane & 31);
    const bool full_tile = m0 + BM <= M && n0 + BN <= N;
    // Full tiles whose rows take 16-byte vectors (output, and C_in when it is read) go
    // through the shuffled epilogue when the LDS ring holds the whole fp32 tile: every
    // store then writes whole 16-byte pieces of contiguous row runs.  In place is still
    // exact: each vector of C_in is read by the thread that then writes it.  Not for the
    // 256 x 256 tile (two chunks): there the shuffle cost more than it saved (4096^3:
    // 121-124 -> 126 us; its 64 MB of output is write-bandwidth bound either way).
    constexpr bool kShuffle = NS * STAGE >= BM * BN * 4;
    if constexpr (kShuffle) {
        const bool vec_ok =
            full_tile && ldo % 4 == 0 && (reinterpret_cast<uintptr_t>(out) & 15u) == 0 &&
            (!use_c || (p.ldcin % 4 == 0 && (reinterpret_cast<uintptr_t>(p.Cin) & 15u) == 0));
        if (vec_ok) {
            const float beta = p.beta;
            shuffle_epilogue<BM, BN, WM, WN, BM>(
                reinterpret_cast<float*>(smem), acc, wm, wn, lane, [&](int r, int c, float4 v) {
                    float4 o = make_float4(alpha * v.x, alpha * v.y, alpha * v.z, alpha * v.w);
                    if (use_c) {
                        const float4 ci = *reinterpret_cast<const float4*>(
                            p.Cin + (int64_t)(m0 + r) * p.ldcin + n0 + c);
                        o.x += beta * ci.x;
                        o.y += beta * ci.y;
                        o.z += beta * ci.z;
                        o.w += beta * ci.w;
                    }
                    *reinterpret_cast<float4*>(out + (int64_t)(m0 + r) * ldo + n0 + c) = o;
                });
            return;
        }
    }
    if (full_tile && !use_c) {
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = row0 + i * 32 + 8 * (r >> 2) + (r & 3);
                    out[(int64_t)row * ldo + col0 + j * 32] = alpha * acc[i][j][r];
                }
    } else if (full_tile) {
        // beta * C_in on a full tile: the C_in reads of 32x32 block b+1 are issued before
        // the stores of block b, so the reads stream instead of waiting one block at a time.
        // In place (C_in == C_out) this is still exact: every element is read by the lane
        // that writes it, and the blocks' addresses are disjoint.
        const float beta = p.beta;
        const float* cin = p.Cin + (int64_t)row0 * p.ldcin + col0;
        float* o = out + (int64_t)row0 * ldo + col0;
        constexpr int NB = FM * FN;
        float cv[2][16];
        auto load_c = [&](int b, float* c) {
#pragma unroll
            for (int r = 0; r < 16; ++r)
                c[r] = cin[(int64_t)((b / FN) * 32 + 8 * (r >> 2) + (r & 3)) * p.ldcin + (b % FN) * 32];
        };
        load_c(0, cv[0]);
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (b + 1 < NB) load_c(b + 1, cv[(b + 1) & 1]);
            const int i = b / FN, j = b % FN;
#pragma unroll
            for (int r = 0; r < 16; ++r)
                o[(int64_t)(i * 32 + 8 * (r >> 2) + (r & 3)) * ldo + j * 32] =
                    alpha * acc[i][j][r] + beta * cv[b & 1][r];
        }
    } else {
        const float beta = p.beta;
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int col = col0 + j * 32;
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int row = row0 + i * 32 + 8 * (r >> 2) + (r & 3);
                    if (row < M && col < N) {
                        float v = alpha * acc[i][j][r];
                        if (use_c) v += beta * p.Cin[(int64_t)row * p.ldcin + col];
                        out[(int64_t)row * ldo + col] = v;
                    }
                }
            }
    }
}

// ------------------------------------------------------------------------------------
// Tiled MFMA kernel
// ------------------------------------------------------------------------------------
template <int BM, int BN, int WM, int WN, bool VEC>
__global__ void __launch_bounds__(WM * WN * kWave)
gemm_tiled_kernel(GemmArgs p) {
    constexpr int NT = WM * WN * kWave;
    constexpr int TM = BM / WM, TN = BN / WN;  // wave tile
    constexpr int FM = TM / 32, FN = TN / 32;  // 32x32 MFMA tiles per wave
    constexpr int A_CH = BM * 8;               // 16-byte chunks of one A stage
    constexpr int B_CH = BN * 8;               // 16-byte chunks of one B^T stage
    constexpr int STAGE = A_CH + B_CH;
    constexpr int A_PER = A_CH / NT;           // A chunks per thread
    constexpr int B_BLK = BN;                  // 8x8 blocks per B stage: (BK/8)*(BN/8)
    constexpr int B_PER = (B_BLK + NT - 1) / NT;
    static_assert(A_CH % NT == 0, "A stage must split evenly over threads");
    static_assert(TM % 32 == 0 && TN % 32 == 0, "wave tile must be a multiple of 32");

    __shared__ u32x4 smem[2 * STAGE];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;

    const int tiles = p.tiles_m * p.tiles_n;
    int tm, tn;
    grouped_tile(xcd_remap(blockIdx.x, tiles), p.tiles_m, p.tiles_n, 4, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * BN;
    const int kbeg = blockIdx.y * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int nk = kend > kbeg ? (kend - kbeg + BK - 1) / BK : 0;

    const int M = p.M, N = p.N;
    const int64_t lda = p.lda, ldb = p.ldb;

    f32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x16{};

    u32x4 ra[A_PER];
    u32x4 rb[B_PER][8];

    // Global -> registers for the stage starting at k0.
    auto gload = [&](int k0) {
        const __amdgpu_buffer_rsrc_t ra_rs = make_rsrc(p.A + (int64_t)m0 * lda + k0);
        const __amdgpu_buffer_rsrc_t rb_rs = make_rsrc(p.B + (int64_t)k0 * ldb + n0);
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int v = tid + i * NT;
            const int r = v >> 3, c = v & 7;
            const bool row_ok = m0 + r < M;
            if constexpr (VEC) {
                const bool ok = row_ok && (k0 + c * 8 < kend);
                ra[i] = buf_load16(ra_rs, ok ? (uint32_t)((r * lda + c * 8) * 2) : kOobOffset);
            } else {
                u32x4 v4;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const int k = k0 + c * 8 + e;
                    uint32_t lo = buf_load2(ra_rs, row_ok && k < kend
                                                       ? (uint32_t)((r * lda + c * 8 + e) * 2)
                                                       : kOobOffset);
                    uint32_t hi = buf_load2(ra_rs, row_ok && k + 1 < kend
                                                       ? (uint32_t)((r * lda + c * 8 + e + 1) * 2)
                                                       : kOobOffset);
                    v4[e >> 1] = lo | (hi << 16);
                }
                ra[i] = v4;
            }
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int b = tid + i * NT;
            const int kb = b / (BN / 8), nb = b % (BN / 8);
            if (B_PER * NT == B_BLK || b < B_BLK) {
#pragma unroll
                for (int r = 0; r < 8; ++r) {
                    const int k = k0 + kb * 8 + r;
                    if constexpr (VEC) {
                        const bool ok = (k < kend) && (n0 + nb * 8 < N);
                        rb[i][r] = buf_load16(
                            rb_rs, ok ? (uint32_t)(((kb * 8 + r) * ldb + nb * 8) * 2) : kOobOffset);
                    } else {
                        u32x4 v4;
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const int n = n0 + nb * 8 + e;
                            uint32_t lo = buf_load2(
                                rb_rs, (k < kend && n < N)
                                           ? (uint32_t)(((kb * 8 + r) * ldb + nb * 8 + e) * 2)
                                           : kOobOffset);
                            uint32_t hi = buf_load2(
                                rb_rs, (k < kend && n + 1 < N)
                                           ? (uint32_t)(((kb * 8 + r) * ldb + nb * 8 + e + 1) * 2)
                                           : kOobOffset);
                            v4[e >> 1] = lo | (hi << 16);
                        }
                        rb[i][r] = v4;
                    }
                }
            }
        }
    };

    // Registers -> LDS stage `buf`.  A rows keep K contiguous; B is stored transposed
    // (row = n, K contiguous).
    auto sstore = [&](int buf) {
        u32x4* s = smem + buf * STAGE;
#pragma unroll
        for (int i = 0; i < A_PER; ++i) {
            const int v = tid + i * NT;
            const int r = v >> 3, c = v & 7;
            s[r * 8 + (c ^ swz8(r))] = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_PER; ++i) {
            const int b = tid + i * NT;
            const int kb = b / (BN / 8), nb = b % (BN / 8);
            if (B_PER * NT == B_BLK || b < B_BLK) {
                u32x4 t[8];
                transpose8x8(rb[i], t);
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    const int n = nb * 8 + j;
                    s[A_CH + n * 8 + (kb ^ swz8(n))] = t[j];
                }
            }
        }
    };

    auto compute = [&](int buf) {
        const u32x4* s = smem + buf * STAGE;
#pragma unroll
        for (int ks = 0; ks < BK / 16; ++ks) {
            const int ch = ks * 2 + (lane >> 5);
            f16x8 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; ++i) {
                const int r = wm * TM + i * 32 + (lane & 31);
                af[i] = as_f16x8(s[r * 8 + (ch ^ swz8(r))]);
            }
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int n = wn * TN + j * 32 + (lane & 31);
                bf[j] = as_f16x8(s[A_CH + n * 8 + (ch ^ swz8(n))]);
            }
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) acc[i][j] = mfma32(af[i], bf[j], acc[i][j]);
        }
    };

    if (nk > 0) {
        gload(kbeg);
        sstore(0);
    }
    __syncthreads();
    for (int it = 0; it < nk; ++it) {
        const int cur = it & 1;
        const bool more = it + 1 < nk;
        if (more) gload(kbeg + (it + 1) * BK);
        compute(cur);
        if (more) sstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue.  D layout: lane column lane%32, element r -> row 8*(r/4)+4*(lane/32)+r%4.
    const bool partial = p.split > 1;
    float* out = partial ? p.ws + (size_t)blockIdx.y * (size_t)M * (size_t)N : p.Cout;
    const int64_t ldo = partial ? (int64_t)N : p.ldc;
    const bool use_c = !partial && p.beta != 0.0f && p.Cin != nullptr;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const int col = n0 + wn * TN + j * 32 + (lane & 31);
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int row = m0 + wm * TM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                if (row < M && col < N) {
                    float v = acc[i][j][r];
                    if (!partial) {
                        v = p.alpha * v;
                        if (use_c) v += p.beta * p.Cin[(int64_t)row * p.ldcin + col];
                    }
                    out[(int64_t)row * ldo + col] = v;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------
// Skinny kernel (M <= 16 * MB, MB = 1, 2, 4): C^T[N,M] = B^T[N,K] A^T[K,M] on MFMA
// 16x16x32.  Workgroup: 4 waves, 128 output columns, K range [kbeg,kend) split round-robin
// over the waves in 32-deep steps.  Lane l loads B rows k0+8*(l/16)+0..7 at columns
// 8*(l%16)+0..7 (16 lanes read 256 contiguous bytes per row), transposes the 8x8 block
// in registers, and issues 8 MFMAs per 16 activation rows: MFMA j covers columns 8*i+j
// (i = matrix row l%16) against rows 16*mb .. +15 of A, so each streamed B byte feeds MB
// times the multiply-adds.
// ------------------------------------------------------------------------------------
constexpr int SK_COLS = kSkinnyBlockN;
constexpr int SK_WAVES = 4;

// B row modes of the skinny kernel.  In every mode but SKB_ELEM, A is read in 16-byte
// vectors (K, lda multiples of 8, A 16-byte aligned).
enum SkinnyB {
    SKB_ELEM = 0,   // A and B element-wise (any alignment)
    SKB_VEC = 1,    // B rows 16-byte aligned: one 16-byte load per row chunk
    SKB_AL4 = 2,    // B 4-byte aligned, ldb even: every row 4-byte aligned.  A 16-byte load
                    // at a 4-byte-aligned address is a legal dword-aligned access.
    SKB_AL4_ODD = 3 // B 4-byte aligned, ldb odd: rows k0+r with r even are 4-byte aligned
                    // (k0 is even), odd ones start 2 bytes past a dword: a 16-byte load from
                    // 2 bytes earlier plus the next dword, shifted together by v_alignbyte.
};

template <int BMODE, int MB>
__global__ void __launch_bounds__(SK_WAVES * kWave)
gemm_skinny_kernel(GemmArgs p) {
    // Partial sums of one 16-row block, row m = lane%16 of each wave, column n at
    // n ^ ((n >> 2) & 16) of a row padded to 129 floats: one store instruction (64 lanes:
    // 16 rows x 4 K quarters) then hits 64 distinct banks (unpadded rows put all 16 rows of
    // a column on one bank), and a reader walking consecutive columns still sees distinct
    // banks.  The MB row blocks take turns in it (the LDS stays small enough for several
    // workgroups per CU).
    __shared__ float red[SK_WAVES][16][SK_COLS + 1];
    auto red_col = [](int n) { return n ^ ((n >> 2) & 16); };

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar descriptors
    const int q = lane >> 4;   // K quarter
    const int c16 = lane & 15;
    const int n0 = blockIdx.x * SK_COLS;
    const int kbeg = blockIdx.y * p.k_per_split;
    const int kend = min(p.K, kbeg + p.k_per_split);
    const int M = p.M, N = p.N;

    f32x4 acc[MB][8];
#pragma unroll
    for (int mb = 0; mb < MB; ++mb)
#pragma unroll
        for (int j = 0; j < 8; ++j) acc[mb][j] = f32x4{};

    const __amdgpu_buffer_rsrc_t a_rs = make_rsrc(p.A);
    const int ncol = n0 + 8 * c16;

    if constexpr (BMODE != SKB_ELEM) {
        // Straight-line double buffering: slab i+1's loads are in flight while slab i is
        // transposed and multiplied.  Every load is unconditional -- rows past kend and
        // columns past N come back as zeros through the buffer range check -- so each
        // wait covers exactly the slab it needs; slabs past the end are all zeros.  In the
        // 4-byte modes the chunk that straddles column N (N not a multiple of 8) is read
        // element-wise by the lanes that own it.
        struct Slab {
            u32x4 b[8];
            u32x4 a[MB];
        };
        constexpr int STEP = SK_WAVES * 32;
        const int nsl = (kend - kbeg + STEP - 1) / STEP;  // slabs per wave (uniform)
        auto load = [&](int i, Slab& S) {
            const int k0 = kbeg + wave * 32 + i * STEP;
            const int ka = k0 + 8 * q;
            const __amdgpu_buffer_rsrc_t b_rs = make_rsrc(p.B + (int64_t)k0 * p.ldb + n0);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const uint32_t off = (uint32_t)(((8 * q + r) * p.ldb + 8 * c16) * 2);
                if constexpr (BMODE == SKB_VEC) {
                    const bool ok = (ka + r < kend) && (ncol < N);
                    S.b[r] = buf_load16_nt(b_rs, ok ? off : kOobOffset);
                } else {
                    const bool k_ok = ka + r < kend;
                    const bool whole = k_ok && ncol + 8 <= N;
                    if (BMODE == SKB_AL4 || (r & 1) == 0) {
                        S.b[r] = buf_load16_nt(b_rs, whole ? off : kOobOffset);
                    } else {
                        // bytes [off-2, off+14) and [off+14, off+18): the dword at off+14
                        // holds the chunk's last element, so it lies inside B
                        const u32x4 x = buf_load16_nt(b_rs, whole ? off - 2 : kOobOffset);
                        const uint32_t y = buf_load4(b_rs, whole ? off + 14 : kOobOffset);
                        S.b[r] = u32x4{__builtin_amdgcn_alignbyte(x[1], x[0], 2),
                                       __builtin_amdgcn_alignbyte(x[2], x[1], 2),
                                       __builtin_amdgcn_alignbyte(x[3], x[2], 2),
                                       __builtin_amdgcn_alignbyte(y, x[3], 2)};
                    }
                    if (k_ok && ncol < N && ncol + 8 > N) {
                        u32x4 v4;
#pragma unroll
                        for (int e = 0; e < 8; e += 2) {
                            const uint32_t lo = buf_load2(b_rs, ncol + e < N ? off + 2 * e : kOobOffset);
                            const uint32_t hi = buf_load2(b_rs, ncol + e + 1 < N ? off + 2 * e + 2 : kOobOffset);
                            v4[e >> 1] = lo | (hi << 16);
                        }
                        S.b[r] = v4;
                    }
                }
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int m = 16 * mb + c16;
                S.a[mb] = buf_load16(a_rs, (m < M && ka < kend) ? (uint32_t)((m * p.lda + ka) * 2)
                                                               : kOobOffset);
            }
        };
        auto compute = [&](const Slab& S) {
            u32x4 bt[8];
            transpose8x8(S.b, bt);
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const f16x8 a8 = as_f16x8(S.a[mb]);
#pragma unroll
                for (int j = 0; j < 8; ++j) acc[mb][j] = mfma16(as_f16x8(bt[j]), a8, acc[mb][j]);
            }
        };
        Slab S0, S1;
        load(0, S0);
        for (int i = 0; i < nsl; i += 2) {
            load(i + 1, S1);
            compute(S0);
            load(i + 2, S0);
            compute(S1);
        }
    } else {
    for (int k0 = kbeg + wave * 32; k0 < kend; k0 += SK_WAVES * 32) {
        const __amdgpu_buffer_rsrc_t b_rs = make_rsrc(p.B + (int64_t)k0 * p.ldb + n0);
        u32x4 rb[8];
        u32x4 av[MB];
        const int ka = k0 + 8 * q;
        {
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                u32x4 v4;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    const bool k_ok = ka + r < kend;
                    uint32_t lo = buf_load2(b_rs, (k_ok && ncol + e < N)
                                                      ? (uint32_t)(((8 * q + r) * p.ldb + 8 * c16 + e) * 2)
                                                      : kOobOffset);
                    uint32_t hi = buf_load2(b_rs, (k_ok && ncol + e + 1 < N)
                                                      ? (uint32_t)(((8 * q + r) * p.ldb + 8 * c16 + e + 1) * 2)
                                                      : kOobOffset);
                    v4[e >> 1] = lo | (hi << 16);
                }
                rb[r] = v4;
            }
#pragma unroll
            for (int mb = 0; mb < MB; ++mb) {
                const int m = 16 * mb + c16;
                u32x4 v4;
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    uint32_t lo = buf_load2(a_rs, (m < M && ka + e < kend)
                                                      ? (uint32_t)((m * p.lda + ka + e) * 2)
                                                      : kOobOffset);
                    uint32_t hi = buf_load2(a_rs, (m < M && ka + e + 1 < kend)
                                                      ? (uint32_t)((m * p.lda + ka + e + 1) * 2)
                                                      : kOobOffset);
                    v4[e >> 1] = lo | (hi << 16);
                }
                av[mb] = v4;
            }
        }
        u32x4 bt[8];
        transpose8x8(rb, bt);
#pragma unroll
        for (int mb = 0; mb < MB; ++mb) {
            const f16x8 a8 = as_f16x8(av[mb]);
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[mb][j] = mfma16(as_f16x8(bt[j]), a8, acc[mb][j]);
        }
    }
    }

    // D of MFMA j: lane holds m = lane%16, rows 4*(lane/16)+r -> column 8*(4q+r)+j.
    // Without a K split the epilogue is applied here; with one, this workgroup's partial
    // goes to the workspace and splitk_reduce_kernel sums the partials in split order and
    // applies the epilogue.
    const bool use_c = p.beta != 0.0f && p.Cin != nullptr;
    float* part = p.split > 1 ? p.ws + (size_t)blockIdx.y * (size_t)M * (size_t)N : nullptr;
#pragma unroll
    for (int mb = 0; mb < MB; ++mb) {
        if (mb > 0) __syncthreads();  // the previous block's readers are done with red
#pragma unroll
        for (int j = 0; j < 8; ++j)
#pragma unroll
            for (int r = 0; r < 4; ++r) red[wave][c16][red_col(8 * (4 * q + r) + j)] = acc[mb][j][r];
        __syncthreads();
        for (int idx = tid; idx < 16 * SK_COLS; idx += SK_WAVES * kWave) {
            const int ml = idx / SK_COLS, n = idx % SK_COLS, m = 16 * mb + ml;
            if (m < M && n0 + n < N) {
                const int cn = red_col(n);
                float v = red[0][ml][cn];
#pragma unroll
                for (int w = 1; w < SK_WAVES; ++w) v += red[w][ml][cn];
                if (p.split == 1) {
                    v = p.alpha * v;
                    if (use_c) v += p.beta * p.Cin[(int64_t)m * p.ldcin + n0 + n];
                    p.Cout[(int64_t)m * p.ldc + n0 + n] = v;
                } else {
                    part[(int64_t)m * N + n0 + n] = v;
                }
            }
        }
    }
}

// ------------------------------------------------------------------------------------
// Split-K reduction + epilogue: out = alpha * sum_s ws[s] (+ beta * C_in).  One thread per
// W columns of a row (W = 4 when N is a multiple of 4 and the workspace 16-byte aligned).
// ------------------------------------------------------------------------------------
template <int W>
__global__ void __launch_bounds__(256)
splitk_reduce_kernel(const float* ws, int split, const float* Cin, int64_t ldcin, float* Cout,
                     int64_t ldc, int M, int N, float alpha, float beta) {
    const int64_t total = (int64_t)M * N;
    const bool use_c = beta != 0.0f && Cin != nullptr;
    const int nv = (N + W - 1) / W;
    for (int row = blockIdx.y; row < M; row += gridDim.y) {
        for (int q = blockIdx.x * blockDim.x + threadIdx.x; q < nv; q += gridDim.x * blockDim.x) {
            const int col = q * W;
            float v[W];
            splitk_sum<W>(ws + (int64_t)row * N + col, total, split, v);
#pragma unroll
            for (int e = 0; e < W; ++e) {
                float r = alpha * v[e];
                if (use_c) r += beta * Cin[(int64_t)row * ldcin + col + e];
                Cout[(int64_t)row * ldc + col + e] = r;
            }
        }
    }
}

// ------------------------------------------------------------------------------------
// Operand repack for rows that break 16-byte vectors: a [rows][cols] fp16 matrix with
// leading dimension ld (any alignment) becomes a dense [rows][cols_p] copy, cols_p = cols
// rounded up to 8, whose columns cols..cols_p-1 are zero.  One wave per row, one output
// dword (two fp16) per lane and step; a row whose start is 4-byte aligned is read a dword
// at a time, any other row in 16-bit halves.  Both sides are contiguous across the lanes
// of a wave.
// ------------------------------------------------------------------------------------
constexpr int RP_WAVES = 4;  // rows per workgroup
constexpr int RP_STEPS = 4;  // dwords per lane and row (a workgroup covers 256 of a row)

__global__ void __launch_bounds__(RP_WAVES * kWave)
gemm_repack_kernel(const f16* src, int64_t ld, int rows, int cols, uint32_t* dst) {
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int dw_row = ((cols + 7) & ~7) >> 1;
    const int w0 = blockIdx.x * (kWave * RP_STEPS) + lane;
    for (int r = blockIdx.y * RP_WAVES + wave; r < rows; r += gridDim.y * RP_WAVES) {
        const f16* s = src + (int64_t)r * ld;
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(s);
        const bool al4 = (reinterpret_cast<uintptr_t>(s) & 3u) == 0;
        uint32_t v[RP_STEPS];
#pragma unroll
        for (int u = 0; u < RP_STEPS; ++u) {
            const int c = 2 * (w0 + u * kWave);  // first column of this dword
            if (al4) {
                v[u] = buf_load4(rs, c + 1 < cols ? (uint32_t)c * 2 : kOobOffset);
                if (c + 1 == cols) v[u] = buf_load2(rs, (uint32_t)c * 2);  // odd cols: last one
            } else {
                const uint32_t lo = buf_load2(rs, c < cols ? (uint32_t)c * 2 : kOobOffset);
                const uint32_t hi = buf_load2(rs, c + 1 < cols ? (uint32_t)(c + 1) * 2 : kOobOffset);
                v[u] = lo | (hi << 16);
            }
        }
        uint32_t* d = dst + (int64_t)r * dw_row;
#pragma unroll
        for (int u = 0; u < RP_STEPS; ++u) {
            const int w = w0 + u * kWave;
            if (w < dw_row) d[w] = v[u];
        }
    }
}

template <int CFG, bool VEC>
void launch_tiled(const GemmArgs& a, hipStream_t stream) {
    constexpr TileShape t = kTiles[CFG];
    dim3 grid(a.tiles_m * a.tiles_n, a.split);
    hipLaunchKernelGGL((gemm_tiled_kernel<t.bm, t.bn, t.wm, t.wn, VEC>), grid,
                       dim3(t.wm * t.wn * kWave), 0, stream, a);
}

template <bool VEC>
void launch_tiled_cfg(int cfg, const GemmArgs& a, hipStream_t stream) {
    switch (cfg) {
        case 0: launch_tiled<0, VEC>(a, stream); break;
        case 1: launch_tiled<1, VEC>(a, stream); break;
        case 2: launch_tiled<2, VEC>(a, stream); break;
        case 3: launch_tiled<3, VEC>(a, stream); break;
        case 4: launch_tiled<4, VEC>(a, stream); break;
        default: launch_tiled<5, VEC>(a, stream); break;
    }
}

// LDS-DMA kernel: K depth of a stage and LDS ring depth per tile configuration, chosen
// so that the ring fits the 160 KB of LDS of one CU.
struct MfmaStages {
    int bk, ns;
};
constexpr MfmaStages kMfmaStages[WMMA_TILE_COUNT] = {
    {64, 4}, {64, 4}, {64, 3}, {64, 4}, {64, 3}, {32, 4}};

template <int CFG>
void launch_mfma(const GemmArgs& a, hipStream_t stream) {
    constexpr TileShape t = kTiles[CFG];
    constexpr MfmaStages st = kMfmaStages[CFG];
    dim3 grid(a.tiles_m * a.tiles_n, a.split);
    hipLaunchKernelGGL((gemm_mfma_kernel<t.bm, t.bn, st.bk, t.wm, t.wn, st.ns>), grid,
                       dim3(t.wm * t.wn * kWave), 0, stream, a);
}

// Skinny kernel with MB 16-row blocks of activations (M <= 16 * MB).
template <int MB>
void launch_skinny(int bmode, const GemmArgs& a, hipStream_t stream) {
    const dim3 grid(ceil_div(a.N, SK_COLS), a.split), block(SK_WAVES * kWave);
    switch (bmode) {
        case SKB_VEC: hipLaunchKernelGGL((gemm_skinny_kernel<SKB_VEC, MB>), grid, block, 0, stream, a); break;
        case SKB_AL4: hipLaunchKernelGGL((gemm_skinny_kernel<SKB_AL4, MB>), grid, block, 0, stream, a); break;
        case SKB_AL4_ODD:
            hipLaunchKernelGGL((gemm_skinny_kernel<SKB_AL4_ODD, MB>), grid, block, 0, stream, a);
            break;
        default: hipLaunchKernelGGL((gemm_skinny_kernel<SKB_ELEM, MB>), grid, block, 0, stream, a); break;
    }
}

void launch_mfma_cfg(int cfg, const GemmArgs& a, hipStream_t stream) {
    switch (cfg) {
        case 0: launch_mfma<0>(a, stream); break;
        case 1: launch_mfma<1>(a, stream); break;
        case 2: launch_mfma<2>(a, stream); break;
        case 3: launch_mfma<3>(a, stream); break;
        case 4: launch_mfma<4>(a, stream); break;
        default: launch_mfma<5>(a, stream); break;
    }
}

}  // namespace

hipError_t launch_gemm_repack(const void* src, int64_t ld, int rows, int cols, void* dst,
                              hipStream_t stream) {
    if (rows <= 0 || cols <= 0) return hipSuccess;
    const int dw_row = ((cols + 7) & ~7) >> 1;
    const dim3 grid(ceil_div(dw_row, kWave * RP_STEPS), std::min(ceil_div(rows, RP_WAVES), 65535));
    hipLaunchKernelGGL(gemm_repack_kernel, grid, dim3(RP_WAVES * kWave), 0, stream,
                       static_cast<const f16*>(src), ld, rows, cols, static_cast<uint32_t*>(dst));
    return hipGetLastError();
}

hipError_t launch_gemm(const GemmLaunch& g, hipStream_t stream) {
    const wmma_gemm_plan& pl = g.plan;
    GemmArgs a{};
    a.A = static_cast<const f16*>(g.A);
    a.B = static_cast<const f16*>(g.B);
    a.Cin = g.C_in;
    a.Cout = g.C_out;
    a.ws = static_cast<float*>(g.workspace);
    a.lda = g.lda;
    a.ldb = g.ldb;
    a.ldcin = g.ldc_in;
    a.ldc = g.ldc;
    a.M = g.M;
    a.N = g.N;
    a.K = g.K;
    a.alpha = g.alpha;
    a.beta = g.beta;
    a.k_per_split = pl.k_per_split > 0 ? pl.k_per_split : 1;
    a.split = pl.split_k;
    a.tiles_m = ceil_div(g.M, pl.tile_m);
    a.tiles_n = ceil_div(g.N, pl.tile_n);

    if (pl.kernel == WMMA_KERNEL_SKINNY) {
        const int bmode = g.vec ? (int)SKB_VEC : g.skinny_b;
        if (g.M <= 16)
            launch_skinny<1>(bmode, a, stream);
        else if (g.M <= 32)
            launch_skinny<2>(bmode, a, stream);
        else
            launch_skinny<4>(bmode, a, stream);
    } else {
        if (g.vec)
            launch_mfma_cfg(pl.tile_cfg, a, stream);
        else
            launch_tiled_cfg<false>(pl.tile_cfg, a, stream);
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || pl.split_k <= 1) return e;

    const bool vec4 = g.N % 4 == 0 && (reinterpret_cast<uintptr_t>(g.workspace) & 15u) == 0;
    const int nv = vec4 ? g.N / 4 : g.N;
    const dim3 grid(std::min(ceil_div(nv, 256), 64), std::min(g.M, 65535));
    const float* ws = static_cast<const float*>(g.workspace);
    if (vec4)
        hipLaunchKernelGGL(splitk_reduce_kernel<4>, grid, dim3(256), 0, stream, ws, pl.split_k,
                           g.C_in, g.ldc_in, g.C_out, g.ldc, g.M, g.N, g.alpha, g.beta);
    else
        hipLaunchKernelGGL(splitk_reduce_kernel<1>, grid, dim3(256), 0, stream, ws, pl.split_k,
                           g.C_in, g.ldc_in, g.C_out, g.ldc, g.M, g.N, g.alpha, g.beta);
    return hipGetLastError();
}

}  // namespace wmma_amd
