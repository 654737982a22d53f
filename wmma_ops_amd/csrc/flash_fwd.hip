// Flash-attention forward for gfx950:  O = softmax(scale * Q K^T [+ causal mask]) V.
//
// The reference documents flash_attention(Q, K, V, causal=False, scale=-1.0) on
// [B, H, N, D] fp16 tensors with default scale 1/sqrt(D) (README.md:221-251); its kernel
// was removed.  This is a new MFMA design:
//
//  * A workgroup owns 128 queries of one (batch, head): 4 waves x 32 queries.
//  * Scores are computed transposed, S^T = K Q^T, on MFMA 32x32x16 with K as the matrix
//    A operand (rows = keys, read K-contiguous from LDS) and the wave's Q fragments as
//    the B operand (held in registers for the whole kernel).  In the S^T accumulator
//    every lane owns ONE query (lane%32) and 16 keys of each 32-key block; the
//    other 16 keys of that query live in lane^32.  Row max and row sum are therefore
//    lane-local plus one exchange with lane^32.
//  * The probabilities stay in registers: the accumulator elements of one lane are
//    exactly the K-operand a lane must supply for the PV product O^T = V^T P^T (P^T as
//    the B operand, lane = query), so no cross-lane movement of P is needed.  V^T is
//    staged in LDS (keys contiguous) by an 8x8 register transpose on the way in, and
//    each lane reads the eight keys that pair with its P elements.
//  * FP32 online softmax in base 2 (scale * log2 e folded into one multiply), FP32
//    accumulation, fp16 output.  K/V tiles of 64 keys are double-buffered in LDS; the
//    next tile's global loads are in flight during the current tile's math.
//  * Causal (key j <= query i, the top-left convention of torch SDPA's is_causal): key
//    tiles beyond the workgroup's last query are never loaded, fully masked tiles are
//    skipped per wave, and the heaviest query blocks are dispatched first.
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
    int nqb;          // query blocks
    float scale_log2;  // scale * log2(e)
};

constexpr int FA_WAVES = 4;
constexpr int FA_BQ = 32 * FA_WAVES;  // 128 queries per workgroup
constexpr int FA_BKV = 64;            // keys per LDS tile
constexpr float kNegInf = -__builtin_huge_valf();

template <int D, bool CAUSAL>
__global__ void __launch_bounds__(FA_WAVES * kWave)
flash_fwd_kernel(FlashArgs p) {
    constexpr int DCH = D / 8;                 // 16-byte chunks per K row
    constexpr int K_CH = FA_BKV * DCH;         // chunks per K tile
    constexpr int VT_CH = D * (FA_BKV / 8);    // chunks per V^T tile (8 per d row)
    constexpr int NDB = D / 32;                // 32-wide d blocks of O
    constexpr int NDS = D / 16;                // 16-deep d steps of QK^T
    constexpr int NT = FA_WAVES * kWave;
    // loaders: threads [0,VT_THREADS) transpose V 8x8 blocks, the rest copy K chunks.
    constexpr int V_BLOCKS = (FA_BKV / 8) * (D / 8);
    constexpr int VT_THREADS = V_BLOCKS;                // one block per thread
    constexpr int K_THREADS = NT - VT_THREADS;
    constexpr int K_PER = (K_CH + K_THREADS - 1) / K_THREADS;
    static_assert(VT_THREADS < NT, "loader split");
    static_assert(K_PER <= 8, "loader registers");

    __shared__ u32x4 sk[2][K_CH];
    __shared__ u32x4 sv[2][VT_CH];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int h = lane >> 5, c32 = lane & 31;
    const int bh = blockIdx.x;
    const int qb = CAUSAL ? (p.nqb - 1 - (int)blockIdx.y) : (int)blockIdx.y;
    const int q0 = qb * FA_BQ;
    const int qw = q0 + wave * 32;
    const int Sq = p.Sq, Sk = p.Sk;

    const f16* Qb = p.Q + (int64_t)bh * Sq * D;
    const f16* Kb = p.K + (int64_t)bh * Sk * D;
    const f16* Vb = p.V + (int64_t)bh * Sk * D;
    f16* Ob = p.O + (int64_t)bh * Sq * D;

    // Q fragments (B operand): query qw + lane%32, d = 16*s + 8*h + 0..7.
    f16x8 qf[NDS];
    {
        const __amdgpu_buffer_rsrc_t rs = make_rsrc(Qb);
        const int q = qw + c32;
#pragma unroll
        for (int s = 0; s < NDS; ++s)
            qf[s] = as_f16x8(buf_load16(
                rs, q < Sq ? (uint32_t)(((int64_t)q * D + 16 * s + 8 * h) * 2) : kOobOffset));
    }

    f32x16 o[NDB];
#pragma unroll
    for (int i = 0; i < NDB; ++i) o[i] = f32x16{};
    float m_run = kNegInf, l_run = 0.0f;

    const int kv_end = CAUSAL ? min(Sk, q0 + FA_BQ) : Sk;
    const int nkv = (kv_end + FA_BKV - 1) / FA_BKV;

    u32x4 pre[8];
    auto gload = [&](int kv0) {
        if (tid < VT_THREADS) {
            const int kb8 = tid / (D / 8), db8 = tid % (D / 8);
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(Vb);
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const int key = kv0 + kb8 * 8 + r;
                pre[r] = buf_load16(rs, key < Sk ? (uint32_t)(((int64_t)key * D + db8 * 8) * 2)
                                                 : kOobOffset);
            }
        } else {
            const __amdgpu_buffer_rsrc_t rs = make_rsrc(Kb);
#pragma unroll
            for (int i = 0; i < K_PER; ++i) {
                const int c = (tid - VT_THREADS) + i * K_THREADS;
                const int key = kv0 + c / DCH, ch = c % DCH;
                if (K_CH % K_THREADS == 0 || c < K_CH)
                    pre[i] = buf_load16(rs, key < Sk ? (uint32_t)(((int64_t)key * D + ch * 8) * 2)
                                                     : kOobOffset);
            }
        }
    };
    auto sstore = [&](int buf) {
        if (tid < VT_THREADS) {
            const int kb8 = tid / (D / 8), db8 = tid % (D / 8);
            u32x4 t[8];
            transpose8x8(pre, t);
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const int d = db8 * 8 + j;
                sv[buf][d * 8 + (kb8 ^ swz8(d))] = t[j];
            }
        } else {
#pragma unroll
            for (int i = 0; i < K_PER; ++i) {
                const int c = (tid - VT_THREADS) + i * K_THREADS;
                const int key = c / DCH, ch = c % DCH;
                if (K_CH % K_THREADS == 0 || c < K_CH) sk[buf][key * DCH + (ch ^ swz8(key))] = pre[i];
            }
        }
    };

    if (nkv > 0) {
        gload(0);
        sstore(0);
    }
    __syncthreads();

    const int myq = qw + c32;
    for (int j = 0; j < nkv; ++j) {
        const int cur = j & 1;
        const int kv0 = j * FA_BKV;
        const bool more = j + 1 < nkv;
        if (more) gload(kv0 + FA_BKV);

        const bool active = !CAUSAL || kv0 <= qw + 31;
        if (active) {
            // S^T = K Q^T for two 32-key sub-blocks.
            f32x16 s[2] = {f32x16{}, f32x16{}};
#pragma unroll
            for (int ds = 0; ds < NDS; ++ds) {
                const int ch = 2 * ds + h;
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
                    const int key = kb * 32 + c32;
                    const f16x8 kf = as_f16x8(sk[cur][key * DCH + (ch ^ swz8(key))]);
                    s[kb] = mfma32(kf, qf[ds], s[kb]);
                }
            }
            // scale, mask, running max
            float mloc = kNegInf;
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int key = kv0 + kb * 32 + 8 * (r >> 2) + 4 * h + (r & 3);
                    bool ok = key < Sk;
                    if (CAUSAL) ok = ok && key <= myq;
                    const float x = ok ? s[kb][r] * p.scale_log2 : kNegInf;
                    s[kb][r] = x;
                    mloc = fmaxf(mloc, x);
                }
            }
            mloc = fmaxf(mloc, __shfl_xor(mloc, 32));
            const float m_new = fmaxf(m_run, mloc);
            const float m_use = m_new == kNegInf ? 0.0f : m_new;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_use);
            m_run = m_new;
            float lsum = 0.0f;
            f16x8 pf[2][2];
#pragma unroll
            for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
                    for (int e = 0; e < 8; ++e) {
                        const float pv = __builtin_amdgcn_exp2f(s[kb][8 * hh + e] - m_use);
                        lsum += pv;
                        pf[kb][hh][e] = (f16)pv;
                    }
                }
            }
            l_run = l_run * alpha + lsum;
#pragma unroll
            for (int i = 0; i < NDB; ++i) o[i] *= alpha;
            // O^T += V^T P^T.  MFMA (kb, hh) pairs element e of lane half h with key
            // kb*32 + 16*hh + 4*h + (e < 4 ? e : e + 4).
#pragma unroll
            for (int db = 0; db < NDB; ++db) {
                const int d = db * 32 + c32;
                const u32x4* row = &sv[cur][d * 8];
                const int sw = swz8(d);
#pragma unroll
                for (int kb = 0; kb < 2; ++kb) {
#pragma unroll
                    for (int hh = 0; hh < 2; ++hh) {
                        const int ch0 = 4 * kb + 2 * hh;  // chunk of keys base..base+7
                        const u32x2 lo = reinterpret_cast<const u32x2*>(&row[ch0 ^ sw])[h];
                        const u32x2 hi = reinterpret_cast<const u32x2*>(&row[(ch0 + 1) ^ sw])[h];
                        const f16x8 vf = as_f16x8(u32x4{lo[0], lo[1], hi[0], hi[1]});
                        o[db] = mfma32(vf, pf[kb][hh], o[db]);
                    }
                }
            }
        }
        if (more) sstore(cur ^ 1);
        __syncthreads();
    }

    // normalise and store: lane owns query myq, d = 32*db + 8*(r/4) + 4*h + r%4.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (myq < Sq) {
#pragma unroll
        for (int db = 0; db < NDB; ++db) {
#pragma unroll
            for (int g = 0; g < 4; ++g) {
                f16x4 v;
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = (f16)(o[db][4 * g + e] * inv);
                const int d = db * 32 + 8 * g + 4 * h;
                *reinterpret_cast<f16x4*>(Ob + (int64_t)myq * D + d) = v;
            }
        }
    }
}

template <int D>
void launch_d(const FlashArgs& a, int BH, bool causal, hipStream_t stream) {
    dim3 grid(BH, a.nqb);
    if (causal)
        hipLaunchKernelGGL((flash_fwd_kernel<D, true>), grid, dim3(FA_WAVES * kWave), 0, stream, a);
    else
        hipLaunchKernelGGL((flash_fwd_kernel<D, false>), grid, dim3(FA_WAVES * kWave), 0, stream, a);
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
    a.nqb = ceil_div(f.Sq, FA_BQ);
    a.scale_log2 = f.scale * 1.4426950408889634f;
    const int BH = f.B * f.H;
    if (f.D == 128)
        launch_d<128>(a, BH, f.causal, stream);
    else
        launch_d<64>(a, BH, f.causal, stream);
    return hipGetLastError();
}

}  // namespace wmma_amd
