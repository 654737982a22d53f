// Host-only GEMM planner.  Chooses the kernel family, tile and split-K partition.
//
// The reference picks a tile from gfx1151-tuned thresholds (select_optimal_tile,
// wmma_tile_selection.hpp:30-66) and has an unreachable split-K config
// (compute_config, wmma_xor_swizzle.hpp:293-332: target tiles = 4 x CUs, split capped at
// 32 and at K/256, k_per_split = ceil(K/split)).  Here the choice is made against a
// 256-CU device, in four tiers: exact shapes from the autotuned table; M <= 16 with
// K > 1024 on the streaming kernel with its split rule; every other M <= 768 by a launch
// model fitted to measured times of every plan (model_plan); larger M by whole waves of
// workgroups, the tile that reuses the most bytes per LDS byte, a K split only when too
// few output tiles exist to occupy the CUs, and bulk + edge plans.  The result never
// depends on the plan beyond fp32 summation order.
#include "plan.hpp"

#include <algorithm>
#include <cstdint>

namespace wmma_amd {

static void finish_split(int M, int N, int K, int tiles, int split, wmma_gemm_plan* p) {
    // k_per_split is a whole number of 64-deep stages so that every split but the last
    // is full; the split count is then recomputed so no split is empty.
    int kps = ceil_div(ceil_div(K, split), kBlockK) * kBlockK;
    if (kps < kBlockK) kps = kBlockK;
    split = std::max(1, ceil_div(K, kps));
    p->split_k = split;
    p->k_per_split = split > 1 ? kps : std::max(K, 0);
    p->grid = tiles * split;
    p->workspace_bytes = split > 1 ? (size_t)split * (size_t)M * (size_t)N * sizeof(float) : 0;
}

// Lower the split of p until its partial sums fit max_ws (a plan without a split needs none).
static void fit_split(int M, int N, int K, size_t max_ws, wmma_gemm_plan* p) {
    const int tiles = p->grid / std::max(p->split_k, 1);
    for (int split = p->split_k - 1; p->workspace_bytes > max_ws && split >= 1; --split)
        finish_split(M, N, K, tiles, split, p);
}

double plan_time_us(const wmma_gemm_plan& p, int M, int N, int K, int num_cus) {
    if (M <= 0 || N <= 0 || K <= 0) return 0.0;
    if (num_cus <= 0) num_cus = 256;
    const double hbm = (2.0 * M * K + 2.0 * K * N + 4.0 * M * N) / kHbmBytesPerUs;
    const int split = std::max(p.split_k, 1);
    double t = hbm;
    if (p.kernel == WMMA_KERNEL_TILED) {
        const TileShape& ts = kTiles[p.tile_cfg];
        const double area = (double)ts.bm * ts.bn / 65536.0;
        const int64_t wgs = (int64_t)ceil_div(M, ts.bm) * ceil_div(N, ts.bn) * split;
        const int kps = split > 1 ? p.k_per_split : K;
        const double wave = area * (kEpiUs256 + kWaveUsPerK256 * kps / kWaveEff[p.tile_cfg]);
        t = std::max((double)ceil_div64(wgs, num_cus) * wave, hbm);
    }
    if (split > 1) t += (split + 1) * 4.0 * M * N / kHbmBytesPerUs + kReduceUs;
    return t + kLaunchUs;
}

double model_time_us(const wmma_gemm_plan& p, int M, int N, int K, int num_cus) {
    if (num_cus <= 0) num_cus = 256;
    const int split = std::max(p.split_k, 1);
    const double kk = split > 1 ? p.k_per_split : K;
    double t;
    if (p.kernel == WMMA_KERNEL_SKINNY) {
        const int mb = M <= 16 ? 16 : 32;
        const int64_t wgs = (int64_t)ceil_div(N, kSkinnyBlockN) * split;
        const double kb = (kSkinnyBlockN + mb) * kk * 2.0 / 1000.0;
        t = (double)ceil_div64(wgs, num_cus) * (kSkinnyWgFixedUs + kb / kSkinnyKbPerUs);
    } else {
        const TileShape& ts = kTiles[p.tile_cfg];
        const int64_t wgs = (int64_t)ceil_div(M, ts.bm) * ceil_div(N, ts.bn) * split;
        const double kb = (std::min(M, ts.bm) + ts.bn) * kk * 2.0 / 1000.0;
        const double mflop = 2.0 * ts.bm * ts.bn * kk / 1e6;
        const TileRate& r = kTileRate[p.tile_cfg];
        t = (double)ceil_div64(wgs, num_cus) *
            (kWgFixedUs + std::max(kb / r.kb_per_us, mflop / r.mflop_per_us));
    }
    const double mb_io = (2.0 * M * K + 2.0 * K * N + 4.0 * M * N) / 1e6;
    t = std::max(t, mb_io / kModelHbmMBPerUs);
    if (split > 1) t += kSplitFixedUs + kPartialUsPerMB * (split + 1) * 4.0 * M * N / 1e6;
    return t;
}

// The plan with the shortest modelled time: every tile with K splits 1, 2, 4, 8, 16 (a
// split only from K = 2048, at least 256 of K per part, and only while the workgroups fit
// one wave of the CUs), and for M <= 32 the streaming kernel with splits up to K / 256.
// Over the fitted shapes the choice costs 0.65% more time than the fastest plan of each
// shape (the previous heuristics: 14%), and 0.8% on a second sweep of 63 shapes.
static wmma_gemm_plan model_plan(int M, int N, int K, int num_cus, size_t max_ws) {
    wmma_gemm_plan best{};
    double best_t = 1e300;
    for (int cfg = 0; cfg < WMMA_TILE_COUNT; ++cfg) {
        const TileShape& ts = kTiles[cfg];
        const int64_t tiles = (int64_t)ceil_div(M, ts.bm) * ceil_div(N, ts.bn);
        for (int sp : {1, 2, 4, 8, 16}) {
            if (sp > 1 && (K / sp < 256 || K < 2048 || tiles * sp > num_cus)) break;
            wmma_gemm_plan c{};
            if (make_custom_plan(M, N, K, WMMA_KERNEL_TILED, cfg, sp, &c) != WMMA_OK ||
                c.workspace_bytes > max_ws)
                continue;
            const double t = model_time_us(c, M, N, K, num_cus);
            if (t < best_t * 0.999) {
                best_t = t;
                best = c;
            }
        }
    }
    if (M <= 32) {
        for (int sp : {1, 2, 3, 4, 5, 6, 8, 12, 16, 24, 32}) {
            if (sp > std::max(1, K / 256)) break;
            wmma_gemm_plan c{};
            if (make_custom_plan(M, N, K, WMMA_KERNEL_SKINNY, -1, sp, &c) != WMMA_OK ||
                c.workspace_bytes > max_ws)
                continue;
            const double t = model_time_us(c, M, N, K, num_cus);
            if (t < best_t * 0.999) {
                best_t = t;
                best = c;
            }
        }
    }
    return best;
}

// The autotuned table: exact shapes measured on a 256-CU MI355X.
#include "tuned_table.inc"

const TunedPlan* tuned_plans(int* count) {
    *count = (int)(sizeof(kTunedPlans) / sizeof(kTunedPlans[0]));
    return kTunedPlans;
}

int make_custom_plan(int M, int N, int K, int kernel, int tile_cfg, int split,
                     wmma_gemm_plan* out) {
    if (!out || M < 0 || N < 0 || K < 0 || split < 1 || split > kMaxSplitK)
        return WMMA_ERR_INVALID_ARG;
    wmma_gemm_plan p{};
    int tiles;
    if (kernel == WMMA_KERNEL_SKINNY) {
        if (M > kSkinnyMaxMWide) return WMMA_ERR_INVALID_ARG;
        p.kernel = WMMA_KERNEL_SKINNY;
        p.tile_cfg = -1;
        p.tile_m = M <= 16 ? 16 : (M <= 32 ? 32 : 64);
        p.tile_n = kSkinnyBlockN;
        tiles = ceil_div(std::max(N, 1), kSkinnyBlockN);
    } else if (kernel == WMMA_KERNEL_TILED) {
        if (tile_cfg < 0 || tile_cfg >= WMMA_TILE_COUNT) return WMMA_ERR_INVALID_ARG;
        const TileShape& t = kTiles[tile_cfg];
        p.kernel = WMMA_KERNEL_TILED;
        p.tile_cfg = tile_cfg;
        p.tile_m = t.bm;
        p.tile_n = t.bn;
        tiles = ceil_div(std::max(M, 1), t.bm) * ceil_div(std::max(N, 1), t.bn);
    } else {
        return WMMA_ERR_INVALID_ARG;
    }
    if (split > 1 && K < split * kBlockK) return WMMA_ERR_INVALID_ARG;
    finish_split(M, N, K, tiles, split, &p);
    *out = p;
    return WMMA_OK;
}

// Bulk + edge: when the 256x256 tiles of the shape fill W >= 1 whole waves plus part of
// another, the whole tile rows (or columns) that fit in W waves run as one launch and the
// rest as a GEMM of its own, planned on its own (it is small, so it may take a smaller
// tile or a K split and spread over the chip).  Measured on MI355X (N = K = 4096): M = 4352
// one launch of 128x128 tiles 193 us, 4096 + 256 rows 148 us; M = 5000: 209 vs 171 us;
// M = 9192: 347 vs 295 us.  Taken when plan_time_us says it gains more than 7%.
static void two_part(int M, int N, int K, int num_cus, size_t max_ws, wmma_gemm_plan* p) {
    const int64_t tm = ceil_div(M, 256), tn = ceil_div(N, 256);
    const int64_t whole = tm * tn / num_cus * num_cus;  // 256x256 tiles in whole waves
    if (whole == 0) return;
    double best_t = kEdgeGain * plan_time_us(*p, M, N, K, num_cus);
    for (int dim : {WMMA_EDGE_ROWS, WMMA_EDGE_COLS}) {
        const int64_t lines = whole / (dim == WMMA_EDGE_ROWS ? tn : tm);
        const int extent = dim == WMMA_EDGE_ROWS ? M : N;
        if (lines < 1 || lines * 256 >= extent) continue;
        const int at = (int)(lines * 256);
        const int bm = dim == WMMA_EDGE_ROWS ? at : M, bn = dim == WMMA_EDGE_ROWS ? N : at;
        const int em = dim == WMMA_EDGE_ROWS ? M - at : M, en = dim == WMMA_EDGE_ROWS ? N : N - at;
        wmma_gemm_plan bulk{}, edge{};
        if (make_custom_plan(bm, bn, K, WMMA_KERNEL_TILED, WMMA_TILE_256x256, 1, &bulk) != WMMA_OK ||
            make_plan_within(em, en, K, WMMA_TILE_AUTO, num_cus, max_ws, &edge) != WMMA_OK ||
            edge.edge_dim != WMMA_EDGE_NONE)
            continue;
        const double t = plan_time_us(bulk, bm, bn, K, num_cus) + plan_time_us(edge, em, en, K, num_cus);
        if (t < best_t) {
            best_t = t;
            bulk.workspace_bytes = edge.workspace_bytes;
            bulk.edge_dim = dim;
            bulk.edge_at = at;
            *p = bulk;
        }
    }
}

int make_plan(int M, int N, int K, int tile_cfg, int num_cus, wmma_gemm_plan* out) {
    return make_plan_within(M, N, K, tile_cfg, num_cus, SIZE_MAX, out);
}

int make_plan_within(int M, int N, int K, int tile_cfg, int num_cus, size_t max_ws,
                     wmma_gemm_plan* out) {
    if (!out || M < 0 || N < 0 || K < 0) return WMMA_ERR_INVALID_ARG;
    if (tile_cfg < WMMA_TILE_AUTO || tile_cfg >= WMMA_TILE_COUNT) return WMMA_ERR_INVALID_ARG;
    if (num_cus <= 0) num_cus = 256;
    wmma_gemm_plan p{};

    if (tile_cfg == WMMA_TILE_AUTO && num_cus == 256) {
        for (const TunedPlan& e : kTunedPlans)
            if (e.M == M && e.N == N && e.K == K &&
                make_custom_plan(M, N, K, e.kernel, e.tile_cfg, e.split, &p) == WMMA_OK &&
                p.workspace_bytes <= max_ws) {
                *out = p;
                return WMMA_OK;
            }
    }

    if (tile_cfg != WMMA_TILE_AUTO) {
        // Explicit tile (matmul_tiled): exactly that tile, no split.
        const TileShape& t = kTiles[tile_cfg];
        p.kernel = WMMA_KERNEL_TILED;
        p.tile_cfg = tile_cfg;
        p.tile_m = t.bm;
        p.tile_n = t.bn;
        int tiles = ceil_div(M, t.bm) * ceil_div(N, t.bn);
        finish_split(M, N, K, tiles, 1, &p);
        *out = p;
        return WMMA_OK;
    }

    if (M <= kSkinnyAutoMaxM && M > 0 && N > 0 && K > 1024) {
        // Streaming kernel (M <= 16 with K > 1024; the launch model takes shorter K, where
        // an unsplit 64x64 tile measured 10-30% faster): each workgroup owns
        // kSkinnyBlockN columns and one K range.
        // The launch lasts as long as the busiest CU, which streams ceil(W / CUs) of the
        // W = tiles x split workgroups, each 1/W of the bytes.  M <= 16: pick the split
        // that minimises ceil(W / CUs) / W over W <= 3 x CUs (measured on MI355X: a split
        // that leaves some CUs one workgroup more than the rest costs 10-25%, and beyond
        // three workgroups per CU the extra partial sums cost more than the balance gains),
        // the smaller split on a tie (fewer partial sums to write and reduce).
        p.kernel = WMMA_KERNEL_SKINNY;
        p.tile_cfg = -1;
        p.tile_m = 16;
        p.tile_n = kSkinnyBlockN;
        const int tiles = ceil_div(N, kSkinnyBlockN);
        const int smax = std::min(std::max(1, K / 256), kMaxSplitK);
        int split = 1;
        double best = 1e300;
        for (int sp = 1; sp <= smax; ++sp) {
            const int64_t w = (int64_t)tiles * sp;
            if (sp > 1 && w > 3 * (int64_t)num_cus) break;
            const double cost = (double)ceil_div64(w, num_cus) / (double)w;
            if (cost < best * 0.99) {
                best = cost;
                split = sp;
            }
        }
        finish_split(M, N, K, tiles, split, &p);
        fit_split(M, N, K, max_ws, &p);
        *out = p;
        return WMMA_OK;
    }

    if (M > 0 && N > 0 && K > 0 && M <= kModelMaxM) {
        *out = model_plan(M, N, K, num_cus, max_ws);
        return WMMA_OK;
    }

    // Tiled MFMA kernel: the tile with the shortest estimated time (plan_time_us: waves of
    // workgroups, one per CU, times the tile's wave time), the larger tile on a tie.
    const int order[] = {WMMA_TILE_256x256, WMMA_TILE_256x128, WMMA_TILE_128x128,
                         WMMA_TILE_256x64, WMMA_TILE_128x64, WMMA_TILE_64x64};
    int best = WMMA_TILE_64x64;
    double best_cost = 1e300;
    for (int cfg : order) {
        wmma_gemm_plan c{};
        if (make_custom_plan(std::max(M, 1), std::max(N, 1), std::max(K, 1), WMMA_KERNEL_TILED, cfg,
                             1, &c) != WMMA_OK)
            continue;
        const double cost = plan_time_us(c, std::max(M, 1), std::max(N, 1), std::max(K, 1), num_cus);
        if (cost < best_cost * 0.999) {
            best_cost = cost;
            best = cfg;
        }
    }
    const TileShape& t = kTiles[best];
    p.kernel = WMMA_KERNEL_TILED;
    p.tile_cfg = best;
    p.tile_m = t.bm;
    p.tile_n = t.bn;
    int tiles = ceil_div(M, t.bm) * ceil_div(N, t.bn);
    int split = 1;
    // Split K only when the chip is under-filled and the GEMM is big enough (>= 2^30
    // multiply-adds) for the extra reduction launch to pay for itself.
    if (tiles > 0 && tiles * 2 <= num_cus && K >= 512 &&
        (int64_t)M * N * K >= (int64_t(1) << 30)) {
        split = std::min({num_cus / tiles, K / 256, kMaxSplitK});
        split = std::max(split, 1);
    }
    finish_split(M, N, K, tiles, split, &p);
    fit_split(M, N, K, max_ws, &p);
    if (tile_cfg == WMMA_TILE_AUTO && p.split_k == 1) two_part(M, N, K, num_cus, max_ws, &p);
    *out = p;
    return WMMA_OK;
}

}  // namespace wmma_amd
