// Host-only GEMM planner.  Chooses the kernel family, tile and split-K partition.
//
// The reference picks a tile from gfx1151-tuned thresholds (select_optimal_tile,
// wmma_tile_selection.hpp:30-66) and has an unreachable split-K config
// (compute_config, wmma_xor_swizzle.hpp:293-332: target tiles = 4 x CUs, split capped at
// 32 and at K/256, k_per_split = ceil(K/split)).  Here the choice is made against a
// 256-CU device: fill the chip with whole waves of workgroups, prefer the tile that
// reuses the most bytes per LDS byte, and split K only when too few output tiles exist
// to occupy the CUs.  The result never depends on the plan beyond fp32 summation order.
#include "plan.hpp"

#include <algorithm>

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
static void two_part(int M, int N, int K, int num_cus, wmma_gemm_plan* p) {
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
            make_plan(em, en, K, WMMA_TILE_AUTO, num_cus, &edge) != WMMA_OK ||
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
    if (!out || M < 0 || N < 0 || K < 0) return WMMA_ERR_INVALID_ARG;
    if (tile_cfg < WMMA_TILE_AUTO || tile_cfg >= WMMA_TILE_COUNT) return WMMA_ERR_INVALID_ARG;
    if (num_cus <= 0) num_cus = 256;
    wmma_gemm_plan p{};

    if (tile_cfg == WMMA_TILE_AUTO && num_cus == 256) {
        for (const TunedPlan& e : kTunedPlans)
            if (e.M == M && e.N == N && e.K == K)
                return make_custom_plan(M, N, K, e.kernel, e.tile_cfg, e.split, out);
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

    if (M <= kSkinnyAutoMaxM && M > 0 && N > 0 && K > 0) {
        // Streaming kernel: each workgroup owns kSkinnyBlockN columns and one K range.
        // The launch lasts as long as the busiest CU, which streams ceil(W / CUs) of the
        // W = tiles x split workgroups, each 1/W of the bytes.  M <= 16: pick the split
        // that minimises ceil(W / CUs) / W over W <= 3 x CUs (measured on MI355X: a split
        // that leaves some CUs one workgroup more than the rest costs 10-25%, and beyond
        // three workgroups per CU the extra partial sums cost more than the balance gains),
        // the smaller split on a tie (fewer partial sums to write and reduce).  16 < M <= 32
        // (two 16-row blocks, twice the partial sums): the largest split that keeps W
        // within one wave of the CUs -- the fastest of splits 1-8 in every case measured
        // (M = 17, 32; N = 4096, 11008, 14336; K = 4096, 14336), e.g. M = 32, N = 11008:
        // split 2 25.9 us against 27.2-31.6 for 3-8, 27.1 for the tiled kernel.
        p.kernel = WMMA_KERNEL_SKINNY;
        p.tile_cfg = -1;
        p.tile_m = M <= 16 ? 16 : 32;
        p.tile_n = kSkinnyBlockN;
        const int tiles = ceil_div(N, kSkinnyBlockN);
        const int smax = std::min(std::max(1, K / 256), kMaxSplitK);
        int split = 1;
        if (M > 16) {
            split = (int)std::max<int64_t>(1, std::min<int64_t>(smax, num_cus / tiles));
        } else {
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
        }
        finish_split(M, N, K, tiles, split, &p);
        *out = p;
        return WMMA_OK;
    }

    if (M <= 128 && K >= 512) {
        // Few rows: the GEMM streams B, and the chip is filled by choosing the tile and the
        // K split together.  Estimated time = (workgroups on the busiest CU) x tile area /
        // (split x tile efficiency x the fraction of the tile's rows that exist), with 15%
        // per extra split for the partial sums.  Measured on MI355X at M = 64, 128 and
        // N = 4096..14336, K = 4096, 14336: this picks the fastest of the 64x64, 128x64 and
        // 128x128 tiles with splits 1, 2, 4 in every case (up to 22% over choosing the tile
        // first and splitting only an under-filled chip; with a 10% split term it chose
        // split 4 for M = 64, N = 11008, measured 17% slower than no split).
        const int cands[] = {WMMA_TILE_64x64, WMMA_TILE_128x64, WMMA_TILE_128x128};
        int best_cfg = WMMA_TILE_64x64, best_split = 1;
        double best_cost = 1e300;
        for (int cfg : cands) {
            const TileShape& t = kTiles[cfg];
            const int64_t tiles = (int64_t)ceil_div(M, t.bm) * ceil_div(N, t.bn);
            const double eff = kTileEff[cfg] * std::min(1.0, (double)M / t.bm);
            for (int sp : {1, 2, 4}) {
                // a split needs K >= 256 per part and K >= 2048 for the partial-sum pass
                // to pay for itself: measured on MI355X, every shape with K >= 2048 split
                // faster (48 x 1024 x 2048: 15.2 -> 11.2 us; 64 x 1024 x 4096: 25.5 ->
                // 12.7; 48 x 4096 x 4096: 26.8 -> 15.0), every one with K <= 1024 slower
                // (64 x 1024 x 1024: 9.4 -> 11.7; 128 x 4096 x 512: 7.9 -> 11.0)
                if (sp > 1 && (K / sp < 256 || K < 2048)) break;
                const int64_t w = tiles * sp;
                const double cost = (double)ceil_div64(w, num_cus) * t.bm * t.bn / (sp * eff) *
                                    (1.0 + 0.15 * (sp - 1));
                if (cost < best_cost * 0.999) {
                    best_cost = cost;
                    best_cfg = cfg;
                    best_split = sp;
                }
            }
        }
        const TileShape& t = kTiles[best_cfg];
        p.kernel = WMMA_KERNEL_TILED;
        p.tile_cfg = best_cfg;
        p.tile_m = t.bm;
        p.tile_n = t.bn;
        finish_split(M, N, K, ceil_div(M, t.bm) * ceil_div(N, t.bn), best_split, &p);
        *out = p;
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
    if (tile_cfg == WMMA_TILE_AUTO && split == 1) two_part(M, N, K, num_cus, &p);
    *out = p;
    return WMMA_OK;
}

}  // namespace wmma_amd
