// Host-only GEMM planning: tile table, tile choice, split-K partition and workspace size.
// Pure C++ (no HIP), so the dispatch math is testable on a machine without a GPU.
#pragma once

#include <cstddef>
#include <cstdint>

#include "../../include/wmma_ops_amd.h"

namespace wmma_amd {

// One row of the tile menu: workgroup output tile and its wave grid.
struct TileShape {
    int bm, bn;    // workgroup tile
    int wm, wn;    // waves along M and N (wm*wn*64 threads)
};

// Tile menu indexed by WMMA_TILE_*.  Rows 0..3 keep the reference's matmul_tiled block
// shapes (wmma_gemm.hip:1500-1520); 4 and 5 are the CDNA4 large tiles.
constexpr TileShape kTiles[WMMA_TILE_COUNT] = {
    {64, 64, 2, 2},    // 0: wave tile 32x32
    {128, 64, 4, 2},   // 1: wave tile 32x32 (8 waves; 5-9% faster than 4 waves of 64x32)
    {256, 64, 4, 1},   // 2: wave tile 64x64
    {128, 128, 2, 2},  // 3: wave tile 64x64
    {256, 128, 2, 2},  // 4: wave tile 128x64
    {256, 256, 2, 4},  // 5: wave tile 128x64 (8 waves, two per SIMD)
};

constexpr int kBlockK = 64;        // K depth of one LDS stage (fp16: 128-byte rows)
constexpr int kSkinnyAutoMaxM = 16; // M at or below this (K > 1024): the streaming kernel's own rule
constexpr int kModelMaxM = 768;     // M at or below this: the measured launch model picks the plan
constexpr int kSkinnyMaxMWide = 64; // the streaming kernel's limit (four 16-row blocks)
constexpr int kSkinnyBlockN = 128; // columns per skinny workgroup
constexpr int kMaxSplitK = 32;     // cap from the reference's split-K config (wmma_xor_swizzle.hpp:318)

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Launch model for M <= kModelMaxM, fitted on MI355X (256 CUs) to the autotuner's timings
// of every plan (6 tiles x splits 1-16, the streaming kernel with splits 1-32) at 819
// shapes, M = 1-768, N = 512-14336, K = 512-14336.  A workgroup streams its operand bytes
// (the rows of A that exist plus the tile's columns of B, over its K range) at a per-CU
// rate, or is held by its MFMA work, whichever is longer, plus a fixed cost; the launch
// takes as many such times as it has waves of workgroups (one per CU), at least the HBM
// time of its operands, plus, with a K split, a fixed cost and the partial sums' bytes.
struct TileRate {
    double kb_per_us;     // operand bytes a workgroup streams per microsecond (KB)
    double mflop_per_us;  // its MFMA rate (MFLOP per microsecond, full tile rows)
};
constexpr TileRate kTileRate[WMMA_TILE_COUNT] = {
    {40, 2}, {40, 4}, {10, 4}, {40, 4}, {30, 3}, {35, 5}};
constexpr double kWgFixedUs = 2.0;         // per workgroup: prologue, epilogue
constexpr double kSkinnyKbPerUs = 50;      // the streaming kernel's per-workgroup rate
constexpr double kSkinnyWgFixedUs = 3.0;
constexpr double kSplitFixedUs = 2.0;      // a K split: the reduction launch
constexpr double kPartialUsPerMB = 0.5;    // and (split + 1) x M x N x 4 bytes of partial sums
constexpr double kModelHbmMBPerUs = 8.0;   // operand bytes per microsecond at most

// Modelled duration (microseconds) of a one-launch plan for M <= kModelMaxM.
double model_time_us(const wmma_gemm_plan& p, int M, int N, int K, int num_cus);

// Time model of the tiled kernel on full waves of workgroups (one workgroup per CU),
// fitted on MI355X to full-wave launches of every tile (4096^3, 8192 x 8192 x 4096,
// 4096 x 4096 x 1024, 4096 x 14336 x 4096, 8192 x 4096 x 8192; random fp16 operands):
// one wave of 256x256 tiles takes kEpiUs256 + kWaveUsPerK256 * K microseconds (the
// first term is the fp32 tile written out), and a wave of another tile the same scaled
// by its area / 65536, with the K term divided by the tile's measured efficiency.
constexpr double kWaveEff[WMMA_TILE_COUNT] = {0.45, 0.57, 0.55, 0.72, 0.81, 1.0};
constexpr double kEpiUs256 = 13.2;
constexpr double kWaveUsPerK256 = 0.0279;
constexpr double kHbmBytesPerUs = 5.0e6;  // sustained HBM rate of the streaming kernels
constexpr double kLaunchUs = 2.0;         // a launch behind another on the same stream
constexpr double kReduceUs = 3.0;         // the split-K reduction's launch

// Estimated duration (microseconds) of one launch of plan p on an M x N x K GEMM:
// waves x wave time for the tiled kernel (at least the HBM time of its operands), the
// operands' HBM time for the skinny kernel, plus the split-K reduction when there is one.
double plan_time_us(const wmma_gemm_plan& p, int M, int N, int K, int num_cus);

// A two-part plan is taken when its estimate is below this fraction of the best
// one-launch plan's (the estimates are within ~15% of measured times).
constexpr double kEdgeGain = 0.93;

// Fill `out` for a GEMM of this shape; returns WMMA_OK or WMMA_ERR_INVALID_ARG.  With
// tile_cfg == WMMA_TILE_AUTO on a 256-CU device, a shape found in the autotuned table
// (tuned_table.inc) takes the measured plan; every other shape the heuristics in
// plan.cpp, which may split it into a bulk and an edge GEMM (out->edge_dim).
int make_plan(int M, int N, int K, int tile_cfg, int num_cus, wmma_gemm_plan* out);

// make_plan among the plans whose split-K partial sums fit max_ws bytes: a tuned-table
// entry or a split that needs more is passed over for the next choice (a plan without a
// split needs none, so there always is one).
int make_plan_within(int M, int N, int K, int tile_cfg, int num_cus, size_t max_ws,
                     wmma_gemm_plan* out);

// A plan with an explicit kernel (WMMA_KERNEL_*), tile (WMMA_TILE_*; ignored by the skinny
// kernel) and K split, completed as the planner completes its own (k_per_split a whole
// number of 64-deep stages, no empty split).  WMMA_ERR_INVALID_ARG for a combination the
// kernels cannot run.
int make_custom_plan(int M, int N, int K, int kernel, int tile_cfg, int split,
                     wmma_gemm_plan* out);

// One entry of the autotuned dispatch table: the fastest measured plan for one shape.
struct TunedPlan {
    int M, N, K;
    int kernel, tile_cfg, split;
};
// The table (generated by wmma_ops_amd/autotune.py) and its length.
const TunedPlan* tuned_plans(int* count);

}  // namespace wmma_amd
