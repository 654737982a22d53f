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
    {128, 64, 2, 2},   // 1: wave tile 64x32
    {256, 64, 4, 1},   // 2: wave tile 64x64
    {128, 128, 2, 2},  // 3: wave tile 64x64
    {256, 128, 2, 2},  // 4: wave tile 128x64
    {256, 256, 2, 4},  // 5: wave tile 128x64 (8 waves, two per SIMD)
};

constexpr int kBlockK = 64;        // K depth of one LDS stage (fp16: 128-byte rows)
constexpr int kSkinnyMaxM = 16;    // M at or below this uses the streaming kernel
constexpr int kSkinnyBlockN = 128; // columns per skinny workgroup
constexpr int kMaxSplitK = 32;     // cap from the reference's split-K config (wmma_xor_swizzle.hpp:318)

inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int64_t ceil_div64(int64_t a, int64_t b) { return (a + b - 1) / b; }

// Relative per-CU throughput of each tile once the chip is full (larger tiles reuse
// more operand bytes per LDS byte).  Used only to rank candidate tiles.
constexpr double kTileEff[WMMA_TILE_COUNT] = {0.40, 0.55, 0.65, 0.75, 0.88, 1.0};

// Fill `out` for a GEMM of this shape; returns WMMA_OK or WMMA_ERR_INVALID_ARG.
int make_plan(int M, int N, int K, int tile_cfg, int num_cus, wmma_gemm_plan* out);

}  // namespace wmma_amd
