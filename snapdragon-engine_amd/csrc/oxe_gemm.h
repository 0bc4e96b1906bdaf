// The int8 matrix-core Q8_0 GEMM of prefill (k_gemm.hip), callable from the host side of the engine.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oxe {

// Token-row tiles: plain (tiles == null: tile y = token rows [64 y, 64 y + 64)) or grouped
// (tiles[y] = {group g, first output row, row count <= 64}: weights of group g at wq + g * wq_stride,
// activation row of output row p = xrow ? xrow[p] : p; tile_count (optional, device): tiles at or
// beyond *tile_count are empty). res (optional): y = chain + res[p][r].
struct GemmArgs {
    const int8_t *wq;
    const uint16_t *wd;
    const int8_t *xq;
    const uint16_t *xd;
    float *y;
    const float *res;
    int64_t nr, nt, k, ldy, ldr;
    const int4 *tiles;
    int64_t wq_stride, wd_stride;
    const int32_t *xrow;
    const int32_t *tile_count;
};

// rows of y: plain -> nt token rows; grouped -> the tiles' rows (ntiles tiles). 0, -1 (bad shape), -2.
int gemm_launch(const GemmArgs &a, int64_t ntiles, hipStream_t st);

}  // namespace oxe
