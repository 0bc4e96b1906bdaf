// Batched Q8_0 GEMM for prefill: y[t][r] = W[r] . x[t] for T tokens, the reference's
// ggml_gemm_q8_0_4x8_q8_0 (vendor/ggml-subset/generated/repack_subset.cpp:3804-3954), whose
// per (row, token) result equals the Q8_0 GEMV's bit for bit (docs/lab-notes/M3-PREFILL.md:70-71):
// for each 32-element block b in order, acc = fma(f32(isum_b), d_x[t][b] * d_w[r][b], acc) from +0,
// isum_b the exact int32 dot of the block's codes.
//
// The int32 block dots are int8 matrix-core products (v_mfma_i32_32x32x32_i8: a 32 x 32 tile of one
// block's dots per instruction, exact in any order; any split of the block's 32 codes over the
// lanes gives the same sums as long as weights and activations use the same split). The scale
// products d_x[t][b] * d_w[r][b] of the same tile are a rank-1 fp32 matrix-core product
// (v_mfma_f32_32x32x2_f32 with the second k column zero: one product and an exact zero added, so
// each element is the correctly rounded fp32 product, the value a VALU multiply gives), in the same
// 32 x 32 output layout as the dots. What is left for the VALU is the chain itself, two operations
// per output and block (convert the block sum, fused multiply-add), one value per (row, token) per
// lane, block by block in order, so the chain is the reference's. The VALU is the kernel's bound;
// each wave issues a tile's matrix-core products for the next block as soon as the tile's chain of
// the current block has read them, so they run under the other tile's chain.
//
// Workgroup tile: 128 weight rows x 64 tokens, 4 waves of 32 rows x 64 tokens (two 32 x 32 tiles).
// The K dimension is staged through LDS 8 blocks (256 bytes per row) at a time with 16-byte
// coalesced loads, the next stage's held in registers while the current one computes; LDS rows are
// padded to 272 bytes so the 16-byte fragment reads of 8 consecutive rows fall on distinct banks.
// Scales are staged as f32 by one thread per row (8 blocks from one 16-byte load), so each LDS
// store instruction writes 64 consecutive words.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/oxe_amd.h"
#include "oxe_common.h"
#include "oxe_gemm.h"

namespace oxe {

namespace gm {
constexpr int BM = 128, BN = 64;       // rows, tokens per workgroup
constexpr int KC = 256;                // K bytes (8 blocks) per LDS stage
constexpr int NBC = KC / 32;           // blocks per stage
constexpr int LDR = KC + 16;           // LDS row stride (bytes)
constexpr int NT = 256;                // threads
constexpr int WR = 32;                 // weight rows per wave
constexpr int SDW = BM + 32;           // weight-scale row of one block: BM scales, then 32 zeros
}  // namespace gm

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(gm::NT, 2) void gemm_q8_kernel(GemmArgs a, int vec4) {
    using namespace gm;
    __shared__ __align__(16) int8_t sw[BM * LDR];
    __shared__ __align__(16) int8_t sx[BN * LDR];
    __shared__ __align__(16) float sdw[NBC][SDW];   // [block][row] weight scales as f32; [.][BM ..] stay 0
    __shared__ __align__(16) float sdx[NBC][BN];    // [block][token] activation scales as f32
    __shared__ int64_t sxr[BN];                     // activation row of each of the tile's output rows
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int64_t k = a.k, nr = a.nr, nb = k / 32;
    const int64_t r0 = (int64_t)blockIdx.x * BM;
    int64_t p0, pn;
    const int8_t *wq = a.wq;
    const uint16_t *wd = a.wd;
    if (a.tiles) {
        if (a.tile_count && (int)blockIdx.y >= *a.tile_count) return;   // uniform: before any barrier
        const int4 tl = a.tiles[blockIdx.y];
        wq += (int64_t)tl.x * a.wq_stride;
        wd += (int64_t)tl.x * a.wd_stride;
        p0 = tl.y;
        pn = tl.z;
    } else {
        p0 = (int64_t)blockIdx.y * BN;
        pn = a.nt - p0 < BN ? a.nt - p0 : BN;
    }
    if (t < BN) sxr[t] = t < pn ? (a.xrow ? (int64_t)a.xrow[p0 + t] : p0 + t) : -1;
    for (int i = t; i < NBC * 32; i += NT) sdw[i / 32][BM + i % 32] = 0.0f;
    __syncthreads();
    // wave w: rows 32 w .. 32 w + 31 of the tile; tile j: tokens 32 j .. 32 j + 31
    const int wr = WR * w, fr = lane & 31, fh = lane >> 5;
    float acc[2][16];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;
    // the next stage's codes and scales are loaded into registers while the current stage computes:
    // thread t stages 16-byte chunk t % 16 of rows t / 16 + 16 p; threads 0-127 the scales of weight
    // row t, threads 128-191 those of token row t - 128 (wave-uniform roles)
    constexpr int NPW = BM * KC / 16 / NT, NPX = BN * KC / 16 / NT;   // 16-byte chunks per thread
    const int crow = t / (KC / 16), cch = t % (KC / 16);
    const int64_t wrows = nr - r0;   // rows of W left from the tile's first
    const int8_t *wqt = wq + (r0 + crow) * k + 16 * cch;
    const int srow = t < BM ? t : t - BM;
    uint4 pu[NPW], pv[NPX], ps;
    auto fetch = [&](int64_t kc) {
#pragma unroll
        for (int p = 0; p < NPW; p++)
            pu[p] = crow + 16 * p < wrows ? *(const uint4 *)(wqt + (int64_t)(16 * p) * k + kc) : make_uint4(0, 0, 0, 0);
#pragma unroll
        for (int p = 0; p < NPX; p++) {
            const int64_t xr = sxr[crow + 16 * p];
            pv[p] = xr >= 0 ? *(const uint4 *)(a.xq + xr * k + 16 * cch + kc) : make_uint4(0, 0, 0, 0);
        }
        ps = make_uint4(0, 0, 0, 0);
        if (t < BM) {
            if (t < wrows) ps = *(const uint4 *)(wd + (r0 + t) * nb + kc / 32);
        } else if (t < BM + BN) {
            const int64_t xr = sxr[srow];
            if (xr >= 0) ps = *(const uint4 *)(a.xd + xr * nb + kc / 32);
        }
    };
    fetch(0);
    // tokens of the tile: a per-expert group fills a tile partly; an empty second tile is skipped
    // (uniform across the workgroup)
    auto run = [&](auto njc) {
        constexpr int NJ = decltype(njc)::value;
        for (int64_t kc = 0; kc < k; kc += KC) {
#pragma unroll
            for (int p = 0; p < NPW; p++) *(uint4 *)(sw + (crow + 16 * p) * LDR + 16 * cch) = pu[p];
#pragma unroll
            for (int p = 0; p < NPX; p++) *(uint4 *)(sx + (crow + 16 * p) * LDR + 16 * cch) = pv[p];
            if (t < BM + BN) {
                const uint32_t h[4] = {ps.x, ps.y, ps.z, ps.w};
                float *dst = t < BM ? &sdw[0][srow] : &sdx[0][srow];
                const int st = t < BM ? SDW : BN;
#pragma unroll
                for (int bb = 0; bb < NBC; bb++) dst[bb * st] = h2f((uint16_t)(h[bb / 2] >> (16 * (bb % 2))));
            }
            __syncthreads();
            if (kc + KC < k) fetch(kc + KC);
            // fragments: row / token lane & 31, codes 16 (lane >> 5) .. + 15 of the block; scale
            // operands: lanes 0-31 the row's / token's scale (k column 0), lanes 32-63 a zero weight
            // scale (k column 1)
            const int8_t *fa_p = sw + (wr + fr) * LDR + 16 * fh;
            const int8_t *fb_p = sx + fr * LDR + 16 * fh;
            const float *sa_p = &sdw[0][fh ? BM + fr : wr + fr];
            const float *sb_p = &sdx[0][fr];
            auto dots = [&](int bb, int j) {
                const i32x4 fa = *(const i32x4 *)(fa_p + 32 * bb);
                const i32x4 fb = *(const i32x4 *)(fb_p + 32 * LDR * j + 32 * bb);
                const i32x16 zero = {};
                return __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, zero, 0, 0, 0);
            };
            auto scales = [&](int bb, int j) {
                const f32x16 zero = {};
                return __builtin_amdgcn_mfma_f32_32x32x2f32(sa_p[bb * SDW], sb_p[bb * BN + 32 * j], zero, 0, 0, 0);
            };
            i32x16 s[NJ];
            f32x16 d[NJ];
#pragma unroll
            for (int j = 0; j < NJ; j++) {
                s[j] = dots(0, j);
                d[j] = scales(0, j);
            }
#pragma unroll
            for (int bb = 0; bb < NBC; bb++) {
                // tile j's outputs in this lane: rows wr + 8 q + 4 (lane >> 5) + e (v = 4 q + e), token 32 j + (lane & 31)
#pragma unroll
                for (int j = 0; j < NJ; j++) {
#pragma unroll
                    for (int v = 0; v < 16; v++) acc[j][v] = __builtin_fmaf((float)s[j][v], d[j][v], acc[j][v]);
                    if (bb + 1 < NBC) {
                        s[j] = dots(bb + 1, j);
                        d[j] = scales(bb + 1, j);
                    }
                }
            }
            __syncthreads();
        }
    };
    if (pn > 32) run(std::integral_constant<int, 2>{});
    else if (pn > 0) run(std::integral_constant<int, 1>{});
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int tt = 32 * j + fr;
        if (tt >= pn) continue;
        const int64_t p = p0 + tt;
        float *yp = a.y + p * a.ldy;
        const float *rp = a.res ? a.res + p * a.ldr : nullptr;
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int64_t gr = r0 + wr + 8 * q + 4 * fh;
            float o[4] = {acc[j][4 * q], acc[j][4 * q + 1], acc[j][4 * q + 2], acc[j][4 * q + 3]};
            if (vec4 && gr + 3 < nr) {
                if (rp) {
                    const float4 r4 = *(const float4 *)(rp + gr);
                    o[0] += r4.x; o[1] += r4.y; o[2] += r4.z; o[3] += r4.w;
                }
                *(float4 *)(yp + gr) = make_float4(o[0], o[1], o[2], o[3]);
            } else {
#pragma unroll
                for (int e = 0; e < 4; e++)
                    if (gr + e < nr) yp[gr + e] = rp ? o[e] + rp[gr + e] : o[e];
            }
        }
    }
}

int gemm_launch(const GemmArgs &a, int64_t ntiles, hipStream_t st) {
    using namespace gm;
    if (a.k <= 0 || a.k % KC != 0 || a.nr <= 0 || a.ldy < a.nr) return -1;
    if (!a.wq || !a.wd || !a.xq || !a.xd || !a.y) return -1;
    // 16-byte loads of codes and of 8 scales at a time
    if (((uintptr_t)a.wq | (uintptr_t)a.wd | (uintptr_t)a.xq | (uintptr_t)a.xd) % 16 != 0) return -1;
    const int64_t ny = a.tiles ? ntiles : (a.nt + BN - 1) / BN;
    if (ny <= 0) return 0;
    // 16-byte output (and residual) accesses where every row group of 4 starts 16-byte aligned
    const int vec4 = a.ldy % 4 == 0 && (uintptr_t)a.y % 16 == 0 && (!a.res || (a.ldr % 4 == 0 && (uintptr_t)a.res % 16 == 0));
    hipLaunchKernelGGL(gemm_q8_kernel, dim3((unsigned)((a.nr + BM - 1) / BM), (unsigned)ny), dim3(NT), 0, st, a, vec4);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace oxe

extern "C" {

int oxe_hip_gemm_q8_0(int64_t k, int64_t nr, int64_t nt, const int8_t *wq, const uint16_t *wd, const int8_t *xq,
                      const uint16_t *xd, float *y, int64_t ldy, void *stream) {
    if (nt <= 0) return -1;
    oxe::GemmArgs a{wq, wd, xq, xd, y, nullptr, nr, nt, k, ldy, 0, nullptr, 0, 0, nullptr};
    return oxe::gemm_launch(a, 0, (hipStream_t)stream);
}

}  // extern "C"
