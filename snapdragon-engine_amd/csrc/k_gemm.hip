// Batched Q8_0 GEMM for prefill: y[t][r] = W[r] . x[t] for T tokens, the reference's
// ggml_gemm_q8_0_4x8_q8_0 (vendor/ggml-subset/generated/repack_subset.cpp:3804-3954), whose
// per (row, token) result equals the Q8_0 GEMV's bit for bit (docs/lab-notes/M3-PREFILL.md:70-71):
// for each 32-element block b in order, acc = fma(f32(isum_b), d_x[t][b] * d_w[r][b], acc) from +0,
// isum_b the exact int32 dot of the block's codes.
//
// The int32 block dots are int8 matrix-core products (v_mfma_i32_16x16x32_i8: one 16 x 16 tile of
// block dots per instruction, exact in any order); the fp32 chain runs in registers, one value per
// (row, token) per lane, block by block in order, so the chain is the reference's.
//
// Workgroup tile: 64 weight rows x 64 tokens, 4 waves of 32 x 32 (2 x 2 MFMA tiles). The K
// dimension is staged through LDS 8 blocks (256 bytes per row) at a time with 16-byte coalesced
// loads, the next stage's held in registers while the current one computes; LDS rows are padded to
// 272 bytes so a wave's 8-byte fragment reads fall on distinct banks.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/oxe_amd.h"
#include "oxe_common.h"
#include "oxe_gemm.h"

namespace oxe {

namespace gm {
constexpr int BM = 64, BN = 64;        // rows, tokens per workgroup
constexpr int KC = 256;                // K bytes (8 blocks) per LDS stage
constexpr int NBC = KC / 32;           // blocks per stage
constexpr int LDR = KC + 16;           // LDS row stride (bytes)
constexpr int NT = 256;                // threads
}  // namespace gm

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(gm::NT) void gemm_q8_kernel(GemmArgs a) {
    using namespace gm;
    __shared__ __align__(16) int8_t sw[BM * LDR];
    __shared__ __align__(16) int8_t sx[BN * LDR];
    __shared__ __align__(16) float sdw[NBC][BM + 4];   // scales transposed: a lane's 4 rows are one 16-byte read
    __shared__ float sdx[NBC][BN + 4];
    __shared__ int64_t sxr[BN];                          // activation row of each of the tile's output rows
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
    __syncthreads();
    // wave w: rows 32 (w & 1) .., tokens 32 (w >> 1) ..; MFMA tile (i, j) at +16 i, +16 j
    const int wr = 32 * (w & 1), wt = 32 * (w >> 1);
    const int fr = lane & 15, fk = 8 * (lane >> 4);   // fragment row / token and its 8 k bytes
    const int64_t wrem = pn - wt;   // tokens of the tile in this wave's column range and beyond
    const int nj = wrem > 16 ? 2 : (wrem > 0 ? 1 : 0);
    float acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[i][j][v] = 0.0f;
    // the next stage's codes and scales are loaded into registers while the current stage computes
    constexpr int NP = BM * KC / 16 / NT;   // 16-byte code chunks per thread and matrix
    uint4 pu[NP], pv[NP];
    float pdw[BM * NBC / NT], pdx[BM * NBC / NT];
    auto fetch = [&](int64_t kc) {
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int i = t + NT * p, row = i / (KC / 16), ch = i % (KC / 16);
            const int64_t gr = r0 + row, xr = sxr[row];
            pu[p] = gr < nr ? *(const uint4 *)(wq + gr * k + kc + 16 * ch) : make_uint4(0, 0, 0, 0);
            pv[p] = xr >= 0 ? *(const uint4 *)(a.xq + xr * k + kc + 16 * ch) : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int p = 0; p < BM * NBC / NT; p++) {
            const int i = t + NT * p, row = i / NBC, bb = i % NBC;
            const int64_t gr = r0 + row, xr = sxr[row];
            pdw[p] = gr < nr ? h2f(wd[gr * nb + kc / 32 + bb]) : 0.0f;
            pdx[p] = xr >= 0 ? h2f(a.xd[xr * nb + kc / 32 + bb]) : 0.0f;
        }
    };
    fetch(0);
    for (int64_t kc = 0; kc < k; kc += KC) {
        // stage codes (64 rows x 256 bytes of W and X) and scales (as f32) from the registers
#pragma unroll
        for (int p = 0; p < NP; p++) {
            const int i = t + NT * p, row = i / (KC / 16), ch = i % (KC / 16);
            *(uint4 *)(sw + row * LDR + 16 * ch) = pu[p];
            *(uint4 *)(sx + row * LDR + 16 * ch) = pv[p];
        }
#pragma unroll
        for (int p = 0; p < BM * NBC / NT; p++) {
            const int i = t + NT * p, row = i / NBC, bb = i % NBC;
            sdw[bb][row] = pdw[p];
            sdx[bb][row] = pdx[p];
        }
        __syncthreads();
        if (kc + KC < k) fetch(kc + KC);
        // the wave's 16-token sub-tiles that hold tokens (a per-expert group fills a tile partly):
        // empty ones are skipped, wave-uniformly
        auto blocks = [&](auto njc) {
            constexpr int NJ = decltype(njc)::value;
#pragma unroll
            for (int bb = 0; bb < NBC; bb++) {
                long fa[2], fb[NJ];
#pragma unroll
                for (int i = 0; i < 2; i++) fa[i] = *(const long *)(sw + (wr + 16 * i + fr) * LDR + 32 * bb + fk);
#pragma unroll
                for (int j = 0; j < NJ; j++) fb[j] = *(const long *)(sx + (wt + 16 * j + fr) * LDR + 32 * bb + fk);
                // this lane's outputs: rows wr + 16 i + 4 (lane >> 4) + v, token wt + 16 j + (lane & 15)
                float dxs[NJ], dws[2][4];
#pragma unroll
                for (int j = 0; j < NJ; j++) dxs[j] = sdx[bb][wt + 16 * j + fr];
#pragma unroll
                for (int i = 0; i < 2; i++) {
                    const float4 d4 = *(const float4 *)&sdw[bb][wr + 16 * i + 4 * (lane >> 4)];
                    dws[i][0] = d4.x; dws[i][1] = d4.y; dws[i][2] = d4.z; dws[i][3] = d4.w;
                }
#pragma unroll
                for (int i = 0; i < 2; i++)
#pragma unroll
                    for (int j = 0; j < NJ; j++) {
                        const i32x4 zero = {0, 0, 0, 0};
                        const i32x4 s = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa[i], fb[j], zero, 0, 0, 0);
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            acc[i][j][v] = __builtin_fmaf((float)s[v], dxs[j] * dws[i][v], acc[i][j][v]);
                    }
            }
        };
        if (nj == 2) blocks(std::integral_constant<int, 2>{});
        else if (nj == 1) blocks(std::integral_constant<int, 1>{});
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int64_t gr = r0 + wr + 16 * i + 4 * (lane >> 4) + v;
                const int tt = wt + 16 * j + (lane & 15);
                if (gr < nr && tt < pn) {
                    const int64_t p = p0 + tt;
                    a.y[p * a.ldy + gr] = a.res ? acc[i][j][v] + a.res[p * a.ldr + gr] : acc[i][j][v];
                }
            }
}

int gemm_launch(const GemmArgs &a, int64_t ntiles, hipStream_t st) {
    using namespace gm;
    if (a.k <= 0 || a.k % KC != 0 || a.nr <= 0 || a.ldy < a.nr) return -1;
    if (!a.wq || !a.wd || !a.xq || !a.xd || !a.y) return -1;
    const int64_t ny = a.tiles ? ntiles : (a.nt + BN - 1) / BN;
    if (ny <= 0) return 0;
    hipLaunchKernelGGL(gemm_q8_kernel, dim3((unsigned)((a.nr + BM - 1) / BM), (unsigned)ny), dim3(NT), 0, st, a);
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
