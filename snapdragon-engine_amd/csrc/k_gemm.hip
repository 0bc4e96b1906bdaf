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
// loads; LDS rows are padded to 272 bytes so a wave's 8-byte fragment reads fall on distinct banks.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/oxe_amd.h"
#include "oxe_common.h"

namespace oxe {

namespace gm {
constexpr int BM = 64, BN = 64;        // rows, tokens per workgroup
constexpr int KC = 256;                // K bytes (8 blocks) per LDS stage
constexpr int NBC = KC / 32;           // blocks per stage
constexpr int LDR = KC + 16;           // LDS row stride (bytes)
constexpr int NT = 256;                // threads
}  // namespace gm

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(gm::NT) void gemm_q8_kernel(const int8_t *__restrict__ wq, const uint16_t *__restrict__ wd,
                                                         const int8_t *__restrict__ xq, const uint16_t *__restrict__ xd,
                                                         float *__restrict__ y, int64_t nr, int64_t nt, int64_t k,
                                                         int64_t ldy) {
    using namespace gm;
    __shared__ __align__(16) int8_t sw[BM * LDR];
    __shared__ __align__(16) int8_t sx[BN * LDR];
    __shared__ __align__(16) float sdw[NBC][BM + 4];   // scales transposed: a lane's 4 rows are one 16-byte read
    __shared__ float sdx[NBC][BN + 4];
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int64_t r0 = (int64_t)blockIdx.x * BM, t0 = (int64_t)blockIdx.y * BN;
    const int64_t nb = k / 32;
    // wave w: rows 32 (w & 1) .., tokens 32 (w >> 1) ..; MFMA tile (i, j) at +16 i, +16 j
    const int wr = 32 * (w & 1), wt = 32 * (w >> 1);
    const int fr = lane & 15, fk = 8 * (lane >> 4);   // fragment row / token and its 8 k bytes
    float acc[2][2][4];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) acc[i][j][v] = 0.0f;
    for (int64_t kc = 0; kc < k; kc += KC) {
        // stage codes: 64 rows x 256 bytes each for W and X, 16 bytes per thread and pass
#pragma unroll
        for (int p = 0; p < BM * KC / 16 / NT; p++) {
            const int i = t + NT * p, row = i / (KC / 16), ch = i % (KC / 16);
            const int64_t gr = r0 + row, gt = t0 + row;
            const uint4 a = gr < nr ? *(const uint4 *)(wq + gr * k + kc + 16 * ch) : make_uint4(0, 0, 0, 0);
            const uint4 b = gt < nt ? *(const uint4 *)(xq + gt * k + kc + 16 * ch) : make_uint4(0, 0, 0, 0);
            *(uint4 *)(sw + row * LDR + 16 * ch) = a;
            *(uint4 *)(sx + row * LDR + 16 * ch) = b;
        }
        // stage scales as f32: 64 rows x 8 blocks for W and X
        for (int i = t; i < BM * NBC; i += NT) {
            const int row = i / NBC, bb = i % NBC;
            const int64_t gr = r0 + row, gt = t0 + row;
            sdw[bb][row] = gr < nr ? h2f(wd[gr * nb + kc / 32 + bb]) : 0.0f;
            sdx[bb][row] = gt < nt ? h2f(xd[gt * nb + kc / 32 + bb]) : 0.0f;
        }
        __syncthreads();
#pragma unroll
        for (int bb = 0; bb < NBC; bb++) {
            long fa[2], fb[2];
#pragma unroll
            for (int i = 0; i < 2; i++) fa[i] = *(const long *)(sw + (wr + 16 * i + fr) * LDR + 32 * bb + fk);
#pragma unroll
            for (int j = 0; j < 2; j++) fb[j] = *(const long *)(sx + (wt + 16 * j + fr) * LDR + 32 * bb + fk);
            // this lane's outputs: rows wr + 16 i + 4 (lane >> 4) + v, token wt + 16 j + (lane & 15)
            float dxs[2], dws[2][4];
#pragma unroll
            for (int j = 0; j < 2; j++) dxs[j] = sdx[bb][wt + 16 * j + fr];
#pragma unroll
            for (int i = 0; i < 2; i++) {
                const float4 d4 = *(const float4 *)&sdw[bb][wr + 16 * i + 4 * (lane >> 4)];
                dws[i][0] = d4.x; dws[i][1] = d4.y; dws[i][2] = d4.z; dws[i][3] = d4.w;
            }
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const i32x4 zero = {0, 0, 0, 0};
                    const i32x4 s = __builtin_amdgcn_mfma_i32_16x16x32_i8(fa[i], fb[j], zero, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; v++) acc[i][j][v] = __builtin_fmaf((float)s[v], dxs[j] * dws[i][v], acc[i][j][v]);
                }
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int64_t gr = r0 + wr + 16 * i + 4 * (lane >> 4) + v, gt = t0 + wt + 16 * j + (lane & 15);
                if (gr < nr && gt < nt) y[gt * ldy + gr] = acc[i][j][v];
            }
}

}  // namespace oxe

extern "C" {

int oxe_hip_gemm_q8_0(int64_t k, int64_t nr, int64_t nt, const int8_t *wq, const uint16_t *wd, const int8_t *xq,
                      const uint16_t *xd, float *y, int64_t ldy, void *stream) {
    using namespace oxe::gm;
    if (k <= 0 || k % KC != 0 || nr <= 0 || nt <= 0 || ldy < nr) return -1;
    if (!wq || !wd || !xq || !xd || !y) return -1;
    const dim3 grid((unsigned)((nr + BM - 1) / BM), (unsigned)((nt + BN - 1) / BN));
    hipLaunchKernelGGL(oxe::gemm_q8_kernel, grid, dim3(NT), 0, (hipStream_t)stream, wq, wd, xq, xd, y, nr, nt, k, ldy);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
