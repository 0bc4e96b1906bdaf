// Batched Q8_0 GEMM for prefill: y[t][r] = W[r] . x[t] for T tokens, the reference's
// ggml_gemm_q8_0_4x8_q8_0 (vendor/ggml-subset/generated/repack_subset.cpp:3804-3954), whose
// per (row, token) result equals the Q8_0 GEMV's bit for bit (docs/lab-notes/M3-PREFILL.md:70-71):
// for each 32-element block b in order, acc = fma(f32(isum_b), d_x[t][b] * d_w[r][b], acc) from +0,
// isum_b the exact int32 dot of the block's codes.
//
// The int32 block dots are int8 matrix-core products (v_mfma_i32_32x32x32_i8: a 32 x 32 tile of one
// block's dots per instruction, exact in any order; any split of the block's 32 codes over the
// lanes gives the same sums as long as weights and activations use the same split). The scale
// products d_x[t][b] * d_w[r][b] of both 32-token tiles of a block are one two-block fp32 matrix-core
// outer product (v_mfma_f32_32x32x1_2b_f32: one product per element and nothing added, so each
// element is the correctly rounded fp32 product, the value a VALU multiply gives), in the same
// 32 x 32 output layout as the dots. What is left for the VALU is the chain itself, two operations
// per output and block (convert the block sum, fused multiply-add), one value per (row, token) per
// lane, block by block in order, so the chain is the reference's. The VALU is the kernel's bound.
//
// Workgroup tile: 128 weight rows x 64 tokens, 4 waves of 32 rows x 64 tokens (two 32 x 32 tiles).
// K is staged 4 blocks (128 bytes per row) at a time, double-buffered in LDS and filled by
// direct global-to-LDS loads (global_load_lds_dwordx4 / _dword: no staging registers), so three
// workgroups fit a CU. Code rows (128 bytes) are stored unpadded with their 16-byte chunks
// XOR-swizzled by f(r) = (r & 7) ^ ((r >> 3) & 1): the 16-byte fragment reads of 8 consecutive rows
// cover 8 distinct chunk slots of 128 bytes, and those of 16 consecutive rows 16 distinct 16-byte
// slots of 256 bytes, so neither a 32-bank nor a 64-bank LDS sees a conflict.
// Scales are staged as the raw f16 (4 per row and stage) and converted when read.
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <type_traits>

#include "../../include/oxe_amd.h"
#include "oxe_common.h"
#include "oxe_gemm.h"

namespace oxe {

namespace gm {
constexpr int BM = 128, BN = 64;       // rows, tokens per workgroup
constexpr int KC = 128;                // K bytes (4 blocks) per stage
constexpr int NBC = KC / 32;           // blocks per stage
constexpr int NT = 256;                // threads
constexpr int WR = 32;                 // weight rows per wave
}  // namespace gm

// one stage of LDS: codes [row][KC] with chunk c of row r at slot c ^ f(r); scales [row][NBC] f16
struct GemmStage {
    int8_t w[gm::BM * gm::KC];
    int8_t x[gm::BN * gm::KC];
    uint16_t dw[gm::BM * gm::NBC];
    uint16_t dx[gm::BN * gm::NBC];
};

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x32 __attribute__((ext_vector_type(32)));
typedef __attribute__((address_space(3))) void lds_void;
typedef __attribute__((address_space(1))) void glb_void;

// global -> LDS, 16 or 4 bytes per lane; lane i's bytes land at dst + 16 i (4 i), dst wave-uniform
__device__ __forceinline__ void to_lds16(const void *src, void *dst) {
    __builtin_amdgcn_global_load_lds((glb_void *)src, (lds_void *)dst, 16, 0, 0);
}
__device__ __forceinline__ void to_lds4(const void *src, void *dst) {
    __builtin_amdgcn_global_load_lds((glb_void *)src, (lds_void *)dst, 4, 0, 0);
}

__global__ __launch_bounds__(gm::NT, 3) void gemm_q8_kernel(GemmArgs a, int vec4) {
    using namespace gm;
    __shared__ __align__(16) GemmStage st0, st1;
    __shared__ int64_t sxr[BN];   // activation row of each of the tile's output rows (-1: none)
    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int64_t k = a.k, nr = a.nr, nb = k / 32;
    // plain GEMMs with a partial last row tile dispatch its workgroups after all full ones, and its
    // waves without a valid row skip the arithmetic: the round that holds them is short
    int64_t bx = blockIdx.x, by = blockIdx.y;
    if (!a.tiles) {
        const int64_t nfull = nr / BM;
        if (nfull < (int64_t)gridDim.x) {
            const int64_t L = (int64_t)blockIdx.y * gridDim.x + blockIdx.x, nf = nfull * gridDim.y;
            if (L < nf) {
                bx = L % nfull;
                by = L / nfull;
            } else {
                bx = nfull;
                by = L - nf;
            }
        }
    }
    const int64_t r0 = bx * BM;
    const bool wave_on = r0 + WR * w < nr;   // wave-uniform
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
        p0 = by * BN;
        pn = a.nt - p0 < BN ? a.nt - p0 : BN;
    }
    if (pn <= 0) return;   // uniform
    if (t < BN) sxr[t] = t < pn ? (a.xrow ? (int64_t)a.xrow[p0 + t] : p0 + t) : -1;
    __syncthreads();
    // Loads of one stage. Rows past the matrix (weights) or the tile (tokens) read a valid row
    // instead (the last weight row, the tile's first token): their outputs are never stored, and
    // each output element depends only on its own row's and token's codes and scales.
    // Wave w fills weight rows 32 w .. + 31 (4 x 8 rows of 128 bytes), token rows 16 w .. + 15 (2 x 8
    // rows), the weight scales of its 32 rows and (waves 0, 1) the token scales of rows 32 w .. + 31.
    // Lane L of a code load: row 8 q + (L >> 3) of the group, chunk (L & 7) ^ f(row) of the 128
    // bytes, stored at slot L & 7 (f(row) = (L >> 3) ^ (q & 1): each group starts at a multiple of
    // 8 rows, odd groups at an odd multiple); lane L of a scale load: row L >> 1, f16 pair L & 1.
    const int lr8 = lane >> 3, cch = (lane & 7) ^ lr8;
    const int64_t wlast = nr - 1;
    uint32_t wofs[4], xofs[2], wsofs, xsofs = 0;
#pragma unroll
    for (int q = 0; q < 4; q++) {
        const int64_t gr = r0 + WR * w + 8 * q + lr8;
        wofs[q] = (uint32_t)((gr < wlast ? gr : wlast) * k + 16 * (cch ^ (q & 1)));
    }
#pragma unroll
    for (int q = 0; q < 2; q++) {
        const int64_t xr = sxr[16 * w + 8 * q + lr8];
        xofs[q] = (uint32_t)((xr >= 0 ? xr : sxr[0]) * k + 16 * (cch ^ (q & 1)));
    }
    {
        const int64_t gr = r0 + WR * w + (lane >> 1);
        wsofs = (uint32_t)(((gr < wlast ? gr : wlast) * nb) * 2 + 4 * (lane & 1));
        if (w < 2) {
            const int64_t xr = sxr[32 * w + (lane >> 1)];
            xsofs = (uint32_t)(((xr >= 0 ? xr : sxr[0]) * nb) * 2 + 4 * (lane & 1));
        }
    }
    auto fetch = [&](GemmStage &S, int64_t kc) {
        const int8_t *wb = wq + kc, *xb = a.xq + kc;
        const int8_t *wsb = (const int8_t *)wd + kc / 16, *xsb = (const int8_t *)a.xd + kc / 16;
        if (wave_on) {
#pragma unroll
            for (int q = 0; q < 4; q++) to_lds16(wb + wofs[q], S.w + (WR * w + 8 * q) * KC);
            to_lds4(wsb + wsofs, S.dw + WR * w * NBC);
        }
#pragma unroll
        for (int q = 0; q < 2; q++) to_lds16(xb + xofs[q], S.x + (16 * w + 8 * q) * KC);
        if (w < 2) to_lds4(xsb + xsofs, S.dx + 32 * w * NBC);
    };
    // wave w: rows 32 w .. + 31 of the tile; tile j: tokens 32 j .. + 31. Fragment of a code row:
    // row / token lane & 31, the 16 bytes 16 (lane >> 5) .. of the block, at slot (2 b + (lane >> 5))
    // ^ f(row); f(row) = f(lane & 31) for both operands (their row bases are multiples of 16).
    const int wr = WR * w, fr = lane & 31, fh = lane >> 5;
    int fofs[NBC];
#pragma unroll
    for (int bb = 0; bb < NBC; bb++) fofs[bb] = fr * KC + 16 * ((2 * bb + fh) ^ (fr & 7) ^ ((fr >> 3) & 1));
    float acc[2][16];
#pragma unroll
    for (int j = 0; j < 2; j++)
#pragma unroll
        for (int v = 0; v < 16; v++) acc[j][v] = 0.0f;
    // one stage's chain: tile j's outputs in this lane are rows wr + 8 q + 4 (lane >> 5) + e
    // (v = 4 q + e), token 32 j + (lane & 31); the two-block scale product's block j is tile j
    auto compute = [&](const GemmStage &S, auto njc) {
        constexpr int NJ = decltype(njc)::value;
        if (!wave_on) return;
        const uint2 hw = *(const uint2 *)&S.dw[(wr + fr) * NBC];   // this lane's weight row, 4 blocks
        const uint2 hx = *(const uint2 *)&S.dx[lane * NBC];        // token `lane`, 4 blocks
        auto dots = [&](int bb, int j) {
            const i32x4 fa = *(const i32x4 *)(S.w + wr * KC + fofs[bb]);
            const i32x4 fb = *(const i32x4 *)(S.x + 32 * KC * j + fofs[bb]);
            const i32x16 zero = {};
            return __builtin_amdgcn_mfma_i32_32x32x32_i8(fa, fb, zero, 0, 0, 0);
        };
        auto scales = [&](int bb) {
            const uint32_t pw = bb < 2 ? hw.x : hw.y, px = bb < 2 ? hx.x : hx.y;
            const float dw = h2f((uint16_t)(pw >> (16 * (bb & 1)))), dx = h2f((uint16_t)(px >> (16 * (bb & 1))));
            const f32x32 zero = {};
            return __builtin_amdgcn_mfma_f32_32x32x1f32(dw, dx, zero, 0, 0, 0);
        };
        i32x16 s[NJ];
#pragma unroll
        for (int j = 0; j < NJ; j++) s[j] = dots(0, j);
        f32x32 d = scales(0);
#pragma unroll
        for (int bb = 0; bb < NBC; bb++) {
#pragma unroll
            for (int j = 0; j < NJ; j++) {
#pragma unroll
                for (int v = 0; v < 16; v++) acc[j][v] = __builtin_fmaf((float)s[j][v], d[16 * j + v], acc[j][v]);
                if (bb + 1 < NBC) s[j] = dots(bb + 1, j);
            }
            if (bb + 1 < NBC) d = scales(bb + 1);
        }
    };
    // every wave's loads of a stage done and visible before any wave reads it; every wave done with a
    // stage before it is refilled
    auto stage_sync = [&]() {
        __builtin_amdgcn_s_waitcnt(0);
        __syncthreads();
    };
    auto run = [&](auto njc) {
        const int64_t ns = k / KC;
        fetch(st0, 0);
        stage_sync();
        for (int64_t i = 0; i < ns; i += 2) {
            if (i + 1 < ns) fetch(st1, (i + 1) * KC);
            compute(st0, njc);
            stage_sync();
            if (i + 1 >= ns) break;
            if (i + 2 < ns) fetch(st0, (i + 2) * KC);
            compute(st1, njc);
            stage_sync();
        }
    };
    // tokens of the tile: a per-expert group fills a tile partly; an empty second tile is skipped
    // (uniform across the workgroup)
    if (pn > 32) run(std::integral_constant<int, 2>{});
    else run(std::integral_constant<int, 1>{});
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
    // 16-byte loads of codes
    if (((uintptr_t)a.wq | (uintptr_t)a.wd | (uintptr_t)a.xq | (uintptr_t)a.xd) % 16 != 0) return -1;
    // the kernel addresses one weight group's and the activations' codes with 32-bit offsets
    if ((uint64_t)a.nr * (uint64_t)a.k > UINT32_MAX || (uint64_t)a.nt * (uint64_t)a.k > UINT32_MAX) return -1;
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
