// Q8_0 GEMV tile for 1-4 activation lanes in one weight pass (gfx950), shared by every kernel that
// reads Q8_0 weights (dense projections, experts, the LM head).
//
// Contract (reference: ggml_gemv_q8_0_4x8_q8_0 NEON+dotprod, vendor/ggml-subset/generated/
// repack_subset.cpp:1633-1679, and the lane GEMV oxe_vl_gemv_q8_0, crates/kernels-sys/csrc/
// oxe_vl_q80.inc:25-89): for output row r and lane l,
//     isum_b = exact int32 dot of the 32 weight codes of block b with the 32 activation codes
//     acc    = fma(f32(isum_b), f32(d_x[l][b]) * f32(d_w[r][b]), acc)   for b = 0, 1, ... from +0
//
// Layout (this build's own; the math is layout-free): codes int8 [rows][K] row-major, fp16 scales
// [rows][K/32]. One 256-thread workgroup owns R consecutive rows. Phase 1 (bandwidth): every thread
// streams 16-byte code chunks (64 threads read 1 KB contiguous per instruction), dots them with the
// activation chunk it keeps in registers (v_dot4_i32_i8), and the two half-block partials meet by a
// lane shuffle; block sums go to LDS. Phase 2 (latency): one thread per (row, lane) runs the serial
// fp32 FMA chain over the blocks, exactly the reference order. Decode is HBM-bound: phase 1 issues
// all of a thread's loads before any arithmetic, so each workgroup keeps R*K bytes in flight.
#pragma once
#include "oxe_common.h"

namespace oxe {

constexpr int GEMV_THREADS = 256;
constexpr int GEMV_MAX_LANES = 4;   // the reference's OXE_VL_MAX_LANES

template <int K>
struct GemvGeom {
    static constexpr int NB = K / 32;      // Q8_0 blocks per row
    static constexpr int KCH = K / 16;     // 16-byte chunks per row
    static_assert(KCH <= 256 && 256 % KCH == 0, "K must be 512..4096");
    static constexpr int RPP = 256 / KCH;  // rows per pass of the workgroup
    static constexpr int WDS = NB / 2 + 1; // LDS scale row stride in words (odd: conflict-free)
};

template <int K, int R, int NL>
struct GemvSmem {
    int32_t isum[NL][R][GemvGeom<K>::NB + 1];
    uint32_t wd[R * GemvGeom<K>::WDS];
    uint16_t xd[NL][GemvGeom<K>::NB];
    float out[NL][R];
};

// Computes sm.out[l][r] for rows row0 .. row0+R-1 (rows >= nrows read as zero) of the matrix at
// (wq, wd), lanes l < NL with activation codes xq[l] / scales xd[l]. Ends with a barrier.
// isum_out (optional): [NL][nrows_total][K/32] int32 block dots, row index row0 + r.
template <int K, int R, int NL>
OXE_DEV void gemv_tile(const int8_t *__restrict__ wq, const uint16_t *__restrict__ wd, int64_t row0, int64_t nrows,
                       const int8_t *const *xq, const uint16_t *const *xd, GemvSmem<K, R, NL> &sm,
                       int32_t *isum_out = nullptr) {
    using G = GemvGeom<K>;
    constexpr int NB = G::NB, KCH = G::KCH, RPP = G::RPP, WDS = G::WDS;
    static_assert(R % RPP == 0, "R must be a multiple of rows per pass");
    constexpr int PASSES = R / RPP;
    const int t = threadIdx.x;
    const int c = t % KCH, rs = t / KCH;

    uint4 w[PASSES];
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int64_t r = row0 + p * RPP + rs;
        w[p] = r < nrows ? *(const uint4 *)(wq + r * K + c * 16) : make_uint4(0, 0, 0, 0);
    }
    uint4 xa[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) xa[l] = *(const uint4 *)(xq[l] + c * 16);
    {
        const uint32_t *wds = (const uint32_t *)(wd + row0 * NB);
        for (int i = t; i < R * NB / 2; i += GEMV_THREADS) {
            const int r = (i * 2) / NB, b2 = i % (NB / 2);
            sm.wd[r * WDS + b2] = row0 + r < nrows ? wds[i] : 0u;
        }
        for (int i = t; i < NL * NB; i += GEMV_THREADS) sm.xd[i / NB][i % NB] = xd[i / NB][i % NB];
    }
#pragma unroll
    for (int p = 0; p < PASSES; p++) {
        const int r = p * RPP + rs;
#pragma unroll
        for (int l = 0; l < NL; l++) {
            int32_t s = dot16(w[p], xa[l], 0);
            s += shfl_xor_i(s, 1);  // the other half of the 32-code block sits in the adjacent lane
            if ((c & 1) == 0) sm.isum[l][r][c >> 1] = s;
        }
    }
    __syncthreads();
    if (t < R * NL) {
        const int r = t % R, l = t / R;
        const uint16_t *sw = (const uint16_t *)(sm.wd + r * WDS);
        float acc = 0.0f;
#pragma unroll 8
        for (int b = 0; b < NB; b++) {
            const float prod = h2f(sm.xd[l][b]) * h2f(sw[b]);
            acc = __builtin_fmaf((float)sm.isum[l][r][b], prod, acc);
        }
        sm.out[l][r] = acc;
    }
    if (isum_out) {
        for (int i = t; i < NL * R * NB; i += GEMV_THREADS) {
            const int l = i / (R * NB), r = (i / NB) % R, b = i % NB;
            if (row0 + r < nrows) isum_out[((int64_t)l * nrows + row0 + r) * NB + b] = sm.isum[l][r][b];
        }
    }
    __syncthreads();
}

// Rows per workgroup for each K: enough to keep ~32-64 KB of codes in flight per workgroup.
template <int K> struct GemvR;
template <> struct GemvR<512> { static constexpr int R = 32; };
template <> struct GemvR<2048> { static constexpr int R = 16; };
template <> struct GemvR<4096> { static constexpr int R = 8; };

// Activation lanes of a plain GEMV: xq [NL][K] int8, xd [NL][K/32] fp16, contiguous per lane.
struct Acts {
    const int8_t *q;
    const uint16_t *d;
};

// Plain GEMV kernel: y rows of one matrix; the epilogue gets the tile (all threads, after barrier).
template <int K, int NL, class Epi>
__global__ __launch_bounds__(GEMV_THREADS) void gemv_kernel(const int8_t *__restrict__ wq,
                                                            const uint16_t *__restrict__ wd, int64_t nrows, Acts a,
                                                            int32_t *isum_out, Epi epi) {
    constexpr int R = GemvR<K>::R;
    __shared__ GemvSmem<K, R, NL> sm;
    const int8_t *xq[NL];
    const uint16_t *xd[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) {
        xq[l] = a.q + (int64_t)l * K;
        xd[l] = a.d + (int64_t)l * (K / 32);
    }
    const int64_t row0 = (int64_t)blockIdx.x * R;
    gemv_tile<K, R, NL>(wq, wd, row0, nrows, xq, xd, sm, isum_out);
    const int nvalid = (int)(nrows - row0 < R ? nrows - row0 : R);
    epi.template tile<NL, R>(row0, nvalid, sm.out);
}

// ---- epilogues -------------------------------------------------------------------------------

// y[l * ld + row] = acc (+ res[l * ld_res + row] when res != nullptr: the mixer residual
// x1 = out + x, crates/model/src/engine.rs:2598-2603)
struct EpiStore {
    float *y;
    int64_t ld;
    const float *res;
    int64_t ld_res;
    template <int NL, int R>
    OXE_DEV void tile(int64_t row0, int nvalid, const float (&out)[NL][R]) const {
        for (int i = threadIdx.x; i < NL * R; i += GEMV_THREADS) {
            const int l = i / R, r = i % R;
            if (r < nvalid) {
                float v = out[l][r];
                if (res) v = v + res[l * ld_res + row0 + r];
                y[l * ld + row0 + r] = v;
            }
        }
    }
};

template <int K, class Epi>
inline int gemv_launch(int nl, const int8_t *wq, const uint16_t *wd, int64_t nrows, Acts a, int32_t *isum_out,
                       Epi epi, hipStream_t st) {
    constexpr int R = GemvR<K>::R;
    const unsigned nb = (unsigned)((nrows + R - 1) / R);
    if (nl == 1) hipLaunchKernelGGL((gemv_kernel<K, 1, Epi>), dim3(nb), dim3(GEMV_THREADS), 0, st, wq, wd, nrows, a, isum_out, epi);
    else if (nl == 2) hipLaunchKernelGGL((gemv_kernel<K, 2, Epi>), dim3(nb), dim3(GEMV_THREADS), 0, st, wq, wd, nrows, a, isum_out, epi);
    else if (nl == 3) hipLaunchKernelGGL((gemv_kernel<K, 3, Epi>), dim3(nb), dim3(GEMV_THREADS), 0, st, wq, wd, nrows, a, isum_out, epi);
    else if (nl == 4) hipLaunchKernelGGL((gemv_kernel<K, 4, Epi>), dim3(nb), dim3(GEMV_THREADS), 0, st, wq, wd, nrows, a, isum_out, epi);
    else return -1;
    return 0;
}

template <class Epi>
inline int gemv_launch_k(int64_t k, int nl, const int8_t *wq, const uint16_t *wd, int64_t nrows, Acts a,
                         int32_t *isum_out, Epi epi, hipStream_t st) {
    switch (k) {
    case 512: return gemv_launch<512>(nl, wq, wd, nrows, a, isum_out, epi, st);
    case 2048: return gemv_launch<2048>(nl, wq, wd, nrows, a, isum_out, epi, st);
    case 4096: return gemv_launch<4096>(nl, wq, wd, nrows, a, isum_out, epi, st);
    default: return -1;
    }
}

}  // namespace oxe
