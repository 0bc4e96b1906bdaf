// Kernel-level C ABI for the Q8_0 activation quantizer and the lane GEMV (the device
// counterparts of the reference's quantize_row_q8_0 and oxe_vl_gemv / ggml_gemv_q8_0_4x8_q8_0).
#include "oxe_gemv.h"
#include "oxe_kernels.h"

namespace oxe {

__global__ void quantize_q8_0_kernel(const float *__restrict__ x, int64_t nblocks, int8_t *__restrict__ q,
                                     uint16_t *__restrict__ d) {
    const int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (b < nblocks) quant_block_q8_0(x + b * 32, q + b * 32, d + b);
}

int quantize_q8_0(const float *x, int64_t n, int8_t *q, uint16_t *d, hipStream_t st) {
    if (n <= 0 || n % 32 != 0) return -1;
    const int64_t nb = n / 32;
    hipLaunchKernelGGL(quantize_q8_0_kernel, dim3((unsigned)((nb + 255) / 256)), dim3(256), 0, st, x, nb, q, d);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Q8_0 lane GEMV for any k that is a multiple of 32 (the shapes without a tuned kernel): one wave
// per row; lane i forms the exact int32 dots of blocks i, i + 64, ... for every activation lane, then
// thread l of the wave runs lane l's fp32 chain over the blocks in order from +0
// (ggml_gemv_q8_0_4x8_q8_0, repack_subset.cpp:1672: acc = fma(isum, d_x * d_w, acc)).
constexpr int GG_ROWS = 4;
__global__ __launch_bounds__(64 * GG_ROWS) void gemv_any_kernel(int64_t k, int64_t nr, int nl, const int8_t *__restrict__ wq,
                                                               const uint16_t *__restrict__ wd, const int8_t *__restrict__ xq,
                                                               const uint16_t *__restrict__ xd, float *__restrict__ y,
                                                               int32_t *__restrict__ isum_out) {
    extern __shared__ int32_t gg_isum[];   // [GG_ROWS][nl][nb]
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t nb = k / 32, r = (int64_t)blockIdx.x * GG_ROWS + w;
    int32_t *is = gg_isum + (int64_t)w * nl * nb;
    if (r < nr) {
        for (int64_t b = lane; b < nb; b += 64) {
            const uint4 *wp = (const uint4 *)(wq + r * k + 32 * b);
            const uint4 w0 = wp[0], w1 = wp[1];
            for (int l = 0; l < nl; l++) {
                const uint4 *xp = (const uint4 *)(xq + l * k + 32 * b);
                is[l * nb + b] = dot16(w1, xp[1], dot16(w0, xp[0], 0));
            }
        }
    }
    __syncthreads();
    if (r < nr && lane < nl) {
        const int l = lane;
        float acc = 0.0f;
        for (int64_t b = 0; b < nb; b++) {
            const int32_t v = is[l * nb + b];
            acc = __builtin_fmaf((float)v, h2f(xd[l * nb + b]) * h2f(wd[r * nb + b]), acc);
            if (isum_out) isum_out[((int64_t)l * nr + r) * nb + b] = v;
        }
        y[(int64_t)l * nr + r] = acc;
    }
}

}  // namespace oxe

extern "C" {

int oxe_hip_quantize_row_q8_0(const float *x, int64_t k, int64_t nrows, int8_t *q, uint16_t *d, void *stream) {
    if (k <= 0 || k % 32 != 0 || nrows <= 0) return -1;
    return oxe::quantize_q8_0(x, k * nrows, q, d, (hipStream_t)stream);
}

// oxe_vl_gemv's contract (crates/kernels-sys/csrc/oxe_vl.inc:78-107, bound as `!= 0` by
// gemv_lanes_raw, crates/kernels-sys/src/lib.rs:652-666): 1 when done; 0 with nothing written when
// there is no kernel for the call (lanes outside 1..4, no rows, k not a positive multiple of 32 or
// past the one-wave-per-row kernel's LDS); -2 on a launch error
int oxe_hip_gemv_q8_0(int64_t k, int64_t nr, int nl, const int8_t *wq, const uint16_t *wd, const int8_t *xq,
                      const uint16_t *xd, float *y, int32_t *isum, void *stream) {
    if (nr <= 0 || nl < 1 || nl > oxe::GEMV_MAX_LANES || k <= 0 || k % 32 != 0) return 0;
    if (k != 512 && k != 2048 && k != 4096) {
        const size_t lds = (size_t)oxe::GG_ROWS * nl * (k / 32) * sizeof(int32_t);
        if (lds > 64 * 1024) return 0;   // k > 32768 with 4 lanes, 65536 with 2, 131072 with 1
        hipLaunchKernelGGL(oxe::gemv_any_kernel, dim3((unsigned)((nr + oxe::GG_ROWS - 1) / oxe::GG_ROWS)),
                           dim3(64 * oxe::GG_ROWS), lds, (hipStream_t)stream, k, nr, nl, wq, wd, xq, xd, y, isum);
        return hipGetLastError() == hipSuccess ? 1 : -2;
    }
    oxe::EpiStore epi{y, nr, nullptr, 0};
    if (oxe::gemv_launch_k(k, nl, wq, wd, nr, oxe::Acts{xq, xd}, isum, epi, (hipStream_t)stream) != 0) return 0;
    return hipGetLastError() == hipSuccess ? 1 : -2;
}

}  // extern "C"
