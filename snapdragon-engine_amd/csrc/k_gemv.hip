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

}  // namespace oxe

extern "C" {

int oxe_hip_quantize_row_q8_0(const float *x, int64_t k, int64_t nrows, int8_t *q, uint16_t *d, void *stream) {
    if (k <= 0 || k % 32 != 0 || nrows <= 0) return -1;
    return oxe::quantize_q8_0(x, k * nrows, q, d, (hipStream_t)stream);
}

int oxe_hip_gemv_q8_0(int64_t k, int64_t nr, int nl, const int8_t *wq, const uint16_t *wd, const int8_t *xq,
                      const uint16_t *xd, float *y, int32_t *isum, void *stream) {
    if (nr <= 0 || nl < 1 || nl > 2 || (k != 512 && k != 2048 && k != 4096)) return -1;
    oxe::EpiStore epi{y, nr, nullptr, 0};
    const int rc = oxe::gemv_launch_k(k, nl, wq, wd, nr, oxe::Acts{xq, xd}, isum, epi, (hipStream_t)stream);
    if (rc != 0) return rc;
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // extern "C"
