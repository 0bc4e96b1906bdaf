// Parity hook: the device's scalar functions evaluated over a range of float bit patterns, so the
// tests can compare them with the host C library and the oracle over every input.
#include "oxe_common.h"

namespace oxe {

__global__ void eval_unary_kernel(int fn, uint32_t start, int64_t n, int64_t stride, float *__restrict__ y) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float x = __builtin_bit_cast(float, (uint32_t)(start + (uint64_t)i * (uint64_t)stride));
    float r;
    switch (fn) {
        case 0: r = oxe_libm::expf_c(x); break;
        case 1: r = oxe_libm::log1pf_c(x); break;
        case 2: r = v_expf(x); break;
        case 3: r = sigmoid_c(x); break;
        case 4: r = softplus_c(x); break;
        default: r = v_silu(x); break;
    }
    y[i] = r;
}

}  // namespace oxe

extern "C" int oxe_hip_eval_unary(int fn, uint32_t start, int64_t n, int64_t stride, float *y, void *stream) {
    if (fn < 0 || fn > 5 || n <= 0 || stride <= 0 || !y) return -1;
    if ((uint64_t)start + (uint64_t)(n - 1) * (uint64_t)stride > 0xffffffffull) return -1;
    hipLaunchKernelGGL(oxe::eval_unary_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, fn,
                       start, n, stride, y);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}
