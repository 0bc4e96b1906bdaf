// Host-side launch helpers shared by the kernel translation units and the engine.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace oxe {
int quantize_q8_0(const float *x, int64_t n, int8_t *q, uint16_t *d, hipStream_t st);
}  // namespace oxe

namespace oxe {
int synth_q8(uint64_t seed, int layer, int kind_a, int kind_b, int64_t rows, int64_t k, int64_t src_rows,
             int64_t expert, int8_t *q, uint16_t *d, hipStream_t st);
int synth_f32(uint64_t seed, int layer, int kind, int64_t n, float *out, hipStream_t st);
// a matrix in another type than Q8_0: the oracle's synthetic K-quant blocks (ggml type 11..14) or
// F32 values (0); rows counts every expert of an expert tensor. 0, -1 (type), -2 (launch)
int synth_raw(uint64_t seed, int layer, int kind, int type, int64_t rows, int64_t k, void *out, hipStream_t st);
}  // namespace oxe
