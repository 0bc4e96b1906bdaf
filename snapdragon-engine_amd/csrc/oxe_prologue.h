// Workgroup prologues shared by the layer kernels: the exact RMS norm of an n_embd vector, the
// Q8_0 quantization of a normalised vector straight into LDS, and the token embedding.
#pragma once
#include "oxe_common.h"
#include "oxe_engine.h"
#include "oxe_shape.h"

namespace oxe {

constexpr int PT = 256;                  // threads of the prologue workgroups
constexpr int EPT = shp::E / PT;         // 8 n_embd elements per thread (thread t owns [8t, 8t+8))
static_assert(EPT == 8, "prologue assumes 8 elements per thread");

struct NormScratch {
    double red[PT / 64 + 1];
    float bc;
};

// oxe_rms_norm_mul_f32 (crates/kernels-sys/csrc/oxe_ops.cpp:32-42) of one n_embd vector: sum of
// double(f32(x*x)), mean = f32(sum / n), scale = 1/sqrtf(mean + eps), y = (x * scale) * w.
// v: this thread's 8 elements of x (in) and of y (out). xg: the same vector in global memory (the
// sequential replay when the parallel sum cannot prove the reference's rounding).
OXE_DEV void rms_norm_mul_e(float v[EPT], const float *xg, const float *w, float eps, NormScratch &ns) {
    const int t = threadIdx.x;
    double p = 0.0;
#pragma unroll
    for (int i = 0; i < EPT; i++) p += (double)(v[i] * v[i]);
    const double P = block_sum_d<PT>(p, ns.red);
    float mean;
    if (!bracket_ok_mean(P, P, shp::E, (double)shp::E, &mean)) {
        if (t == 0) {
            double s = 0.0;
            for (int i = 0; i < shp::E; i++) s += (double)(xg[i] * xg[i]);
            ns.bc = (float)(s / (double)shp::E);
        }
        __syncthreads();
        mean = ns.bc;
        __syncthreads();
    }
    const float scale = 1.0f / sqrtf(mean + eps);
    const float4 w0 = *(const float4 *)(w + EPT * t), w1 = *(const float4 *)(w + EPT * t + 4);
    const float wv[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
#pragma unroll
    for (int i = 0; i < EPT; i++) v[i] = (v[i] * scale) * wv[i];
}

// quantize_row_q8_0 NEON (quants_subset.c:6-42) of 8 consecutive values per thread, 4 threads per
// 32-block (lanes t..t+3 aligned to 4): codes to q[0..8), the block's fp16 scale to *d by the
// first thread of the four.
OXE_DEV void quant8(const float v[8], int8_t *q, uint16_t *d) {
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; i++) am = fmaxf(am, __builtin_fabsf(v[i]));
    am = fmaxf(am, dpp_f<DPP_XOR1>(am));
    am = fmaxf(am, dpp_f<DPP_XOR2>(am));
    const float dd = am / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    uint32_t lo = 0, hi = 0;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        lo |= ((uint32_t)((int32_t)__builtin_rintf(v[i] * id) & 0xff)) << (8 * i);
        hi |= ((uint32_t)((int32_t)__builtin_rintf(v[i + 4] * id) & 0xff)) << (8 * i);
    }
    *(uint2 *)q = make_uint2(lo, hi);
    if ((threadIdx.x & 3) == 0) *d = f2h(dd);
}

// this thread's 8 elements of a global vector
OXE_DEV void load8(const float *x, float v[8]) {
    const float4 a = *(const float4 *)(x + EPT * threadIdx.x), b = *(const float4 *)(x + EPT * threadIdx.x + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
OXE_DEV void store8(float *x, const float v[8]) {
    *(float4 *)(x + EPT * threadIdx.x) = make_float4(v[0], v[1], v[2], v[3]);
    *(float4 *)(x + EPT * threadIdx.x + 4) = make_float4(v[4], v[5], v[6], v[7]);
}

// dequantize_row_q8_0 (vendor/ggml-subset/generated/quants_base.c:64-78) of this thread's 8
// elements of token row `tok`: y = q * f32(d)
OXE_DEV void embed8(const Q8W &emb, uint32_t tok, float v[8]) {
    const int t = threadIdx.x;
    const int8_t *q = emb.q + (int64_t)tok * shp::E + EPT * t;
    const float d = h2f(emb.d[(int64_t)tok * (shp::E / 32) + (EPT * t) / 32]);
    const uint2 c = *(const uint2 *)q;
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[i] = (float)(int8_t)(c.x >> (8 * i)) * d;
        v[i + 4] = (float)(int8_t)(c.y >> (8 * i)) * d;
    }
}

// Exact sum of squares of a 128-element vector held 2 per lane by one wave, for the l2 / gated
// norms (oxe_ops.cpp:19-49): returns f32(sum/n). All 64 lanes of the wave call it.
OXE_DEV float wave_mean_sq_128(float a, float b, const float *x_replay) {
    const double p = wave_sum_d_any((double)(a * a) + (double)(b * b));
    float mean;
    if (!bracket_ok_mean(p, p, 128, 128.0, &mean)) {
        double s = 0.0;
        for (int i = 0; i < 128; i++) s += (double)(x_replay[i] * x_replay[i]);
        mean = (float)(s / 128.0);
    }
    return mean;
}

// The same for a 256-element vector held 4 per lane (q / k norms of attention).
OXE_DEV float wave_mean_sq_256(const float v[4], const float *x_replay) {
    double q = 0.0;
#pragma unroll
    for (int i = 0; i < 4; i++) q += (double)(v[i] * v[i]);
    const double p = wave_sum_d_any(q);
    float mean;
    if (!bracket_ok_mean(p, p, 256, 256.0, &mean)) {
        double s = 0.0;
        for (int i = 0; i < 256; i++) s += (double)(x_replay[i] * x_replay[i]);
        mean = (float)(s / 256.0);
    }
    return mean;
}

// rotate_pairs NEOX (oxe_ops.cpp:443-455) of x[0..64) in LDS with the position's cache (cos, sin
// pairs); lanes 0..31 of the calling wave each rotate one pair. The product fused into each
// expression is the first one (fma(x0, c, -(x1*s)), fma(x0, s, x1*c)): the reference's C compiler
// contracts a*b - c*d that way.
OXE_DEV void rope_neox_lds(float *x, const float *cache, int lane) {
    if (lane < shp::NROT / 2) {
        const float c = cache[2 * lane], s = cache[2 * lane + 1];
        const float x0 = x[lane], x1 = x[lane + shp::NROT / 2];
        x[lane] = __builtin_fmaf(x0, c, -(x1 * s));
        x[lane + shp::NROT / 2] = __builtin_fmaf(x0, s, x1 * c);
    }
}

}  // namespace oxe
