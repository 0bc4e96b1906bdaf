// Device-side building blocks shared by the gfx950 kernels: binary16 conversions, the integer
// dot, wave shuffles, and the exact-reduction helpers that let a parallel GPU reduction return the
// same bits as the reference's sequential double-precision sums.
//
// Every kernel source is compiled with -ffp-contract=off (no implicit fusion) and correctly rounded
// f32 division/sqrt, so each float operation below is one IEEE operation, as in the reference.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/oxe_model.h"
#include "oxe_libm.h"

#define OXE_DEV __device__ __forceinline__

namespace oxe {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

OXE_DEV float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// v_cvt_f16_f32 under the default round-to-nearest-even mode (= __fp16 conversion on aarch64).
// The empty asm pins f as a rounded f32 value: without it the compiler may fold a preceding f32
// multiply into the conversion (v_fma_mixlo_f16, one rounding straight to f16), which differs from
// the reference's f32 rounding followed by the f16 conversion in rare double-rounding cases.
OXE_DEV uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
OXE_DEV _Float16 hbits(uint16_t h) { return __builtin_bit_cast(_Float16, h); }
OXE_DEV uint16_t bitsh(_Float16 h) { return __builtin_bit_cast(uint16_t, h); }

// 4 x int8 dot with int32 accumulate (v_dot4_i32_i8): exact integer arithmetic
OXE_DEV int32_t dot4(uint32_t a, uint32_t b, int32_t c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}
OXE_DEV int32_t dot16(uint4 a, uint4 b, int32_t c) {
    c = dot4(a.x, b.x, c);
    c = dot4(a.y, b.y, c);
    c = dot4(a.z, b.z, c);
    return dot4(a.w, b.w, c);
}

OXE_DEV float shfl_xor_f(float v, int m) { return __shfl_xor(v, m, 64); }
OXE_DEV double shfl_xor_d(double v, int m) { return __shfl_xor(v, m, 64); }
OXE_DEV int shfl_xor_i(int v, int m) { return __shfl_xor(v, m, 64); }

// ---- DPP lane moves (no LDS round trip). Within a row of 16 lanes, row_ror:8 pairs lane c with
// c ^ 8; after that step every value is symmetric under ^ 8, so row_ror:4 then pairs c with c ^ 4;
// quad_perm gives ^ 1 and ^ 2 directly.
constexpr int DPP_XOR1 = 0xB1;   // quad_perm [1, 0, 3, 2]
constexpr int DPP_XOR2 = 0x4E;   // quad_perm [2, 3, 0, 1]
constexpr int DPP_ROR1 = 0x121, DPP_ROR2 = 0x122, DPP_ROR4 = 0x124, DPP_ROR8 = 0x128;
template <int CTRL>
OXE_DEV int dpp_i(int v) { return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false); }
template <int CTRL>
OXE_DEV float dpp_f(float v) { return __builtin_bit_cast(float, dpp_i<CTRL>(__builtin_bit_cast(int, v))); }
template <int CTRL>
OXE_DEV double dpp_d(double v) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const uint32_t lo = (uint32_t)dpp_i<CTRL>((int)(uint32_t)u), hi = (uint32_t)dpp_i<CTRL>((int)(uint32_t)(u >> 32));
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
OXE_DEV double readlane_d(double v, int lane) {
    const unsigned long long u = __builtin_bit_cast(unsigned long long, v);
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)u, lane);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)(u >> 32), lane);
    return __builtin_bit_cast(double, ((unsigned long long)hi << 32) | lo);
}
OXE_DEV float readlane_f(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// Sum over the wave of a double whose summation order is free (the exact-sum bracket below accepts
// any order): rows of 16 by rotation, then the four row sums. Uniform result.
OXE_DEV double wave_sum_d_any(double v) {
    v += dpp_d<DPP_ROR8>(v);
    v += dpp_d<DPP_ROR4>(v);
    v += dpp_d<DPP_ROR2>(v);
    v += dpp_d<DPP_ROR1>(v);
    return (readlane_d(v, 0) + readlane_d(v, 16)) + (readlane_d(v, 32) + readlane_d(v, 48));
}
// (v > o ? v : o) over the wave. Uniform result.
OXE_DEV float wave_max_any(float v) {
    float o;
    o = dpp_f<DPP_ROR8>(v); v = v > o ? v : o;
    o = dpp_f<DPP_ROR4>(v); v = v > o ? v : o;
    o = dpp_f<DPP_ROR2>(v); v = v > o ? v : o;
    o = dpp_f<DPP_ROR1>(v); v = v > o ? v : o;
    const float a = readlane_f(v, 0), b = readlane_f(v, 16), c = readlane_f(v, 32), d = readlane_f(v, 48);
    const float ab = a > b ? a : b, cd = c > d ? c : d;
    return ab > cd ? ab : cd;
}
// the 16-lane tree of ggml_vec_dot_f32's NEON reduce (lane c = chain c): ^8, ^4, ^1, ^2
OXE_DEV float dot16_tree_dpp(float acc) {
    acc = acc + dpp_f<DPP_ROR8>(acc);
    acc = acc + dpp_f<DPP_ROR4>(acc);
    acc = acc + dpp_f<DPP_XOR1>(acc);
    acc = acc + dpp_f<DPP_XOR2>(acc);
    return acc;
}

// ggml_v_expf NEON (vendor/ggml-subset/generated/upstream/src/ggml-cpu/vec.h:1154-1175), one lane
OXE_DEV float v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = __builtin_fmaf(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, __builtin_fmaf(-n, 0x1.62e4p-1f, x));
    const uint32_t e = __builtin_bit_cast(uint32_t, z) << 23;
    const float k = __builtin_bit_cast(float, e + 0x3f800000u);
    const bool c = __builtin_fabsf(n) > 126.0f;
    const float u = b * b;
    const float j = __builtin_fmaf(__builtin_fmaf(__builtin_fmaf(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                                                  __builtin_fmaf(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                                   u, 0x1.ffffecp-1f * b);
    if (!c) return __builtin_fmaf(j, k, k);
    const uint32_t d = (n <= 0.0f) ? 0x82000000u : 0u;
    const float s1 = __builtin_bit_cast(float, d + 0x7f000000u);
    const float s2 = __builtin_bit_cast(float, e - d);
    if (__builtin_fabsf(n) > 192.0f) return s1 * s1;
    return __builtin_fmaf(s2, j, s2) * s1;
}
// ggml_v_silu (vec.h:1178-1185)
OXE_DEV float v_silu(float x) { return x / (1.0f + v_expf(0.0f - x)); }
// op_sigmoid with the C library's expf (crates/kernels-sys/csrc/oxe_ops.cpp:80-84)
OXE_DEV float sigmoid_c(float x) { return 1.f / (1.f + oxe_libm::expf_c(-x)); }
// op_softplus (oxe_ops.cpp:85-89)
OXE_DEV float softplus_c(float x) { return (x > 20.0f) ? x : oxe_libm::log1pf_c(oxe_libm::expf_c(x)); }
// the same two with the expf table passed in (an LDS copy)
template <class Tab>
OXE_DEV float sigmoid_t(float x, Tab tab) { return 1.f / (1.f + oxe_libm::expf_t(-x, tab)); }
template <class Tab>
OXE_DEV float softplus_t(float x, Tab tab) { return (x > 20.0f) ? x : oxe_libm::log1pf_c(oxe_libm::expf_t(x, tab)); }

// quantize_row_q8_0, NEON branch (vendor/ggml-subset/generated/quants_subset.c:6-42), one thread
// per 32-value block: amax (exact), d = amax/127, id = d ? 1/d : 0 from the f32 d, fp16(d) by RNE,
// codes = round-to-nearest-even(x * id) (vcvtnq_s32_f32).
OXE_DEV void quant_block_q8_0(const float *x, int8_t *q, uint16_t *d) {
    float v[32];
#pragma unroll
    for (int j = 0; j < 32; j += 4) {
        const float4 f = *(const float4 *)(x + j);
        v[j] = f.x; v[j + 1] = f.y; v[j + 2] = f.z; v[j + 3] = f.w;
    }
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 32; j++) amax = fmaxf(amax, __builtin_fabsf(v[j]));
    const float dd = amax / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    *d = f2h(dd);
    uint32_t packed[8];
#pragma unroll
    for (int j = 0; j < 8; j++) {
        uint32_t u = 0;
#pragma unroll
        for (int b = 0; b < 4; b++) {
            const int32_t qi = (int32_t)__builtin_rintf(v[4 * j + b] * id);
            u |= ((uint32_t)(qi & 0xff)) << (8 * b);
        }
        packed[j] = u;
    }
    *(uint4 *)q = make_uint4(packed[0], packed[1], packed[2], packed[3]);
    *(uint4 *)(q + 16) = make_uint4(packed[4], packed[5], packed[6], packed[7]);
}

// max over the 32-lane half of the wave holding this lane (exact, any order)
OXE_DEV float half_max(float v) {
    v = fmaxf(v, dpp_f<DPP_ROR8>(v));
    v = fmaxf(v, dpp_f<DPP_ROR4>(v));
    v = fmaxf(v, dpp_f<DPP_ROR2>(v));
    v = fmaxf(v, dpp_f<DPP_ROR1>(v));
    const float lo = fmaxf(readlane_f(v, 0), readlane_f(v, 16)), hi = fmaxf(readlane_f(v, 32), readlane_f(v, 48));
    return (threadIdx.x & 63) < 32 ? lo : hi;
}
// quantize_row_q8_0 (NEON) of the 32-value block held one value per lane by each half of the
// wave: *d = the block scale; returns in lane 4 i the codes of lanes 4 i .. 4 i + 3 (byte order)
OXE_DEV uint32_t quant32_lanes(float v, float *d) {
    const float m = half_max(__builtin_fabsf(v));
    const float dd = m / 127.0f;
    const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
    const int32_t q = (int32_t)__builtin_rintf(v * id);
    int p = (int)((uint32_t)(q & 0xff) << (8 * (threadIdx.x & 3)));
    p |= dpp_i<DPP_XOR1>(p);
    p |= dpp_i<DPP_XOR2>(p);
    *d = dd;
    return (uint32_t)p;
}

// ---- block reductions (blockDim.x threads, all participating)

template <int NT>
OXE_DEV double block_sum_d(double v, double *red) {
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_d(v, m);
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[w] = v;
    __syncthreads();
    double s = 0.0;
    if (threadIdx.x == 0) {
        for (int i = 0; i < NT / 64; i++) s += red[i];
        red[NT / 64] = s;
    }
    __syncthreads();
    s = red[NT / 64];
    __syncthreads();
    return s;
}

template <int NT>
OXE_DEV float block_max_f(float v, float *red) {
    for (int m = 32; m >= 1; m >>= 1) {
        const float o = shfl_xor_f(v, m);
        v = (v > o) ? v : o;
    }
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    if (lane == 0) red[w] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float s = red[0];
        for (int i = 1; i < NT / 64; i++) s = (s > red[i]) ? s : red[i];
        red[NT / 64] = s;
    }
    __syncthreads();
    const float s = red[NT / 64];
    __syncthreads();
    return s;
}

// Exact-match helper for the reference's sequential double sums.
// The reference forms S = (((0 + t0) + t1) + ...) over m terms in double and only uses a float
// derived from S by a monotone map g (g(S) = (float)(S / n) or (float)(1.0 / S)). Both S and a
// parallel tree sum P lie within (m - 1) * 2^-53 * sum|t_i| of the exact sum, so with
// B = (m + 64) * 2^-52 * sum|t_i|, g(P - B) == g(P + B) proves g(S) == g(P); otherwise the caller
// replays the sequential sum (rare: the interval must straddle a float rounding edge).
OXE_DEV double bracket_width(double abs_sum, int m) { return abs_sum * (double)(m + 64) * 0x1p-52; }
OXE_DEV bool bracket_ok_mean(double p, double abs_sum, int m, double n, float *out) {
    const double b = bracket_width(abs_sum, m);
    const float lo = (float)((p - b) / n), hi = (float)((p + b) / n);
    *out = (float)(p / n);
    return lo == hi;
}
OXE_DEV bool bracket_ok_recip(double p, double abs_sum, int m, float *out) {
    const double b = bracket_width(abs_sum, m);
    const float lo = (float)(1.0 / (p + b)), hi = (float)(1.0 / (p - b));
    *out = (float)(1.0 / p);
    return lo == hi;
}

}  // namespace oxe
