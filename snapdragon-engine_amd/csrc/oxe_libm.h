// C-library transcendental functions the reference calls on the decode path, restated so the GPU
// computes the same bits as the host C library (glibc) the oracle links:
//   expf   - sigmoid / softplus gates and e^g of the delta rule (crates/kernels-sys/csrc/oxe_ops.cpp:80-89, 221, 235)
//   log1pf - softplus (oxe_ops.cpp:85-89)
// Both are __host__ __device__ so the same source is checked exhaustively on the CPU against the
// C library (tests/test_libm.py) and compiled unchanged for gfx950. Compile with
// -ffp-contract=off: every fused operation is an explicit fma().
#pragma once
#include <stdint.h>

#if defined(__HIPCC__)
#define OXE_HD __host__ __device__ inline
#else
#define OXE_HD static inline
#include <math.h>
#include <string.h>
#endif

namespace oxe_libm {

OXE_HD uint32_t f2u(float f) { return __builtin_bit_cast(uint32_t, f); }
OXE_HD float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }
OXE_HD uint64_t d2u(double d) { return __builtin_bit_cast(uint64_t, d); }
OXE_HD double u2d(uint64_t u) { return __builtin_bit_cast(double, u); }

// expf by the published method of Szabolcs Nagy (ARM optimized-routines, exp2f_data; glibc >= 2.27
// sysdeps/ieee754/flt-32/e_expf.c, FMA variant): x*32/ln2 = k + r with k rounded to nearest even
// by the 1.5*2^52 shift, 2^(k/32) from a 32-entry table of bits(2^(i/32)) - (i << 47), and
// 2^(r/32) by a cubic in r evaluated in double with fused multiply-adds.
// The table entries are 2^(i/32) rounded to double.
#if defined(__HIPCC__)
__device__ __constant__ static const uint64_t kExp2fTab[32] = {
#else
static const uint64_t kExp2fTab[32] = {
#endif
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL,
};

// tab: the 32 entries above, from any address space (a device caller may pass a copy in LDS so the
// lookup is an LDS read instead of a global load behind the memory operations in flight)
template <class Tab>
OXE_HD float expf_t(float x, Tab tab) {
    const double xd = (double)x;
    const uint32_t abstop = (f2u(x) >> 20) & 0x7ff;
    if (abstop >= (f2u(88.0f) >> 20)) {
        if (f2u(x) == f2u(-__builtin_inff())) return 0.0f;
        if (abstop >= (f2u(__builtin_inff()) >> 20)) return x + x;
        if (x > 0x1.62e42ep6f) return __builtin_inff();       // overflow
        if (x < -0x1.9fe368p6f) return 0.0f;                  // underflow
    }
    const double invln2n = 0x1.71547652b82fep+0 * 32;
    const double shift = 0x1.8p+52;
    // the product x*32/ln2 is fused into both of its uses (the C library's FMA build contracts them)
    double kd = __builtin_fma(invln2n, xd, shift);
    const uint64_t ki = d2u(kd);
    kd -= shift;
    const double r = __builtin_fma(invln2n, xd, -kd);
    uint64_t t = tab[ki % 32];
    t += ki << 47;
    const double s = u2d(t);
    const double c0 = 0x1.c6af84b912394p-5 / 32 / 32 / 32;
    const double c1 = 0x1.ebfce50fac4f3p-3 / 32 / 32;
    const double c2 = 0x1.62e42ff0c52d6p-1 / 32;
    const double z = __builtin_fma(c0, r, c1);
    const double r2 = r * r;
    double y = __builtin_fma(c2, r, 1.0);
    y = __builtin_fma(z, r2, y);
    y = y * s;
    return (float)y;
}
OXE_HD float expf_c(float x) { return expf_t(x, kExp2fTab); }

// log1pf by the classic fdlibm single-precision method (s_log1pf.c, glibc <= 2.40): reduce
// 1+x = 2^k (1+f) with a correction term c for the rounding of 1+x, then
// log(1+f) = f - (hfsq - s*(hfsq + R)) with s = f/(2+f) and R a degree-7 polynomial in s^2.
// Evaluated in float without fused operations (the x86-64 C library build has none).
OXE_HD float log1pf_c(float x) {
    const float ln2_hi = u2f(0x3f317180u), ln2_lo = u2f(0x3717f7d1u);
    const float Lp1 = u2f(0x3F2AAAABu), Lp2 = u2f(0x3ECCCCCDu), Lp3 = u2f(0x3E924925u),
                Lp4 = u2f(0x3E638E29u), Lp5 = u2f(0x3E3A3325u), Lp6 = u2f(0x3E1CD04Fu),
                Lp7 = u2f(0x3E178897u);
    float hfsq, f = 0.0f, c = 0.0f, s, z, R, u;
    int32_t k, hu = 0;
    const int32_t hx = (int32_t)f2u(x);
    const int32_t ax = hx & 0x7fffffff;
    k = 1;
    if (hx < 0x3ed413d7) {                               // x < 0.41422
        if (ax >= 0x3f800000) {                          // x <= -1
            if (x == -1.0f) return -__builtin_inff();
            return (x - x) / (x - x);
        }
        if (ax < 0x31000000) {                           // |x| < 2^-29
            if (ax < 0x24800000) return x;               // |x| < 2^-54
            return x - x * x * 0.5f;
        }
        if (hx > 0 || hx <= (int32_t)0xbe95f61f) {       // -0.2929 < x < 0.41422
            k = 0; f = x; hu = 1;
        }
    } else if (hx >= 0x7f800000) {
        return x + x;
    }
    if (k != 0) {
        if (hx < 0x5a000000) {
            u = 1.0f + x;
            hu = (int32_t)f2u(u);
            k = (hu >> 23) - 127;
            c = (k > 0) ? 1.0f - (u - x) : x - (u - 1.0f);  // correction term
            c /= u;
        } else {
            u = x;
            hu = (int32_t)f2u(u);
            k = (hu >> 23) - 127;
            c = 0;
        }
        hu &= 0x007fffff;
        if (hu < 0x3504f7) {
            u = u2f((uint32_t)hu | 0x3f800000u);          // normalize u
        } else {
            k += 1;
            u = u2f((uint32_t)hu | 0x3f000000u);          // normalize u/2
            hu = (0x00800000 - hu) >> 2;
        }
        f = u - 1.0f;
    }
    hfsq = 0.5f * f * f;
    if (hu == 0) {                                        // |f| < 2^-20
        if (f == 0.0f) {
            if (k == 0) return 0.0f;
            c += k * ln2_lo;
            return k * ln2_hi + c;
        }
        R = hfsq * (1.0f - 0.66666666666666666f * f);
        if (k == 0) return f - R;
        return k * ln2_hi - ((R - (k * ln2_lo + c)) - f);
    }
    s = f / (2.0f + f);
    z = s * s;
    R = z * (Lp1 + z * (Lp2 + z * (Lp3 + z * (Lp4 + z * (Lp5 + z * (Lp6 + z * Lp7))))));
    if (k == 0) return f - (hfsq - s * (hfsq + R));
    return k * ln2_hi - ((hfsq - (s * (hfsq + R) + (k * ln2_lo + c))) - f);
}

}  // namespace oxe_libm
