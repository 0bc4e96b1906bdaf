// TEST INFRASTRUCTURE ONLY (see oxo.h). Kernel-level restatement of the reference's CPU ops in
// the float order of its aarch64 NEON build. Compiled with -ffp-contract=off: every fused
// multiply-add of the reference appears here as an explicit fmaf().
#include "oxo.h"

#include <algorithm>
#include <cfenv>
#include <cmath>
#include <cstring>

namespace {

inline uint32_t f2u(float f) { uint32_t u; memcpy(&u, &f, 4); return u; }
inline float u2f(uint32_t u) { float f; memcpy(&f, &u, 4); return f; }
inline uint64_t d2u(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }

// Round a double to binary16, round-to-nearest-even, with subnormals, overflow to inf.
uint16_t d_to_f16(double d) {
    uint16_t sign = std::signbit(d) ? 0x8000 : 0;
    if (std::isnan(d)) return (uint16_t)(sign | 0x7e00);
    double a = std::fabs(d);
    if (a >= 65520.0) return (uint16_t)(sign | 0x7c00);           // rounds to +-inf
    if (a < 6.103515625e-05) {                                     // below 2^-14: subnormal grid 2^-24
        double q = std::nearbyint(a * 16777216.0);                 // exact scaling, RNE
        return (uint16_t)(sign | (uint16_t)q);                     // q == 1024 encodes 2^-14
    }
    int ex;
    double m = std::frexp(a, &ex);                                 // a = m * 2^ex, m in [0.5, 1)
    double q = std::nearbyint(m * 2048.0);                         // 11 significant bits, RNE
    // value = q * 2^(ex - 11); biased exponent of 1.f*2^(ex-1) is ex - 1 + 15
    uint32_t bits = (uint32_t)((ex - 1 + 15) << 10) + (uint32_t)q - 1024u;  // q == 2048 carries
    return (uint16_t)(sign | bits);
}

// Exact error of s = fl(a + b) (Knuth TwoSum).
inline double two_sum_err(double a, double b, double s) {
    double bb = s - a;
    double aa = s - bb;
    return (a - aa) + (b - bb);
}

}  // namespace

extern "C" {

float oxo_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000) << 16;
    uint32_t e = (h >> 10) & 0x1f, m = h & 0x3ff;
    if (e == 0x1f) return u2f(sign | 0x7f800000u | (m << 13));
    if (e == 0) {
        // subnormal: exact value m * 2^-24
        float v = (float)m * 5.9604644775390625e-08f;
        return sign ? -v : v;
    }
    return u2f(sign | ((e + 112) << 23) | (m << 13));
}

// GGML_CPU_FP32_TO_FP16 on aarch64 = (__fp16) f: IEEE round-to-nearest-even (compat.h:44-50).
uint16_t oxo_f32_to_f16(float f) { return d_to_f16((double)f); }  // exact widening, one rounding

uint16_t oxo_f16_fma(uint16_t a, uint16_t b, uint16_t c) {
    double da = oxo_f16_to_f32(a), db = oxo_f16_to_f32(b), dc = oxo_f16_to_f32(c);
    double p = da * db;                        // exact: 11 x 11 significant bits
    double s = p + dc;
    if (!std::isfinite(s) || !std::isfinite(p)) return d_to_f16(s);
    double e = two_sum_err(p, dc, s);          // p + dc == s + e exactly
    // s is the exact sum rounded to double; only an exact binary16 midpoint can round the wrong
    // way, and then the sign of e decides: nudge s one double ulp toward the exact value.
    if (e != 0.0) s = std::nextafter(s, e > 0 ? INFINITY : -INFINITY);
    if (s == 0.0 && e == 0.0) {
        // exact zero: IEEE sign rules for x*y + z (round-to-nearest)
        if (p == 0.0 && dc == 0.0) return (std::signbit(p) && std::signbit(dc)) ? 0x8000 : 0x0000;
        return 0x0000;
    }
    return d_to_f16(s);
}

uint16_t oxo_f16_add(uint16_t a, uint16_t b) {
    double s = (double)oxo_f16_to_f32(a) + (double)oxo_f16_to_f32(b);  // exact for binary16 inputs
    if (s == 0.0) {
        bool na = (a & 0x8000) != 0, nb = (b & 0x8000) != 0;
        double za = oxo_f16_to_f32(a), zb = oxo_f16_to_f32(b);
        if (za == 0.0 && zb == 0.0) return (na && nb) ? 0x8000 : 0x0000;
        return 0x0000;
    }
    return d_to_f16(s);
}

// ---------------------------------------------------------------------------------------------
// quantize_row_q8_0, NEON branch (quants_subset.c:6-42): amax by vmaxq/vmaxvq (exact), d = amax/127
// (f32 division), id = d ? 1/d : 0 computed from the f32 d, d stored as fp16 (RNE), codes =
// vcvtnq_s32_f32(x * id): round to nearest, ties to even.
void oxo_quantize_row_q8_0(const float *x, int64_t k, int8_t *q, uint16_t *d) {
    const int64_t nb = k / 32;
    for (int64_t i = 0; i < nb; i++) {
        float amax = 0.0f;
        for (int j = 0; j < 32; j++) {
            float a = std::fabs(x[i * 32 + j]);
            amax = std::max(amax, a);   // vmaxq_f32: max of non-NaN magnitudes is order-free
        }
        const float dd = amax / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        d[i] = oxo_f32_to_f16(dd);
        for (int j = 0; j < 32; j++) {
            const float v = x[i * 32 + j] * id;
            q[i * 32 + j] = (int8_t)(int32_t)std::nearbyint(v);  // default rounding mode: RNE
        }
    }
}

void oxo_dequantize_row_q8_0(const int8_t *q, const uint16_t *d, int64_t k, float *y) {
    for (int64_t i = 0; i < k / 32; i++) {
        const float dd = oxo_f16_to_f32(d[i]);
        for (int j = 0; j < 32; j++) y[i * 32 + j] = (float)q[i * 32 + j] * dd;
    }
}

// ---------------------------------------------------------------------------------------------
// ggml_gemv_q8_0_4x8_q8_0, NEON + dotprod (repack_subset.cpp:1633-1679): for each row and block,
// isum = exact int32 dot of the 32 codes; acc = vfmaq_f32(acc, f32(isum), f32(d_x) * f32(d_w)).
// The lane GEMV (oxe_vl_q80.inc:25-89) forms the same integers and the same float updates per lane.
void oxo_gemv_q8_0(int64_t k, int64_t nr, int nl, const int8_t *wq, const uint16_t *wd,
                   const int8_t *xq, const uint16_t *xd, float *y, int32_t *isum) {
    const int64_t nb = k / 32;
#pragma omp parallel for schedule(static)
    for (int64_t r = 0; r < nr; r++) {
        const int8_t *w = wq + r * k;
        for (int l = 0; l < nl; l++) {
            const int8_t *x = xq + (int64_t)l * k;
            float acc = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                int32_t s = 0;
                for (int j = 0; j < 32; j++) s += (int32_t)w[b * 32 + j] * (int32_t)x[b * 32 + j];
                const float prod = oxo_f16_to_f32(xd[(int64_t)l * nb + b]) * oxo_f16_to_f32(wd[r * nb + b]);
                acc = std::fma((float)s, prod, acc);
                if (isum) isum[((int64_t)l * nr + r) * nb + b] = s;
            }
            y[(int64_t)l * nr + r] = acc;
        }
    }
}

// ---------------------------------------------------------------------------------------------
// ggml_vec_dot_f32, NEON (vec.cpp:104-125 with simd-mappings.h:358-395): GGML_F32_STEP 16,
// GGML_F32_EPR 4, 4 accumulators: element i+4a+l of each 16-step goes to lane l of accumulator a,
// vfmaq_f32; reduce a0+=a2, a1+=a3, a0+=a1, then vaddvq_f32 = (l0+l1)+(l2+l3); leftovers
// sumf += x*y (contracted by the C build).
float oxo_vec_dot_f32(int n, const float *x, const float *y) {
    const int np = n & ~15;
    float acc[4][4] = {};
    for (int i = 0; i < np; i += 16)
        for (int a = 0; a < 4; a++)
            for (int l = 0; l < 4; l++) acc[a][l] = std::fma(x[i + 4 * a + l], y[i + 4 * a + l], acc[a][l]);
    float r[4];
    for (int l = 0; l < 4; l++) {
        float a0 = acc[0][l] + acc[2][l];
        float a1 = acc[1][l] + acc[3][l];
        r[l] = a0 + a1;
    }
    float sumf = (r[0] + r[1]) + (r[2] + r[3]);
    for (int i = np; i < n; i++) sumf = std::fma(x[i], y[i], sumf);
    return sumf;
}

// ggml_vec_dot_f16, NEON with FP16 vector arithmetic (vec.cpp:345-371, simd-mappings.h:400-429):
// GGML_F16_STEP 32, EPR 8, 4 accumulators of 8 fp16 lanes, vfmaq_f16 (one fp16 rounding);
// GGML_F16x8_REDUCE: a0+=a2, a1+=a3, a0+=a1 in fp16, widen, t0+t1 (f32), vaddvq pairwise;
// sumf (double) += leftovers; store (float)sumf.
float oxo_vec_dot_f16(int n, const uint16_t *x, const uint16_t *y) {
    const int np = n & ~31;
    uint16_t acc[4][8] = {};
    for (int i = 0; i < np; i += 32)
        for (int j = 0; j < 4; j++)
            for (int l = 0; l < 8; l++) acc[j][l] = oxo_f16_fma(x[i + 8 * j + l], y[i + 8 * j + l], acc[j][l]);
    double sumf = 0.0;
    {
        uint16_t a0[8], a1[8];
        for (int l = 0; l < 8; l++) {
            a0[l] = oxo_f16_add(acc[0][l], acc[2][l]);
            a1[l] = oxo_f16_add(acc[1][l], acc[3][l]);
        }
        for (int l = 0; l < 8; l++) a0[l] = oxo_f16_add(a0[l], a1[l]);
        float u[4];
        for (int l = 0; l < 4; l++) u[l] = oxo_f16_to_f32(a0[l]) + oxo_f16_to_f32(a0[l + 4]);
        sumf = (double)((u[0] + u[1]) + (u[2] + u[3]));
    }
    for (int i = np; i < n; i++) sumf += (double)(oxo_f16_to_f32(x[i]) * oxo_f16_to_f32(y[i]));
    return (float)sumf;
}

// ggml_v_expf, NEON (vec.h:1154-1175); vfmaq_f32(a,b,c) = a + b*c, vfmsq_f32(a,b,c) = a - b*c.
float oxo_v_expf(float x) {
    const float r = 0x1.8p23f;
    const float z = std::fma(x, 0x1.715476p+0f, r);
    const float n = z - r;
    const float b = std::fma(-n, 0x1.7f7d1cp-20f, std::fma(-n, 0x1.62e4p-1f, x));
    const uint32_t e = f2u(z) << 23;
    const float k = u2f(e + f2u(1.0f));
    const bool c = std::fabs(n) > 126.0f;
    const float u = b * b;
    const float j = std::fma(std::fma(std::fma(0x1.0e4020p-7f, b, 0x1.573e2ep-5f), u,
                                      std::fma(0x1.555e66p-3f, b, 0x1.fffdb6p-2f)),
                             u, 0x1.ffffecp-1f * b);
    if (!c) return std::fma(j, k, k);
    const uint32_t d = (n <= 0.0f) ? 0x82000000u : 0u;
    const float s1 = u2f(d + 0x7f000000u);
    const float s2 = u2f(e - d);
    if (std::fabs(n) > 192.0f) return s1 * s1;
    return std::fma(s2, j, s2) * s1;
}

// ggml_v_silu (vec.h:1178-1185): x / (1 + v_expf(0 - x))
float oxo_v_silu(float x) { return x / (1.0f + oxo_v_expf(0.0f - x)); }

// ggml_vec_silu_f32 NEON (vec.cpp:380-419): groups of 4 through ggml_v_silu; the scalar tail is
// ggml_silu_f32 = x/(1+expf(-x)) with the C library's expf.
void oxo_silu_f32(int n, float *y, const float *x) {
    const int n4 = n & ~3;
    int i = 0;
    for (; i < n4; i++) y[i] = oxo_v_silu(x[i]);
    for (; i < n; i++) y[i] = x[i] / (1.0f + expf(-x[i]));
}

// ggml_vec_swiglu_f32 NEON (vec.cpp:421-440): vmulq_f32(ggml_v_silu(g), u)
void oxo_swiglu_f32(int n, float *y, const float *g, const float *u) {
    const int n4 = n & ~3;
    int i = 0;
    for (; i < n4; i++) y[i] = oxo_v_silu(g[i]) * u[i];
    for (; i < n; i++) y[i] = (g[i] / (1.0f + expf(-g[i]))) * u[i];
}

// ggml_vec_soft_max_f32 NEON (vec.cpp:625-697): groups of 4: val = v_expf(x - max), sum (double)
// += vaddvq(val) = (v0+v1)+(v2+v3); tail: expf (C library).
double oxo_vec_soft_max_f32(int n, float *y, const float *x, float max) {
    int i = 0;
    double sum = 0.0;
    for (; i + 3 < n; i += 4) {
        float v[4];
        for (int l = 0; l < 4; l++) { v[l] = oxo_v_expf(x[i + l] - max); y[i + l] = v[l]; }
        sum += (double)((v[0] + v[1]) + (v[2] + v[3]));
    }
    for (; i < n; ++i) {
        float val = expf(x[i] - max);
        sum += (double)val;
        y[i] = val;
    }
    return sum;
}

float oxo_vec_sum_f32(int n, const float *x) {
    double sum = 0.0;
    for (int i = 0; i < n; ++i) sum += (double)x[i];
    return (float)sum;
}

float oxo_vec_max_f32(int n, const float *x) {
    float max = -INFINITY;
    for (int i = 0; i < n; ++i) max = (max > x[i]) ? max : x[i];   // MAX(a,b) macro
    return max;
}

// ---------------------------------------------------------------------------------------------
// oxe_ops.cpp

void oxo_rms_norm_f32(const float *x, float *y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; i++) y[i] = x[i] * scale;   // memcpy + ggml_vec_scale_f32
}

void oxo_rms_norm_mul_f32(const float *x, const float *w, float *y, int64_t n, float eps) {
    double sum = 0.0;
    for (int64_t i = 0; i < n; i++) sum += (double)(x[i] * x[i]);
    const float mean = (float)(sum / (double)n);
    const float scale = 1.0f / sqrtf(mean + eps);
    for (int64_t i = 0; i < n; i++) y[i] = (x[i] * scale) * w[i];
}

void oxo_gdn_l2_norm_f32(float *x, int64_t n, float eps) {
    const float nf = (float)n;
    oxo_rms_norm_f32(x, x, n, eps / nf);
    const float s = 1.0f / sqrtf(nf);
    for (int64_t i = 0; i < n; i++) x[i] = x[i] * s;
}

// unary-ops op_sigmoid (oxe_ops.cpp:80-84): the C library's expf
void oxo_sigmoid_f32(int64_t n, float *y, const float *x) {
    for (int64_t i = 0; i < n; i++) y[i] = 1.f / (1.f + expf(-x[i]));
}

void oxo_softplus_f32(int64_t n, float *y, const float *x) {
    for (int64_t i = 0; i < n; i++) y[i] = (x[i] > 20.0f) ? x[i] : log1pf(expf(x[i]));
}

// oxe_soft_max_f32 (oxe_ops.cpp:101-115): wp = sp*scale (+ slope*mask, slope 1), max, exp/sum,
// dp *= (float)(1.0/sum).
void oxo_soft_max_f32(int n, float *dp, const float *sp, float scale, const float *mask, float *wp) {
    for (int i = 0; i < n; i++) wp[i] = sp[i] * scale;
    if (mask)
        for (int i = 0; i < n; i++) wp[i] = std::fma(1.0f, mask[i], wp[i]);   // wp += slope*mask
    const float max = oxo_vec_max_f32(n, wp);
    double sum = oxo_vec_soft_max_f32(n, dp, wp, max);
    sum = 1.0 / sum;
    const float s = (float)sum;
    for (int i = 0; i < n; i++) dp[i] = dp[i] * s;
}

// oxe_argsort_top_k_f32 (oxe_ops.cpp:121-165): fast selection when the k+1 largest values are
// distinct (and distinct from the rest); else std::sort of all indices, descending. `tie` (optional)
// is set to 1 when the sort path was taken.
void oxo_argsort_top_k_f32(const float *x, int n, int k, int32_t *out, int32_t *scratch, int *tie) {
    const int kk = std::min(n, k + 1);
    int m = 0;
    for (int i = 0; i < n; i++) {
        const float v = x[i];
        if (m == kk && !(v > x[scratch[m - 1]])) continue;
        int j = (m < kk) ? m++ : kk - 1;
        while (j > 0 && v > x[scratch[j - 1]]) { scratch[j] = scratch[j - 1]; j--; }
        scratch[j] = i;
    }
    bool ties = false;
    for (int j = 1; j < m; j++) ties |= !(x[scratch[j - 1]] > x[scratch[j]]);
    if (m == kk && kk == k + 1) {
        const float t = x[scratch[k]];
        int eq = 0;
        for (int i = 0; i < n; i++) { eq += (x[i] == t); ties |= std::isnan(x[i]); }
        ties |= eq != 1;
    }
    if (tie) *tie = ties ? 1 : 0;
    if (!ties) {
        for (int j = 0; j < k; j++) out[j] = scratch[j];
        return;
    }
    for (int j = 0; j < n; j++) scratch[j] = j;
    std::sort(scratch, scratch + n, [x](int32_t a, int32_t b) { return x[a] > x[b]; });
    for (int j = 0; j < k; j++) out[j] = scratch[j];
}

// oxe_ssm_conv_step_f32 (oxe_ops.cpp:175-201): blocks of 4 products added in order to sumf (no
// fusion), fmaf tail for nc % 4; then the state shifts.
void oxo_ssm_conv_step_f32(float *state, const float *x_new, const float *c, int nr, int nc, float *out) {
    float s[16];
    for (int i1 = 0; i1 < nr; ++i1) {
        float *st = state + (int64_t)i1 * (nc - 1);
        for (int i0 = 0; i0 < nc - 1; ++i0) s[i0] = st[i0];
        s[nc - 1] = x_new[i1];
        const float *ci = c + (int64_t)i1 * nc;
        float sumf = 0.0f;
        int i0 = 0;
        for (; i0 + 4 <= nc; i0 += 4) {
            float p[4];
            for (int l = 0; l < 4; l++) p[l] = s[i0 + l] * ci[i0 + l];
            sumf = sumf + p[0];
            sumf = sumf + p[1];
            sumf = sumf + p[2];
            sumf = sumf + p[3];
        }
        for (; i0 < nc; ++i0) sumf = std::fma(s[i0], ci[i0], sumf);
        out[i1] = sumf;
        for (int kk = 0; kk < nc - 1; ++kk) st[kk] = s[kk + 1];
    }
}

// oxe_gated_delta_net_step_f32_x4_from (oxe_ops.cpp:268-345), bitwise the reference step
// (oxe_ops.cpp:207-251): per state row j (s[j*S_v + i] = S[i][j]): row *= e^g; sum = dot(row, k)
// (ggml_vec_dot_f32 order); delta = (v_j - sum) * beta; row = fma(k, delta, row); out_j =
// dot(row, q) * (1/sqrt(S_v)). s_in == s_out is the in-place step.
void oxo_gated_delta_net_step_f32_from(float *s_out, const float *s_in, const float *q, const float *k,
                                       const float *v, float g, float beta, int64_t S_v, float *attn) {
    const float scale = 1.0f / sqrtf((float)S_v);
    const float eg = expf(g);
    for (int64_t j = 0; j < S_v; j++) {
        float *row = s_out + j * S_v;
        const float *rin = s_in + j * S_v;
        for (int64_t i = 0; i < S_v; i++) row[i] = rin[i] * eg;
        const float s1 = oxo_vec_dot_f32((int)S_v, row, k);
        const float delta = (v[j] - s1) * beta;
        for (int64_t i = 0; i < S_v; i++) row[i] = std::fma(k[i], delta, row[i]);
        const float s2 = oxo_vec_dot_f32((int)S_v, row, q);
        attn[j] = s2 * scale;
    }
}

// ---- RoPE (oxe_ops.cpp:357-455). The cache uses the C library's powf/logf/cosf/sinf.
static float rope_yarn_corr_dim(int n_dims, int n_ctx_orig, float n_rot, float base) {
    return n_dims * logf(n_ctx_orig / (n_rot * 2 * (float)M_PI)) / (2 * logf(base));
}

void oxo_mrope_cache_init(int64_t p, const int32_t *sections_in, int is_imrope, int n_dims, int64_t ne0,
                          float freq_base, float freq_scale, float ext_factor, float attn_factor,
                          float beta_fast, float beta_slow, int n_ctx_orig, int truncate, float *cache) {
    int sections[4] = {sections_in[0], sections_in[1], sections_in[2], sections_in[3]};
    const float theta_scale = powf(freq_base, -2.0f / n_dims);
    float corr_dims[2];
    {
        float start = rope_yarn_corr_dim(n_dims, n_ctx_orig, beta_fast, freq_base);
        float end = rope_yarn_corr_dim(n_dims, n_ctx_orig, beta_slow, freq_base);
        if (truncate) { start = floorf(start); end = ceilf(end); }
        corr_dims[0] = std::max(0.0f, start);
        corr_dims[1] = std::min((float)(n_dims - 1), end);
    }
    float theta_t = (float)p, theta_h = (float)p, theta_w = (float)p, theta_e = 0.0f;
    const int sect_dims = sections[0] + sections[1] + sections[2] + sections[3];
    const int sec_w = sections[1] + sections[0];
    for (int64_t i0 = 0; i0 < ne0; i0 += 2) {
        const int sector = (int)((i0 / 2) % sect_dims);
        float theta = theta_t;
        if (is_imrope) {
            if (sector % 3 == 1 && sector < 3 * sections[1]) theta = theta_h;
            else if (sector % 3 == 2 && sector < 3 * sections[2]) theta = theta_w;
            else if (sector % 3 == 0 && sector < 3 * sections[0]) theta = theta_t;
            else theta = theta_e;
        } else {
            if (sector >= sections[0] && sector < sec_w) theta = theta_h;
            else if (sector >= sec_w && sector < sec_w + sections[2]) theta = theta_w;
            else if (sector >= sec_w + sections[2]) theta = theta_e;
        }
        // rope_yarn (oxe_ops.cpp:372-382), freq_factors = NULL
        float theta_interp = freq_scale * theta;
        float th = theta_interp;
        float mscale = attn_factor;
        if (ext_factor != 0.0f) {
            const float y = ((float)(i0 / 2) - corr_dims[0]) / std::max(0.001f, corr_dims[1] - corr_dims[0]);
            const float ramp = 1 - std::min(1.0f, std::max(0.0f, y));
            const float ramp_mix = ramp * ext_factor;
            th = theta_interp * (1 - ramp_mix) + theta * ramp_mix;
            mscale *= 1.0f + 0.1f * logf(1.0f / freq_scale);
        }
        cache[i0 + 0] = cosf(th) * mscale;
        cache[i0 + 1] = sinf(th) * mscale;
        theta_t *= theta_scale;
        theta_w *= theta_scale;
        theta_h *= theta_scale;
        theta_e *= theta_scale;
    }
}

// rotate_pairs (oxe_ops.cpp:443-455). The fused form of x0*c - x1*s is the C compiler's choice on
// the reference machine; this restatement fuses the first product of each expression (GCC's
// convert_mult_to_fma visits the first multiplication first): fma(x0, c, -(x1*s)) and
// fma(x0, s, x1*c).
void oxo_rope_neox_inplace(float *x, int n_dims, const float *cache) {
    const int64_t n_offset = n_dims / 2;
    for (int64_t i0 = 0; i0 < n_dims; i0 += 2) {
        const int64_t ic = i0 / 2;
        const float c = cache[i0 + 0], s = cache[i0 + 1];
        float *src = x + ic;
        const float x0 = src[0], x1 = src[n_offset];
        src[0] = std::fma(x0, c, -(x1 * s));
        src[n_offset] = std::fma(x0, s, x1 * c);
    }
}

// oxe_attn_head_f16 (oxe_ops.cpp:465-493): FA-off single-query attention for one head over n_kv
// (padded) positions, causal mask at pos_last, K row pos_last from k_last.
void oxo_attn_head_f16(const float *q, const uint16_t *k, int64_t k_stride, const uint16_t *k_last,
                       const uint16_t *vt, int64_t v_stride, int n_kv, int pos_last, int head_dim,
                       float scale, float *out) {
    uint16_t q16[512];
    for (int i = 0; i < head_dim; i++) q16[i] = oxo_f32_to_f16(q[i]);
    float *kq = new float[n_kv], *mask = new float[n_kv], *wp = new float[n_kv];
    uint16_t *p16 = new uint16_t[n_kv];
    for (int p = 0; p < n_kv; p++) {
        if (p <= pos_last) {
            const uint16_t *kr = p == pos_last ? k_last : k + (int64_t)p * k_stride;
            kq[p] = oxo_vec_dot_f16(head_dim, kr, q16);
            mask[p] = 0.0f;
        } else {
            kq[p] = 0.0f;
            mask[p] = -INFINITY;
        }
    }
    oxo_soft_max_f32(n_kv, kq, kq, scale, mask, wp);
    for (int p = 0; p < n_kv; p++) p16[p] = oxo_f32_to_f16(kq[p]);
    for (int d = 0; d < head_dim; d++) out[d] = oxo_vec_dot_f16(n_kv, vt + (int64_t)d * v_stride, p16);
    delete[] kq; delete[] mask; delete[] wp; delete[] p16;
}

// Test helper: the host-side counterparts of oxe_hip_eval_unary (0 the C library's expf, 1 its
// log1pf, 2 oxo_v_expf, 3 sigmoid, 4 softplus, 5 oxo_v_silu) over float bit patterns start + i*stride.
void oxo_eval_unary(int fn, uint32_t start, int64_t n, int64_t stride, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; i++) {
        const float x = u2f((uint32_t)(start + (uint64_t)i * (uint64_t)stride));
        float r;
        switch (fn) {
            case 0: r = expf(x); break;
            case 1: r = log1pf(x); break;
            case 2: r = oxo_v_expf(x); break;
            case 3: oxo_sigmoid_f32(1, &r, &x); break;
            case 4: oxo_softplus_f32(1, &r, &x); break;
            default: r = oxo_v_silu(x); break;
        }
        y[i] = r;
    }
}

}  // extern "C"
