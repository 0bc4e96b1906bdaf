// TEST INFRASTRUCTURE ONLY. The CPU oracle: a C++ restatement of the reference's CPU arithmetic for
// the MTP depth-1 decode step of n0rpan/snapdragon-engine (the `oxe` engine), in the reference's
// float order. Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it,
// and only as the checker (never as the thing measured or shipped).
//
// Every function cites the reference file:line it follows (paths relative to the reference root).
// Float semantics follow the aarch64 NEON build of the reference: vfmaq_f32 / vfmsq_f32 are fused,
// vaddvq_f32 is pairwise ((a0+a1)+(a2+a3)), fp16 vector FMAs round once to fp16, Rust scalar code
// is never contracted. This file is compiled with -ffp-contract=off and every fused operation is
// written as an explicit fmaf().
#pragma once
#include <stdint.h>
#include <stddef.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- fp16 <-> fp32 (simd-mappings.h / compat.h:37-50: __fp16 conversions, RNE)
float    oxo_f16_to_f32(uint16_t h);
uint16_t oxo_f32_to_f16(float f);
// IEEE binary16 fused multiply-add with one rounding (vfmaq_f16), and binary16 add (vaddq_f16)
uint16_t oxo_f16_fma(uint16_t a, uint16_t b, uint16_t c);
uint16_t oxo_f16_add(uint16_t a, uint16_t b);

// ---- Q8_0 activation quantizer, NEON branch (vendor/ggml-subset/generated/quants_subset.c:6-42)
// x[k] -> codes q[k] (int8) and per-32 block fp16 scales d[k/32]
void oxo_quantize_row_q8_0(const float *x, int64_t k, int8_t *q, uint16_t *d);
// dequantize_row_q8_0 (quants_base.c:64-78): y = q * f32(d)
void oxo_dequantize_row_q8_0(const int8_t *q, const uint16_t *d, int64_t k, float *y);

// ---- Q8_0 GEMV, NEON+dotprod branch of ggml_gemv_q8_0_4x8_q8_0 (repack_subset.cpp:1633-1679),
// also the lane GEMV contract of oxe_vl_gemv_q8_0 (crates/kernels-sys/csrc/oxe_vl_q80.inc:1-89).
// Weights: codes wq[nr][k] row-major + scales wd[nr][k/32]; nl activation lanes xq[nl][k], xd[nl][k/32].
// y[l*nr + r] = chain over blocks b ascending of fmaf(f32(isum_b), f32(xd_b) * f32(wd_rb), acc) from +0.
// isum (optional) receives the exact int32 block dots [nl][nr][k/32].
void oxo_gemv_q8_0(int64_t k, int64_t nr, int nl, const int8_t *wq, const uint16_t *wd,
                   const int8_t *xq, const uint16_t *xd, float *y, int32_t *isum);

// ---- K-quants (kquants.cpp): quantize_row_q8_K_ref (quants_base.c:14-48) into ggml block_q8_K
// (float d, int8 qs[256], int16 bsums[16]; 292 bytes); the lane GEMV contract of oxe_vl_gemv
// (crates/kernels-sys/csrc/oxe_vl.inc:78-107, oxe_vl_q{3,4,5,6}k.inc) per lane over ggml blocks:
// s[l*nr + r] = W[r] . y[l]; type 3 Q3_K, 4 Q4_K, 5 Q5_K, 6 Q6_K; returns 0 for another type.
void oxo_quantize_row_q8_K(const float *x, void *y, int64_t k);
int  oxo_vl_gemv(int type, int64_t k, int64_t nr, int nl, const void *w, const void *y, float *s);
// synthetic K-quant tensor bytes (ggml type 11..14, rows x k/256 blocks of expert `expert`) for the
// tests' model files; returns the bytes written or 0
// dequantize_row_q{3,4,5,6}_K as the reference builds it (types 11..14); 1, or 0 for another type
int oxo_dequantize_row_kq(int type, const void *x, float *y, int64_t k);
int64_t oxo_synth_kq(uint64_t seed, int layer, int kind, int type, int64_t expert, int64_t rows, int64_t k, uint8_t *out);

// ---- f32 / f16 vector helpers (vendor/ggml-subset/generated/upstream/src/ggml-cpu/vec.{h,cpp})
float oxo_vec_dot_f32(int n, const float *x, const float *y);            // vec.cpp:104-125
float oxo_vec_dot_f16(int n, const uint16_t *x, const uint16_t *y);      // vec.cpp:345-371
float oxo_v_expf(float x);                                               // vec.h:1154-1175
float oxo_v_silu(float x);                                               // vec.h:1178-1185
void  oxo_silu_f32(int n, float *y, const float *x);                     // vec.cpp:380-419
void  oxo_swiglu_f32(int n, float *y, const float *g, const float *u);   // vec.cpp:421-440
double oxo_vec_soft_max_f32(int n, float *y, const float *x, float max); // vec.cpp:625-697
float oxo_vec_sum_f32(int n, const float *x);                            // vec.h:1634-1644
float oxo_vec_max_f32(int n, const float *x);                            // vec.h:1680-1690

// ---- ported decode ops (crates/kernels-sys/csrc/oxe_ops.cpp)
void  oxo_rms_norm_f32(const float *x, float *y, int64_t n, float eps);                     // :19-28
void  oxo_rms_norm_mul_f32(const float *x, const float *w, float *y, int64_t n, float eps);  // :32-42
void  oxo_gdn_l2_norm_f32(float *x, int64_t n, float eps);                                  // :45-49
void  oxo_sigmoid_f32(int64_t n, float *y, const float *x);                                 // :80-84
void  oxo_softplus_f32(int64_t n, float *y, const float *x);                                // :85-89
void  oxo_soft_max_f32(int n, float *dp, const float *sp, float scale, const float *mask, float *wp); // :101-115
void  oxo_argsort_top_k_f32(const float *x, int n, int k, int32_t *out, int32_t *scratch, int *tie); // :121-165
void  oxo_ssm_conv_step_f32(float *state, const float *x_new, const float *c, int nr, int nc, float *out); // :175-201
void  oxo_gated_delta_net_step_f32_from(float *s_out, const float *s_in, const float *q, const float *k,
                                        const float *v, float g, float beta, int64_t S_v, float *attn); // :268-345
void  oxo_mrope_cache_init(int64_t p, const int32_t *sections, int is_imrope, int n_dims, int64_t ne0,
                           float freq_base, float freq_scale, float ext_factor, float attn_factor,
                           float beta_fast, float beta_slow, int n_ctx_orig, int truncate, float *cache); // :386-439
void  oxo_rope_neox_inplace(float *x, int n_dims, const float *cache);                      // :443-455
void  oxo_attn_head_f16(const float *q, const uint16_t *k, int64_t k_stride, const uint16_t *k_last,
                        const uint16_t *vt, int64_t v_stride, int n_kv, int pos_last, int head_dim,
                        float scale, float *out);                                             // :465-493

// test helper: host counterparts of the device's oxe_hip_eval_unary over float bit patterns
void  oxo_eval_unary(int fn, uint32_t start, int64_t n, int64_t stride, float *y);

#ifdef __cplusplus
}
#endif
