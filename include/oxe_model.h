/* Model description and synthetic-weight specification shared by the MI355X engine and its
 * checker. Plain C, no HIP types.
 *
 * oxe_model_desc mirrors the qwen35moe hyper-parameters the reference reads from GGUF metadata
 * (crates/model/src/desc.rs:15-140, ModelDesc::from_header); oxe_model_desc_35b_a3b() returns the
 * BASELINE "35B-A3B" shape (tests/fixtures/ornith.json of the reference, vocab 151936, all matmul
 * weights Q8_0).
 *
 * Synthetic weights (the benchmark has no checkpoint): every tensor is a pure function of
 * (seed, tensor uid, element index) through a counter-based generator, so the GPU and the CPU
 * oracle build identical 36 GB models independently:
 *   oxe_rng(key, i)   = splitmix64 output for counter i under `key`
 *   tensor key        = oxe_rng(seed, uid)
 *   Q8_0 codes        = uniform integers in [-127, 127]: 16-bit slice s of oxe_rng(key, i/4),
 *                       ((s * 255) >> 16) - 127
 *   Q8_0 fp16 scales  = fp16_rne(lo + u * (hi - lo)), u = (oxe_rng(key', i) >> 40) * 2^-24
 *   f32 "normal"      = mu + sigma * z, z = (sum of twelve 16-bit uniforms - 393210) / 65536
 *                       (Irwin-Hall: mean 0, variance 1, exact integer arithmetic)
 * All float steps are single IEEE operations with no fused multiply-add.
 */
#ifndef OXE_MODEL_H
#define OXE_MODEL_H
#include <stdint.h>

#if defined(__HIPCC__)
#define OXE_HDI __host__ __device__ static inline
#else
#define OXE_HDI static inline
#endif

#ifdef __cplusplus
extern "C" {
#endif

typedef struct oxe_model_desc {
    int32_t n_layer;          /* target layers (MTP block excluded) */
    int32_t n_embd;
    int32_t n_vocab;
    int32_t n_head, n_head_kv, head_dim;
    int32_t n_expert, n_expert_used, ff_exp, ff_shexp;
    int32_t ssm_conv_kernel, ssm_d_state, ssm_n_kheads, ssm_n_vheads, ssm_d_inner;
    int32_t full_attention_interval; /* layer il is attention iff (il + 1) % interval == 0 */
    int32_t n_rot;
    int32_t rope_sections[4];
    float rms_eps;
    float rope_freq_base;
    int32_t n_ctx_train;
    int32_t has_mtp;          /* one nextn block blk.{n_layer} */
} oxe_model_desc;

/* the BASELINE 35B-A3B shape (the reference's qwen35moe fixture with vocab 151936) */
OXE_HDI oxe_model_desc oxe_model_desc_35b_a3b(void) {
    oxe_model_desc d;
    d.n_layer = 40; d.n_embd = 2048; d.n_vocab = 151936;
    d.n_head = 16; d.n_head_kv = 2; d.head_dim = 256;
    d.n_expert = 256; d.n_expert_used = 8; d.ff_exp = 512; d.ff_shexp = 512;
    d.ssm_conv_kernel = 4; d.ssm_d_state = 128; d.ssm_n_kheads = 16; d.ssm_n_vheads = 32;
    d.ssm_d_inner = 4096; d.full_attention_interval = 4; d.n_rot = 64;
    d.rope_sections[0] = 11; d.rope_sections[1] = 11; d.rope_sections[2] = 10; d.rope_sections[3] = 0;
    d.rms_eps = 9.999999974752427e-07f; d.rope_freq_base = 10000000.0f; d.n_ctx_train = 262144;
    d.has_mtp = 1;
    return d;
}

/* tensor kinds of the synthetic model (uid = layer * 64 + kind; layer n_layer = MTP block,
 * layer 63 = global tensors) */
enum oxe_tensor_kind {
    OXE_T_ATTN_NORM = 0, OXE_T_POST_NORM = 1,
    OXE_T_DN_QKV = 2, OXE_T_DN_Z = 3, OXE_T_DN_BETA = 4, OXE_T_DN_ALPHA = 5, OXE_T_DN_CONV = 6,
    OXE_T_DN_A = 7, OXE_T_DN_DT = 8, OXE_T_DN_NORM = 9, OXE_T_DN_OUT = 10,
    OXE_T_ATT_Q = 11, OXE_T_ATT_K = 12, OXE_T_ATT_V = 13, OXE_T_ATT_QNORM = 14, OXE_T_ATT_KNORM = 15,
    OXE_T_ATT_OUT = 16,
    OXE_T_ROUTER = 17, OXE_T_SHEXP_GATE = 18, OXE_T_GATE_EXPS = 19, OXE_T_UP_EXPS = 20,
    OXE_T_DOWN_EXPS = 21, OXE_T_GATE_SHEXP = 22, OXE_T_UP_SHEXP = 23, OXE_T_DOWN_SHEXP = 24,
    OXE_T_EH_PROJ = 25, OXE_T_ENORM = 26, OXE_T_HNORM = 27, OXE_T_HEAD_NORM = 28,
    OXE_T_TOK_EMBD = 29, OXE_T_OUT_NORM = 30, OXE_T_OUTPUT = 31,
    OXE_T_SCALE_OFFSET = 32  /* scales of Q8_0 tensor kind t use uid + 32 */
};
#define OXE_GLOBAL_LAYER 63

/* Per-kind distribution parameters (Q8_0: fp16 scale range; f32: mu, sigma). */
typedef struct oxe_synth_param { float a, b; } oxe_synth_param;

OXE_HDI uint64_t oxe_rng(uint64_t key, uint64_t i) {
    uint64_t z = key + (i + 1) * 0x9e3779b97f4a7c15ULL;
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ULL;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebULL;
    return z ^ (z >> 31);
}

OXE_HDI uint64_t oxe_tensor_key(uint64_t seed, int layer, int kind) {
    return oxe_rng(seed, (uint64_t)(layer * 64 + kind));
}

OXE_HDI int8_t oxe_synth_code(uint64_t key, uint64_t i) {
    const uint64_t r = oxe_rng(key, i >> 2);
    const uint32_t s = (uint32_t)((r >> (16 * (i & 3))) & 0xffffu);
    return (int8_t)((int32_t)((s * 255u) >> 16) - 127);
}

/* float parts of the generator: u in [0,1) with 24 bits; z ~ Irwin-Hall(12) normalised */
OXE_HDI float oxe_synth_unit(uint64_t key, uint64_t i) {
    return (float)(oxe_rng(key, i) >> 40) * 5.9604644775390625e-08f;
}
OXE_HDI float oxe_synth_z(uint64_t key, uint64_t i) {
    int32_t s = 0;
    for (int j = 0; j < 3; j++) {
        const uint64_t r = oxe_rng(key, 3 * i + (uint64_t)j);
        s += (int32_t)(r & 0xffff) + (int32_t)((r >> 16) & 0xffff) + (int32_t)((r >> 32) & 0xffff) +
             (int32_t)((r >> 48) & 0xffff);
    }
    return (float)(s - 393210) * 1.52587890625e-05f;
}

/* float -> binary16, round to nearest even (subnormals, overflow to inf), integer-only so host
 * and device agree bit for bit */
OXE_HDI uint16_t oxe_f32_to_f16_rne(float f) {
    union { float f; uint32_t u; } v;
    v.f = f;
    const uint32_t x = v.u;
    const uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    const uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) return (uint16_t)(sign | 0x7e00u);
    if (ax >= 0x477ff000u) return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) {
        const uint32_t r = ax + 0x00000fffu + ((ax >> 13) & 1u);
        return (uint16_t)(sign | ((r - 0x38000000u) >> 13));
    }
    if (ax < 0x33000000u) return sign;
    const uint32_t e = ax >> 23, m = (ax & 0x7fffffu) | 0x800000u, sh = 126u - e;
    uint32_t q = m >> sh;
    const uint32_t rem = m & ((1u << sh) - 1u), half = 1u << (sh - 1u);
    if (rem > half || (rem == half && (q & 1u))) q++;
    return (uint16_t)(sign | q);
}

/* Distribution of each tensor kind: Q8_0 kinds -> fp16 scale range [a, b); OXE_T_DN_A -> uniform
 * [a, b); other f32 kinds -> a + b * z. Scales follow BASELINE (U(0.001, 0.02)); the beta/alpha
 * projections use a 10x smaller range so the gates are not saturated. */
OXE_HDI oxe_synth_param oxe_synth_param_of(int kind) {
    oxe_synth_param p;
    switch (kind) {
    case OXE_T_DN_BETA: case OXE_T_DN_ALPHA: p.a = 0.0001f; p.b = 0.002f; break;
    case OXE_T_DN_QKV: case OXE_T_DN_Z: case OXE_T_DN_OUT: case OXE_T_ATT_Q: case OXE_T_ATT_K:
    case OXE_T_ATT_V: case OXE_T_ATT_OUT: case OXE_T_GATE_EXPS: case OXE_T_UP_EXPS:
    case OXE_T_DOWN_EXPS: case OXE_T_GATE_SHEXP: case OXE_T_UP_SHEXP: case OXE_T_DOWN_SHEXP:
    case OXE_T_EH_PROJ: case OXE_T_TOK_EMBD: case OXE_T_OUTPUT: p.a = 0.001f; p.b = 0.02f; break;
    case OXE_T_ROUTER: case OXE_T_SHEXP_GATE: p.a = 0.0f; p.b = 0.02f; break;
    case OXE_T_DN_CONV: p.a = 0.0f; p.b = 0.25f; break;
    case OXE_T_DN_A: p.a = -2.0f; p.b = -0.5f; break;
    case OXE_T_DN_DT: p.a = 0.0f; p.b = 0.5f; break;
    default: p.a = 1.0f; p.b = 0.1f; break; /* norm weights */
    }
    return p;
}

OXE_HDI int oxe_kind_is_q8(int kind) {
    switch (kind) {
    case OXE_T_DN_QKV: case OXE_T_DN_Z: case OXE_T_DN_BETA: case OXE_T_DN_ALPHA: case OXE_T_DN_OUT:
    case OXE_T_ATT_Q: case OXE_T_ATT_K: case OXE_T_ATT_V: case OXE_T_ATT_OUT: case OXE_T_GATE_EXPS:
    case OXE_T_UP_EXPS: case OXE_T_DOWN_EXPS: case OXE_T_GATE_SHEXP: case OXE_T_UP_SHEXP:
    case OXE_T_DOWN_SHEXP: case OXE_T_EH_PROJ: case OXE_T_TOK_EMBD: case OXE_T_OUTPUT: return 1;
    default: return 0;
    }
}

/* fp16 scale of block `i` (flat over the tensor's [expert][row][k/32]) */
OXE_HDI uint16_t oxe_synth_scale(uint64_t skey, uint64_t i, oxe_synth_param p) {
    const float u = oxe_synth_unit(skey, i);
    const float span = p.b - p.a;
    const float t = u * span;
    return oxe_f32_to_f16_rne(p.a + t);
}

/* f32 tensor element `i` */
OXE_HDI float oxe_synth_f32(uint64_t key, uint64_t i, int kind) {
    const oxe_synth_param p = oxe_synth_param_of(kind);
    if (kind == OXE_T_DN_A) {
        const float span = p.b - p.a;
        const float t = oxe_synth_unit(key, i) * span;
        return p.a + t;
    }
    const float t = p.b * oxe_synth_z(key, i);
    return p.a + t;
}

#ifdef __cplusplus
}
#endif
#endif /* OXE_MODEL_H */
