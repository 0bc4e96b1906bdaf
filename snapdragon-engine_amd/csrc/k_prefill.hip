// Batched prefill (Engine::prefill / prefill_nextn, crates/model/src/engine/prefill.rs:752-773): the
// prompt's tokens go through each layer together, the weight matrices as int8 matrix-core GEMMs
// (k_gemm.hip, bitwise equal to the decode GEMV for Q8_0), everything else as token-parallel
// kernels in the decode's float order. The recurrences (conv window, delta-rule state) run token
// by token; each attention query sees exactly the positions a single-token step at its position
// sees. So the KV cache, the recurrent state, every position's h_nextn and the last token's logits
// are the bits of token-by-token decoding, which is what the reference's batched prefill gives
// for Q8_0 weights (docs/lab-notes/M3-PREFILL.md:55-75). The recurrent state is read from and
// written back to the engine's current slot.
//
// Also the batched MTP KV seeding (MtpDriver::flush of many pairs, mtp.rs:425-446): eh_proj entry
// and the MTP layer's K / V rows for all pending (token, h) pairs in one pass.
#include <algorithm>
#include <vector>

#include "oxe_engine_host.h"
#include "oxe_gemm.h"
#include "oxe_prologue.h"
#include "oxe_route.h"
#include "oxe_shape.h"

namespace oxe {

using namespace shp;

namespace pf {

// ---- per-token norm + Q8_0 (the decode prologue for T rows) ---------------------------------
// row t: y = rms_norm(x_t) * w (oxe_ops.cpp:32-42); codes / scales to xq / xd (row stride xq_ld
// bytes, xq_ld / 32 scales); optional f32 y to xn. toks (optional): x_t is the token's embedding,
// stored to x first (the residual of layer 0, the replay source of the norm).
__global__ __launch_bounds__(PT) void norm_quant_kernel(Q8W emb, const uint32_t *toks, float *x, const float *w, float eps,
                                                        int8_t *xq, uint16_t *xd, int64_t xq_ld, float *xn) {
    __shared__ NormScratch ns;
    const int64_t t = blockIdx.x;
    float v[EPT];
    float *xr = x + t * E;
    if (toks) {
        embed8(emb, toks[t], v);
        store8(xr, v);
        __syncthreads();
    } else {
        load8(xr, v);
    }
    rms_norm_mul_e(v, xr, w, eps, ns);
    quant8(v, xq + t * xq_ld + EPT * threadIdx.x, xd + t * (xq_ld / 32) + (EPT * threadIdx.x) / 32);
    if (xn) store8(xn + t * E, v);
}

// ---- delta-net -----------------------------------------------------------------------------
// causal conv + silu (oxe_ssm_conv_step_f32, oxe_ops.cpp:175-201, nc = 4): the window of token t is
// (x_{t-3}, x_{t-2}, x_{t-1}, x_t), the positions before the chunk from the layer's state, so every
// (token, channel) is independent; the four products are rounded, then added in order to +0.
OXE_DEV float conv4_pf(float s0, float s1, float s2, float xn, const float *c) {
    const float p0 = s0 * c[0], p1 = s1 * c[1], p2 = s2 * c[2], p3 = xn * c[3];
    float sumf = 0.0f;
    sumf = sumf + p0;
    sumf = sumf + p1;
    sumf = sumf + p2;
    sumf = sumf + p3;
    return sumf;
}
__global__ __launch_bounds__(256) void conv_kernel(const float *proj, int T, const float *conv_w, const float *state,
                                                   float *cy) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    const int64_t t = blockIdx.y;
    float cw[KC];
#pragma unroll
    for (int i = 0; i < KC; i++) cw[i] = conv_w[(int64_t)c * KC + i];
    const float *st = state + (int64_t)c * (KC - 1);
    float s[KC];
#pragma unroll
    for (int i = 0; i < KC; i++) {
        const int64_t tt = t - (KC - 1) + i;   // token of window slot i (< 0: the state's slot tt + 3)
        s[i] = tt >= 0 ? proj[tt * DN_ROWS + c] : st[tt + (KC - 1)];
    }
    cy[t * NCH + c] = v_silu(conv4_pf(s[0], s[1], s[2], s[3], cw));
}
// the window after the chunk: the last three inputs (for T < 3 partly the older state)
__global__ __launch_bounds__(256) void conv_state_kernel(const float *proj, int T, float *state) {
    const int c = blockIdx.x * 256 + threadIdx.x;
    float *st = state + (int64_t)c * (KC - 1);
    float n[KC - 1];
#pragma unroll
    for (int i = 0; i < KC - 1; i++) {
        const int tt = T - (KC - 1) + i;   // token of new slot i (< 0: old slot tt + 3)
        n[i] = tt >= 0 ? proj[(int64_t)tt * DN_ROWS + c] : st[tt + (KC - 1)];
    }
#pragma unroll
    for (int i = 0; i < KC - 1; i++) st[i] = n[i];
}

// l2 norms of q and k (oxe_gdn_l2_norm_f32: rms_norm with eps/n, then * 1/sqrt(n)), one wave per
// (token, key head, q|k), in place; the gates of (token, value head) (engine.rs:2509-2524)
__global__ __launch_bounds__(256) void dn_prep_kernel(float *cy, const float *proj, const float *dt_bias,
                                                      const float *ssm_a, float eps, float *gg, float *gb) {
    const int64_t t = blockIdx.x;
    const int w = blockIdx.y * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;   // 0..31
    const int kh = w >> 1;
    float *xv = cy + t * NCH + ((w & 1) ? NKH * DS : 0) + kh * DS;
    const float a0 = xv[lane], a1 = xv[lane + 64];
    const float nf = (float)DS;
    const float mean = wave_mean_sq_128(a0, a1, xv);
    const float scale = 1.0f / sqrtf(mean + eps / nf);
    const float sq = 1.0f / sqrtf(nf);
    const float o0 = (a0 * scale) * sq, o1 = (a1 * scale) * sq;
    xv[lane] = o0;
    xv[lane + 64] = o1;
    if (blockIdx.y == 0 && threadIdx.x < NVH) {
        const int vh = threadIdx.x;
        const float ab = proj[t * DN_ROWS + DN_ALPHA + vh] + dt_bias[vh];
        gg[t * NVH + vh] = oxe_libm::expf_c(softplus_c(ab) * ssm_a[vh]);
        gb[t * NVH + vh] = sigmoid_c(proj[t * DN_ROWS + DN_BETA + vh]);
    }
}

// delta rule (oxe_gated_delta_net_step_f32_x4_from, oxe_ops.cpp:268-345) over the T tokens in order.
// Workgroup = (value head vh = b / 8, state rows 16 (b % 8) ..); thread (row rg = t / 16, chain
// c = t % 16) holds row elements c + 16 s in registers: chain c of ggml_vec_dot_f32, whose NEON
// reduction tree is the DPP sequence of dot16_tree_dpp. The token inputs (q, k, the 16 v rows,
// gates) are staged through LDS DT_T tokens at a time, double-buffered: the next stage's global
// loads are in flight while the current stage runs, and each token's q / k values are read from
// LDS one token ahead. o[t][vh * 128 + row] = (S_row . q) / sqrt(128).
constexpr int DT_T = 32;
__global__ __launch_bounds__(256) void delta_kernel(const float *cy, const float *gg, const float *gb, float *ssm, float *o,
                                                    int T) {
    // q and k of a token, transposed per chain: [q|k][c][s] = element c + 16 s (a lane's 8 values are
    // two 16-byte reads)
    __shared__ __align__(16) float s_qk[2][DT_T][2][16][8];
    __shared__ float s_v[2][DT_T][16], s_g[2][DT_T], s_b[2][DT_T], s_out[2][DT_T][16];
    __shared__ float s_junk[256];   // the output stores of the chains other than chain 0
    const int vh = blockIdx.x >> 3, row0 = (blockIdx.x & 7) * 16, kh = vh % NKH;
    const int t = threadIdx.x, rg = t >> 4, cc = t & 15;
    float *srow = ssm + ((int64_t)vh * HV + row0 + rg) * HV;
    float r[8];
#pragma unroll
    for (int s = 0; s < 8; s++) r[s] = srow[cc + 16 * s];
    const float scale = 1.0f / sqrtf((float)HV);
    // this thread's share of a stage: element t of every token's [q | k], and two v values
    const int64_t qk_off = t < DS ? kh * DS + t : NKH * DS + kh * DS + (t - DS);
    const int vt0 = t >> 4, ve = t & 15;   // v: tokens vt0 and vt0 + 16, row row0 + ve
    const int64_t v_off = 2 * NKH * DS + vh * HV + row0 + ve;
    float pf[DT_T], pv[2], pg = 0.0f, pb = 0.0f;
    auto fetch = [&](int t0) {
        const int nt = T - t0 < DT_T ? T - t0 : DT_T;
#pragma unroll
        for (int j = 0; j < DT_T; j++) pf[j] = j < nt ? cy[(int64_t)(t0 + j) * NCH + qk_off] : 0.0f;
#pragma unroll
        for (int j = 0; j < 2; j++) pv[j] = vt0 + 16 * j < nt ? cy[(int64_t)(t0 + vt0 + 16 * j) * NCH + v_off] : 0.0f;
        if (t < nt) {
            pg = gg[(int64_t)(t0 + t) * NVH + vh];
            pb = gb[(int64_t)(t0 + t) * NVH + vh];
        }
    };
    auto put = [&](int buf) {
#pragma unroll
        for (int j = 0; j < DT_T; j++) s_qk[buf][j][t >> 7][t & 15][(t >> 4) & 7] = pf[j];
#pragma unroll
        for (int j = 0; j < 2; j++) s_v[buf][vt0 + 16 * j][ve] = pv[j];
        if (t < DT_T) {
            s_g[buf][t] = pg;
            s_b[buf][t] = pb;
        }
    };
    fetch(0);
    put(0);
    __syncthreads();
    int buf = 0;
    for (int t0 = 0; t0 < T; t0 += DT_T, buf ^= 1) {
        const int nt = T - t0 < DT_T ? T - t0 : DT_T;
        const bool more = t0 + DT_T < T;
        if (more) fetch(t0 + DT_T);
        auto ld8 = [&](const float *p, float v[8]) {
            const float4 a = *(const float4 *)p, b = *(const float4 *)(p + 4);
            v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
        };
        // g, beta, v of a token, read with its q / k one token ahead
        auto gbv = [&](int tt, float &eg, float &beta, float &vv) {
            eg = s_g[buf][tt];
            beta = s_b[buf][tt];
            vv = s_v[buf][tt][rg];
        };
        auto step = [&](int tt, const float kc[8], const float qc[8], float eg, float beta, float vv) {
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                r[s] = r[s] * eg;
                acc = __builtin_fmaf(r[s], kc[s], acc);
            }
            const float sk = dot16_tree_dpp(acc);
            const float delta = (vv - sk) * beta;
            acc = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                r[s] = __builtin_fmaf(kc[s], delta, r[s]);
                acc = __builtin_fmaf(r[s], qc[s], acc);
            }
            const float sq = dot16_tree_dpp(acc);
            // every chain stores (chain 0 the row's output), so no branch splits the token loop and
            // this token's output dot overlaps the next token's recurrence
            float *dst = cc == 0 ? &s_out[buf][tt][rg] : &s_junk[t];
            *dst = sq * scale;
        };
        // tokens in pairs, each token's q / k read from LDS while the previous one runs
        float ka[8], qa[8], kb[8], qb[8], ga, ba, va, gb2, bb, vb;
        ld8(s_qk[buf][0][0][cc], qa);
        ld8(s_qk[buf][0][1][cc], ka);
        gbv(0, ga, ba, va);
        // tokens tt, tt + 1 without a branch inside
        auto pair = [&](int tt) {
            const int t1 = tt + 1, t2 = tt + 2 < DT_T ? tt + 2 : DT_T - 1;
            ld8(s_qk[buf][t1][0][cc], qb);
            ld8(s_qk[buf][t1][1][cc], kb);
            gbv(t1, gb2, bb, vb);
            step(tt, ka, qa, ga, ba, va);
            ld8(s_qk[buf][t2][0][cc], qa);
            ld8(s_qk[buf][t2][1][cc], ka);
            gbv(t2, ga, ba, va);
            step(tt + 1, kb, qb, gb2, bb, vb);
        };
        if (nt == DT_T) {
            // a whole stage unrolled (every LDS address a constant offset), each token's operands
            // read two tokens ahead (three register sets in rotation)
            float qs[3][8], ks[3][8], gs[3], bs[3], vs[3];
#pragma unroll
            for (int i = 0; i < 8; i++) { qs[0][i] = qa[i]; ks[0][i] = ka[i]; }
            gs[0] = ga; bs[0] = ba; vs[0] = va;
            ld8(s_qk[buf][1][0][cc], qs[1]);
            ld8(s_qk[buf][1][1][cc], ks[1]);
            gbv(1, gs[1], bs[1], vs[1]);
#pragma unroll
            for (int tt = 0; tt < DT_T; tt++) {
                if (tt + 2 < DT_T) {
                    const int n = (tt + 2) % 3;
                    ld8(s_qk[buf][tt + 2][0][cc], qs[n]);
                    ld8(s_qk[buf][tt + 2][1][cc], ks[n]);
                    gbv(tt + 2, gs[n], bs[n], vs[n]);
                }
                const int c3 = tt % 3;
                step(tt, ks[c3], qs[c3], gs[c3], bs[c3], vs[c3]);
            }
        } else {
            int tt = 0;
            for (; tt + 1 < nt; tt += 2) pair(tt);
            if (tt < nt) step(tt, ka, qa, ga, ba, va);
        }
        if (more) put(buf ^ 1);
        __syncthreads();
        // the stage's outputs, coalesced (the buffer is rewritten two stages later, after a barrier)
        for (int i = t; i < nt * 16; i += 256)
            o[(int64_t)(t0 + (i >> 4)) * DIN + vh * HV + row0 + (i & 15)] = s_out[buf][i >> 4][i & 15];
    }
#pragma unroll
    for (int s = 0; s < 8; s++) srow[cc + 16 * s] = r[s];
}

// gated norm (rms_norm(o) * ssm_norm * silu(z), engine.rs:2560-2566) + Q8_0 of (token, value head),
// one wave each
__global__ __launch_bounds__(256) void gated_norm_kernel(const float *o, const float *proj, const float *ssm_norm, float eps,
                                                         int8_t *oq, uint16_t *od) {
    const int64_t t = blockIdx.x;
    const int vh = blockIdx.y * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const float *orow = o + t * DIN + vh * HV;
    const float x0 = orow[lane], x1 = orow[lane + 64];
    const float mean = wave_mean_sq_128(x0, x1, orow);
    const float sc = 1.0f / sqrtf(mean + eps);
    const float *z = proj + t * DN_ROWS + DN_Z + vh * HV;
    const float o0 = ((x0 * sc) * ssm_norm[lane]) * v_silu(z[lane]);
    const float o1 = ((x1 * sc) * ssm_norm[lane + 64]) * v_silu(z[lane + 64]);
    // Q8_0 blocks of 32: lanes 0..31 hold blocks 0 (o0) and 2 (o1), lanes 32..63 blocks 1 and 3
    float d0, d1;
    const uint32_t p0 = quant32_lanes(o0, &d0), p1 = quant32_lanes(o1, &d1);
    int8_t *q = oq + t * DIN + vh * HV;
    if ((lane & 3) == 0) {
        *(uint32_t *)(q + lane) = p0;
        *(uint32_t *)(q + lane + 64) = p1;
    }
    uint16_t *d = od + t * (DIN / 32) + vh * (HV / 32);
    if (lane == 0) { d[0] = f2h(d0); d[2] = f2h(d1); }
    if (lane == 32) { d[1] = f2h(d0); d[3] = f2h(d1); }
}

// ---- attention -------------------------------------------------------------------------------
// q heads: rms_norm * q_norm, RoPE NEOX, f16 (engine.rs:2614-2703); K heads the same with k_norm
// into the K cache at the token's position; the V rows f16 into V^T. One wave per vector: waves
// 0..15 the q heads (skipped when kv_only), 16..17 the K heads, 18 the V rows.
__global__ __launch_bounds__(256) void attn_prep_kernel(const float *proj, const float *q_norm, const float *k_norm,
                                                        const float *rope, int pos0, float eps, uint16_t *qh,
                                                        uint16_t *kc, uint16_t *vt, int n_ctx, int kv_only) {
    const int64_t t = blockIdx.x;
    const int w = blockIdx.y * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int pos = pos0 + (int)t;
    const float *pr = proj + t * DN_ROWS;
    if (w < NH + NKV) {
        if (w < NH && kv_only) return;
        const bool isk = w >= NH;
        const float *src = isk ? pr + AT_K + (w - NH) * HD : pr + w * 2 * HD;
        const float *nw = isk ? k_norm : q_norm;
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = src[lane + 64 * i];
        const float mean = wave_mean_sq_256(v, src);
        const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = (v[i] * scale) * nw[lane + 64 * i];
        // rotate_pairs NEOX (oxe_ops.cpp:443-455) of pairs (i, i + 32), i < 32, as rope_neox_lds
        const float *cs = rope + (int64_t)pos * NROT + 2 * (lane & (NROT / 2 - 1));
        const float c = cs[0], s = cs[1];
        const float oth = __shfl_xor(v[0], NROT / 2, 64);
        if (lane < NROT / 2) v[0] = __builtin_fmaf(v[0], c, -(oth * s));
        else v[0] = __builtin_fmaf(oth, s, v[0] * c);
        uint16_t *dst = isk ? kc + ((int64_t)(w - NH) * n_ctx + pos) * HD : qh + (t * NH + w) * HD;
#pragma unroll
        for (int i = 0; i < 4; i++) dst[lane + 64 * i] = f2h(v[i]);
    } else if (w == NH + NKV) {
        for (int i = lane; i < NKV * HD; i += 64) vt[(int64_t)i * n_ctx + pos] = f2h(pr[AT_V + i]);
    }
}

typedef _Float16 h2p __attribute__((ext_vector_type(2)));
OXE_DEV h2p u2h(uint32_t u) { return __builtin_bit_cast(h2p, u); }
OXE_DEV uint32_t h2u(h2p v) { return __builtin_bit_cast(uint32_t, v); }
// GGML_F16x8_REDUCE of the 4 accumulators held by the 4 lanes of a quad, then the f32 widening and
// vaddvq (the decode attention's reduce)
OXE_DEV float f16x8_reduce_quad(h2p acc[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = acc[i] + u2h((uint32_t)dpp_i<DPP_XOR2>((int)h2u(acc[i])));
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = acc[i] + u2h((uint32_t)dpp_i<DPP_XOR1>((int)h2u(acc[i])));
    const float t0 = (float)acc[0].x + (float)acc[2].x;
    const float t1 = (float)acc[0].y + (float)acc[2].y;
    const float t2 = (float)acc[1].x + (float)acc[3].x;
    const float t3 = (float)acc[1].y + (float)acc[3].y;
    return (t0 + t1) + (t2 + t3);
}

// One query (token t at position pos) and head h per workgroup (oxe_attn_head_f16,
// oxe_ops.cpp:465-493): scores over positions <= pos (ggml_vec_dot_f16: 4 x 8 fp16 FMA chains,
// chain (j, l) takes positions 32 s + 8 j + l), softmax over n_kv = pad256(pos + 1) with the -inf
// mask (oxe_soft_max_f32, scale 1/16, the group sums added in double), f16 probabilities, then
// V^T . p over n_kv (positions after pos contribute +0 . +0, as the zeroed cache rows of a
// single-token step) and the sigmoid gate. f32 output o[t][h * 256 + d]. Dynamic LDS: scores
// (f32) and probabilities (f16) of up to kv_cap positions.
__global__ __launch_bounds__(256) void attn_kernel(const uint16_t *qh, const uint16_t *kc, const uint16_t *vt,
                                                   const float *proj, int pos0, int n_ctx, int kv_cap, float *o) {
    extern __shared__ __align__(16) float s_dyn[];
    float *s_s = s_dyn;                             // [kv_cap]
    uint16_t *s_p = (uint16_t *)(s_dyn + kv_cap);   // [kv_cap]
    __shared__ __align__(16) uint16_t s_q[HD];
    __shared__ double s_red[4];
    __shared__ float s_mx[4];
    __shared__ float s_f;
    const int64_t t = blockIdx.x;
    const int h = blockIdx.y, kvh = h / GQA, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int pos = pos0 + (int)t;
    int n_kv = (pos + 1 + 255) / 256 * 256;
    if (n_kv > n_ctx) n_kv = n_ctx;
    if (tid < HD / 8) *(uint4 *)&s_q[8 * tid] = *(const uint4 *)(qh + (t * NH + h) * HD + 8 * tid);
    __syncthreads();
    // scores: thread (position pp = tid / 4 of a pass of 64, chain quad lane j = tid % 4)
    {
        const int pp = tid >> 2, j = tid & 3;
        const uint16_t *kb = kc + (int64_t)kvh * n_ctx * HD;
        for (int p0 = 0; p0 <= pos; p0 += 64) {
            const int p = p0 + pp;
            const uint16_t *krow = kb + (int64_t)(p <= pos ? p : pos) * HD;
            h2p acc[4];
#pragma unroll
            for (int i = 0; i < 4; i++) acc[i] = h2p{(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
            for (int sx = 0; sx < HD / 32; sx++) {
                const uint4 kv = *(const uint4 *)(krow + 32 * sx + 8 * j);
                const uint4 qv = *(const uint4 *)(&s_q[32 * sx + 8 * j]);
                acc[0] = __builtin_elementwise_fma(u2h(kv.x), u2h(qv.x), acc[0]);
                acc[1] = __builtin_elementwise_fma(u2h(kv.y), u2h(qv.y), acc[1]);
                acc[2] = __builtin_elementwise_fma(u2h(kv.z), u2h(qv.z), acc[2]);
                acc[3] = __builtin_elementwise_fma(u2h(kv.w), u2h(qv.w), acc[3]);
            }
            const float sc = f16x8_reduce_quad(acc);
            if (j == 0 && p <= pos) s_s[p] = sc;
        }
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    const int ng = n_kv / 4;
    float mx = -__builtin_inff();
    for (int g = tid; g < ng; g += 256)
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = 4 * g + i;
            const float wv = p <= pos ? s_s[p] * scale : -__builtin_inff();
            mx = (mx > wv) ? mx : wv;
        }
    mx = wave_max_any(mx);
    if (lane == 0) s_mx[w] = mx;
    __syncthreads();
    {
        const float m01 = s_mx[0] > s_mx[1] ? s_mx[0] : s_mx[1], m23 = s_mx[2] > s_mx[3] ? s_mx[2] : s_mx[3];
        mx = m01 > m23 ? m01 : m23;
    }
    // e = v_expf(w - max) kept in the score slots; group sums (e0 + e1) + (e2 + e3) added in double
    double part = 0.0;
    for (int g = tid; g < ng; g += 256) {
        float e[4];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int p = 4 * g + i;
            e[i] = v_expf((p <= pos ? s_s[p] * scale : -__builtin_inff()) - mx);
        }
        part += (double)((e[0] + e[1]) + (e[2] + e[3]));
#pragma unroll
        for (int i = 0; i < 4; i++) s_s[4 * g + i] = e[i];
    }
    part = wave_sum_d_any(part);
    if (lane == 0) s_red[w] = part;
    __syncthreads();
    const double P = (s_red[0] + s_red[1]) + (s_red[2] + s_red[3]);
    float f;
    const bool ok = bracket_ok_recip(P, P, ng, &f);   // uniform
    if (!ok) {
        if (tid == 0) {
            double sum = 0.0;
            for (int g = 0; g < ng; g++) sum += (double)((s_s[4 * g] + s_s[4 * g + 1]) + (s_s[4 * g + 2] + s_s[4 * g + 3]));
            s_f = (float)(1.0 / sum);
        }
        __syncthreads();
        f = s_f;
    }
    for (int p = tid; p < n_kv; p += 256) s_p[p] = f2h(s_s[p] * f);
    __syncthreads();
    // V^T . p: thread (dim d0 + tid / 16, lane cp = tid % 16 of a 16-lane row): positions 32 s + 2 cp,
    // + 1, i.e. chain quad j = cp / 4, accumulator cp % 4; the F16x8 reduce inside the row: ror 8 and
    // ror 4 pair the quads as xor 2 / xor 1 of the reference tree, then the f32 tail in the quad
    const int cp = tid & 15;
    const uint16_t *vb = vt + (int64_t)kvh * HD * n_ctx;
    for (int d0 = 0; d0 < HD; d0 += 16) {
        const int d = d0 + (tid >> 4);
        const uint16_t *vrow = vb + (int64_t)d * n_ctx;
        h2p acc = h2p{(_Float16)0.0f, (_Float16)0.0f};
        for (int s = 0; s < n_kv / 32; s++) {
            const int p = 32 * s + 2 * cp;
            uint32_t vw = *(const uint32_t *)(vrow + p);
            if (p > pos) vw = 0u;
            else if (p + 1 > pos) vw &= 0xffffu;
            acc = __builtin_elementwise_fma(u2h(vw), u2h(*(const uint32_t *)&s_p[p]), acc);
        }
        h2p x = acc;
        x = x + u2h((uint32_t)dpp_i<DPP_ROR8>((int)h2u(x)));
        x = x + u2h((uint32_t)dpp_i<DPP_ROR4>((int)h2u(x)));
        const float lo = (float)x.x, hi = (float)x.y;
        const float tlo = lo + dpp_f<DPP_XOR2>(lo), thi = hi + dpp_f<DPP_XOR2>(hi);
        const float s2 = tlo + thi;
        const float out = s2 + dpp_f<DPP_XOR1>(s2);
        if (cp == 0) {
            const float gate = proj[t * DN_ROWS + h * 2 * HD + HD + d];
            o[t * MIX_W + h * HD + d] = out * sigmoid_c(gate);
        }
    }
}

// The same per (query, head) arithmetic with the 8 query heads of one KV head in one workgroup
// (grid (token, kv head)): each K row and V^T chunk is loaded once for the 8 heads. Scores: thread
// (position pp = tid / 4 of a pass of 64, chain quad lane j) keeps the 8 heads' accumulators;
// softmax: wave w takes heads 2 w and 2 w + 1 (wave-level reductions only), the f16 probabilities
// overwrite the front half of the head's f32 score row (in lane order: a write only reaches score
// slots the wave has already read); V^T . p: thread (dim, chain quad lane j) keeps the 8 heads'
// 4 accumulators, as the decode's pv kernel. Dynamic LDS: [8][kv_cap] f32.
constexpr int AQ_LDS_MAX = 150 * 1024;   // dynamic LDS cap of attn_gqa_kernel (32 bytes per position)
constexpr int AQ_BYTES_PER_POS = 4 * GQA;
__global__ __launch_bounds__(256, 2) void attn_gqa_kernel(const uint16_t *qh, const uint16_t *kc, const uint16_t *vt,
                                                          const float *proj, int pos0, int n_ctx, int kv_cap, float *o) {
    extern __shared__ __align__(16) float s_dyn[];
    float *s_s = s_dyn;   // [GQA][kv_cap] f32 scores, then f16 probabilities in the first half of each row
    __shared__ __align__(16) uint16_t s_q[GQA][HD];
    // the chunk's tokens from the last: the longest causal rows start first
    const int64_t t = (int64_t)gridDim.x - 1 - blockIdx.x;
    const int kvh = blockIdx.y, tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    const int pos = pos0 + (int)t;
    int n_kv = (pos + 1 + 255) / 256 * 256;
    if (n_kv > n_ctx) n_kv = n_ctx;
    *(uint4 *)&s_q[tid >> 5][8 * (tid & 31)] = *(const uint4 *)(qh + (t * NH + kvh * GQA + (tid >> 5)) * HD + 8 * (tid & 31));
    __syncthreads();
    const int j = tid & 3;
    {
        // thread (positions pp and pp + 64 of a pass of 128, chain quad j): each query chunk read
        // from LDS serves both positions
        const int pp = tid >> 2;
        const uint16_t *kb = kc + (int64_t)kvh * n_ctx * HD;
        // the next pass's K chunks load while this pass runs (rows past pos clamped to pos)
        uint4 kva[HD / 32], kvb[HD / 32];
        auto kload = [&](int p0, uint4 (&xa)[HD / 32], uint4 (&xb)[HD / 32]) {
            const int pa = p0 + pp, pb = p0 + 64 + pp;
            const uint16_t *ka = kb + (int64_t)(pa <= pos ? pa : pos) * HD;
            const uint16_t *kr = kb + (int64_t)(pb <= pos ? pb : pos) * HD;
#pragma unroll
            for (int sx = 0; sx < HD / 32; sx++) {
                xa[sx] = *(const uint4 *)(ka + 32 * sx + 8 * j);
                xb[sx] = *(const uint4 *)(kr + 32 * sx + 8 * j);
            }
        };
        kload(0, kva, kvb);
        for (int p0 = 0; p0 <= pos; p0 += 128) {
            const int pa = p0 + pp, pb = p0 + 64 + pp;
            uint4 nka[HD / 32], nkb[HD / 32];
            kload(p0 + 128, nka, nkb);
            // one query head at a time: its two scores are finished and stored before the next
            // head's query chunks are read, so only the K chunks stay in registers
#pragma unroll 2
            for (int h = 0; h < GQA; h++) {
                h2p acc[4], acb[4];
#pragma unroll
                for (int i = 0; i < 4; i++) acc[i] = acb[i] = h2p{(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
                for (int sx = 0; sx < HD / 32; sx++) {
                    const uint4 qv = *(const uint4 *)(&s_q[h][32 * sx + 8 * j]);
                    const uint4 kv = kva[sx], kw = kvb[sx];
                    acc[0] = __builtin_elementwise_fma(u2h(kv.x), u2h(qv.x), acc[0]);
                    acc[1] = __builtin_elementwise_fma(u2h(kv.y), u2h(qv.y), acc[1]);
                    acc[2] = __builtin_elementwise_fma(u2h(kv.z), u2h(qv.z), acc[2]);
                    acc[3] = __builtin_elementwise_fma(u2h(kv.w), u2h(qv.w), acc[3]);
                    acb[0] = __builtin_elementwise_fma(u2h(kw.x), u2h(qv.x), acb[0]);
                    acb[1] = __builtin_elementwise_fma(u2h(kw.y), u2h(qv.y), acb[1]);
                    acb[2] = __builtin_elementwise_fma(u2h(kw.z), u2h(qv.z), acb[2]);
                    acb[3] = __builtin_elementwise_fma(u2h(kw.w), u2h(qv.w), acb[3]);
                }
                const float sa = f16x8_reduce_quad(acc), sb = f16x8_reduce_quad(acb);
                if (j == 0 && pa <= pos) s_s[h * kv_cap + pa] = sa;
                if (j == 0 && pb <= pos) s_s[h * kv_cap + pb] = sb;
            }
#pragma unroll
            for (int sx = 0; sx < HD / 32; sx++) {
                kva[sx] = nka[sx];
                kvb[sx] = nkb[sx];
            }
        }
    }
    __syncthreads();
    const float scale = 1.0f / sqrtf((float)HD);
    const int ng = n_kv / 4;
#pragma unroll 1
    for (int hh = 0; hh < 2; hh++) {
        const int h = 2 * w + hh;
        float *ss = s_s + h * kv_cap;
        float mx = -__builtin_inff();
        for (int p = lane; p < n_kv; p += 64) {
            const float wv = p <= pos ? ss[p] * scale : -__builtin_inff();
            mx = (mx > wv) ? mx : wv;
        }
        mx = wave_max_any(mx);
        double part = 0.0;
        for (int g = lane; g < ng; g += 64) {
            float e[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int p = 4 * g + i;
                e[i] = v_expf((p <= pos ? ss[p] * scale : -__builtin_inff()) - mx);
            }
            part += (double)((e[0] + e[1]) + (e[2] + e[3]));
#pragma unroll
            for (int i = 0; i < 4; i++) ss[4 * g + i] = e[i];
        }
        const double P = wave_sum_d_any(part);
        float f;
        wave_lds_sync();
        if (!bracket_ok_recip(P, P, ng, &f)) {   // wave-uniform
            double sum = 0.0;
            for (int g = 0; g < ng; g++) sum += (double)((ss[4 * g] + ss[4 * g + 1]) + (ss[4 * g + 2] + ss[4 * g + 3]));
            f = (float)(1.0 / sum);
            wave_lds_sync();
        }
        // iteration k reads score slots [64 k, 64 k + 64) and writes f16 slots [64 k, 64 k + 64), i.e.
        // bytes [128 k, 128 k + 128): score slots of iteration k / 2 <= k, already read
        uint16_t *sp = (uint16_t *)ss;
        for (int p = lane; p < n_kv; p += 64) sp[p] = f2h(ss[p] * f);
    }
    __syncthreads();
    const uint16_t *vb = vt + (int64_t)kvh * HD * n_ctx;
    const float *gate = proj + t * DN_ROWS + kvh * GQA * 2 * HD + HD;
    // thread (dims d and d + 64 of a pass of 128, chain quad j): each probability chunk read from
    // LDS serves both dims
    for (int d0 = 0; d0 < HD; d0 += 128) {
        const int d = d0 + (tid >> 2);
        const uint16_t *vrow = vb + (int64_t)d * n_ctx, *vrw = vrow + (int64_t)64 * n_ctx;
        h2p acc[GQA][4], acb[GQA][4];
#pragma unroll
        for (int h = 0; h < GQA; h++)
#pragma unroll
            for (int i = 0; i < 4; i++) acc[h][i] = acb[h][i] = h2p{(_Float16)0.0f, (_Float16)0.0f};
        // n_kv is a multiple of 256: blocks of 32 positions in pairs, the pair's V^T loads first
        // the next pair's V^T chunks load while this pair runs (the last pair loads itself again)
        uint4 vvs[2], vws[2];
        auto vload = [&](int sx0, uint4 (&xa)[2], uint4 (&xb)[2]) {
#pragma unroll
            for (int u = 0; u < 2; u++) {
                xa[u] = *(const uint4 *)(vrow + 32 * (sx0 + u) + 8 * j);
                xb[u] = *(const uint4 *)(vrw + 32 * (sx0 + u) + 8 * j);
            }
        };
        vload(0, vvs, vws);
        for (int sx0 = 0; sx0 < n_kv / 32; sx0 += 2) {
          uint4 nvv[2], nvw[2];
          vload(sx0 + 2 < n_kv / 32 ? sx0 + 2 : sx0, nvv, nvw);
#pragma unroll
          for (int u = 0; u < 2; u++) {
            const int sx = sx0 + u;
            const int p = 32 * sx + 8 * j;   // this lane's 8 positions p .. p + 7 (chain quad j of block sx)
            uint4 vv = vvs[u], vw = vws[u];
            if (p + 7 > pos) {   // V^T of positions after pos is +0 in a single-token step
                uint32_t m[4];
#pragma unroll
                for (int i = 0; i < 4; i++) {
                    const int q0 = p + 2 * i;
                    m[i] = q0 > pos ? 0u : (q0 + 1 > pos ? 0xffffu : 0xffffffffu);
                }
                vv.x &= m[0]; vv.y &= m[1]; vv.z &= m[2]; vv.w &= m[3];
                vw.x &= m[0]; vw.y &= m[1]; vw.z &= m[2]; vw.w &= m[3];
            }
#pragma unroll
            for (int h = 0; h < GQA; h++) {
                const uint4 pv = *(const uint4 *)((const uint16_t *)(s_s + h * kv_cap) + p);
                acc[h][0] = __builtin_elementwise_fma(u2h(vv.x), u2h(pv.x), acc[h][0]);
                acc[h][1] = __builtin_elementwise_fma(u2h(vv.y), u2h(pv.y), acc[h][1]);
                acc[h][2] = __builtin_elementwise_fma(u2h(vv.z), u2h(pv.z), acc[h][2]);
                acc[h][3] = __builtin_elementwise_fma(u2h(vv.w), u2h(pv.w), acc[h][3]);
                acb[h][0] = __builtin_elementwise_fma(u2h(vw.x), u2h(pv.x), acb[h][0]);
                acb[h][1] = __builtin_elementwise_fma(u2h(vw.y), u2h(pv.y), acb[h][1]);
                acb[h][2] = __builtin_elementwise_fma(u2h(vw.z), u2h(pv.z), acb[h][2]);
                acb[h][3] = __builtin_elementwise_fma(u2h(vw.w), u2h(pv.w), acb[h][3]);
            }
          }
#pragma unroll
          for (int u = 0; u < 2; u++) {
            vvs[u] = nvv[u];
            vws[u] = nvw[u];
          }
        }
#pragma unroll
        for (int h = 0; h < GQA; h++) {
            const float oa = f16x8_reduce_quad(acc[h]), ob = f16x8_reduce_quad(acb[h]);
            if (j == 0) {
                o[t * MIX_W + (kvh * GQA + h) * HD + d] = oa * sigmoid_c(gate[h * 2 * HD + d]);
                o[t * MIX_W + (kvh * GQA + h) * HD + d + 64] = ob * sigmoid_c(gate[h * 2 * HD + d + 64]);
            }
        }
    }
}

// ---- router, routing, MoE ------------------------------------------------------------------
// router logits (ggml_vec_dot_f32: chain c of 16 over elements c + 16 q, then the NEON tree) of
// (token, expert e < 256), and the shared-expert gate (e == 256: sigmoid of the dot with shexp_gate).
// Workgroup = 16 tokens x 16 rows (row 256 is the shared gate); lane group g (16 lanes, lane = chain
// c) holds the chains of 4 tokens x 4 rows; token and weight rows are staged through LDS 256
// elements at a time. Every dot keeps the reference's 16 chains in order and its reduction tree.
constexpr int RT_TB = 16, RT_KC = 256, RT_Q = RT_KC / 16, RT_QP = RT_Q + 4, RT_NR = NEXP + 1;
// LDS rows are stored chain-major: element 16 q + c of a stage at [row][c][q] (rows of RT_QP floats,
// padded so that 16-byte reads of 16 consecutive chains fall on distinct banks), so a thread reads
// four consecutive steps of its chain in one 16-byte load
__global__ __launch_bounds__(256) void router_kernel(const float *xn, const float *router, const float *shg, int T, float *lg,
                                                     float *sg) {
    __shared__ __align__(16) float s_x[RT_TB][16][RT_QP], s_w[RT_TB][16][RT_QP];
    const int tid = threadIdx.x, g = tid >> 4, c = tid & 15, tb = g & 3, eb = g >> 2;
    const int64_t t0 = (int64_t)blockIdx.x * RT_TB;
    const int e0 = blockIdx.y * RT_TB;
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) acc[i][e] = 0.0f;
    // a stage's token and weight elements in registers: the next stage's are loaded while the
    // current one runs (the last stage loads itself again)
    constexpr int RT_R = RT_TB * RT_KC / 4 / 256;
    float4 xr[RT_R], wr4[RT_R];
    auto stage_load = [&](int k0) {
#pragma unroll
        for (int r = 0; r < RT_R; r++) {
            const int i = tid + 256 * r, row = i / (RT_KC / 4), c4 = i % (RT_KC / 4);
            const int64_t tt = t0 + row;
            const int ee = e0 + row;
            xr[r] = tt < T ? *(const float4 *)(xn + tt * E + k0 + 4 * c4) : make_float4(0, 0, 0, 0);
            const float *wr = ee < NEXP ? router + (int64_t)ee * E : shg;
            wr4[r] = ee < RT_NR ? *(const float4 *)(wr + k0 + 4 * c4) : make_float4(0, 0, 0, 0);
        }
    };
    stage_load(0);
    for (int k0 = 0; k0 < E; k0 += RT_KC) {
        __syncthreads();
#pragma unroll
        for (int r = 0; r < RT_R; r++) {
            const int i = tid + 256 * r, row = i / (RT_KC / 4), c4 = i % (RT_KC / 4);
            const float4 xv = xr[r], wv = wr4[r];
            // elements 4 c4 .. 4 c4 + 3 of the stage: step q = c4 / 4, chains 4 (c4 % 4) ..
            const int q = c4 >> 2, cb = 4 * (c4 & 3);
            s_x[row][cb][q] = xv.x; s_x[row][cb + 1][q] = xv.y; s_x[row][cb + 2][q] = xv.z; s_x[row][cb + 3][q] = xv.w;
            s_w[row][cb][q] = wv.x; s_w[row][cb + 1][q] = wv.y; s_w[row][cb + 2][q] = wv.z; s_w[row][cb + 3][q] = wv.w;
        }
        __syncthreads();
        stage_load(k0 + RT_KC < E ? k0 + RT_KC : k0);
#pragma unroll
        for (int q4 = 0; q4 < RT_Q / 4; q4++) {
            float4 xv[4], wv[4];
#pragma unroll
            for (int i = 0; i < 4; i++) xv[i] = *(const float4 *)&s_x[4 * tb + i][c][4 * q4];
#pragma unroll
            for (int e = 0; e < 4; e++) wv[e] = *(const float4 *)&s_w[4 * eb + e][c][4 * q4];
#pragma unroll
            for (int qq = 0; qq < 4; qq++)
#pragma unroll
                for (int i = 0; i < 4; i++)
#pragma unroll
                    for (int e = 0; e < 4; e++) {
                        const float xs = qq == 0 ? xv[i].x : qq == 1 ? xv[i].y : qq == 2 ? xv[i].z : xv[i].w;
                        const float ws = qq == 0 ? wv[e].x : qq == 1 ? wv[e].y : qq == 2 ? wv[e].z : wv[e].w;
                        acc[i][e] = __builtin_fmaf(ws, xs, acc[i][e]);
                    }
        }
    }
    float v[4][4];
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++) v[i][e] = dot16_tree_dpp(acc[i][e]);
    // every lane of the group holds all 16 sums; lane c writes (token c / 4, row c % 4)
    float mine = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int e = 0; e < 4; e++)
            if (c == 4 * i + e) mine = v[i][e];
    const int64_t tt = t0 + 4 * tb + (c >> 2);
    const int ee = e0 + 4 * eb + (c & 3);
    if (tt < T && ee < RT_NR) {
        if (ee < NEXP) lg[tt * NEXP + ee] = mine;
        else sg[tt] = sigmoid_c(mine);
    }
}

// routing of one token per wave (softmax, top-8 with the reference's tie rules, renormalised
// weights: route_wave, engine.rs:3414-3475)
__global__ __launch_bounds__(256) void route_kernel(const float *lg, int T, int32_t *ids, float *wts, uint32_t *tie_count) {
    __shared__ RouteOut ro[4];
    const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + w;
    if (t >= T) return;
    if (lane == 0) ro[w].tie = 0;
    wave_lds_sync();
    route_wave(lg + t * NEXP, 0, ro[w]);
    wave_lds_sync();
    if (lane < KUSED) {
        ids[t * KUSED + lane] = ro[w].ids[0][lane];
        wts[t * KUSED + lane] = ro[w].w[0][lane];
    }
    if (lane == 0 && ro[w].tie) atomicAdd(tie_count, 1u);
}

// (token, rank) pairs grouped by expert: counts, then (one workgroup) offsets and the 64-pair tiles
// of every expert, then the scatter. The order of pairs inside an expert's group is free: every
// (pair, row) result of the grouped GEMMs is independent of its neighbours.
constexpr int MO_CNT = 0, MO_OFF = NEXP, MO_FILL = 2 * NEXP, MO_NT = 3 * NEXP, MO_WORDS = 3 * NEXP + 1;
__global__ void moe_count_kernel(const int32_t *ids, int np, int32_t *mo) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i < np) atomicAdd(&mo[MO_CNT + ids[i]], 1);
}
__global__ __launch_bounds__(NEXP) void moe_tiles_kernel(int32_t *mo, int4 *tiles) {
    __shared__ int s_c[NEXP], s_t[NEXP];
    const int e = threadIdx.x;
    const int c = mo[MO_CNT + e], nt = (c + 63) / 64;
    s_c[e] = c;
    s_t[e] = nt;
    __syncthreads();
    for (int d = 1; d < NEXP; d <<= 1) {
        const int a = e >= d ? s_c[e - d] : 0, b = e >= d ? s_t[e - d] : 0;
        __syncthreads();
        s_c[e] += a;
        s_t[e] += b;
        __syncthreads();
    }
    const int off = s_c[e] - c, tb = s_t[e] - nt;
    mo[MO_OFF + e] = off;
    mo[MO_FILL + e] = 0;
    for (int s = 0; s < nt; s++) tiles[tb + s] = make_int4(e, off + 64 * s, min(64, c - 64 * s), 0);
    if (e == NEXP - 1) mo[MO_NT] = s_t[e];
}
__global__ void moe_scatter_kernel(const int32_t *ids, int np, int32_t *mo, int32_t *ptok, int32_t *pair_of) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= np) return;
    const int e = ids[i];
    const int p = mo[MO_OFF + e] + atomicAdd(&mo[MO_FILL + e], 1);
    ptok[p] = i / KUSED;
    pair_of[i] = p;
}

// swiglu (ggml_vec_swiglu_f32: silu(gate) * up) of a gate/up output row with the 16-row interleave
// (8 gate rows, then 8 up rows) and the Q8_0 of the 512 values: one workgroup per row
__global__ __launch_bounds__(256) void swiglu_quant_kernel(const float *gu, int8_t *hq, uint16_t *hd) {
    const int64_t r = blockIdx.x;
    const float *g = gu + r * (2 * FF);
#pragma unroll
    for (int k = 0; k < 2; k++) {
        const int i = threadIdx.x + 256 * k, tl = i >> 3, rr = i & 7;
        const float h = v_silu(g[tl * 16 + rr]) * g[tl * 16 + 8 + rr];
        float dd;
        const uint32_t word = quant32_lanes(h, &dd);
        if ((i & 3) == 0) *(uint32_t *)(hq + r * FF + i) = word;
        if ((i & 31) == 0) hd[r * (FF / 32) + i / 32] = f2h(dd);
    }
}

// combine (engine.rs:3591-3601): m = d_0 w_0, m = m + d_j w_j (j = 1..7), f = m + d_sh g_sh,
// x2 = f + x1, per (token, row)
__global__ __launch_bounds__(256) void combine_kernel(const float *dout, const int32_t *pair_of, const float *wts,
                                                      const float *sh, const float *sg, const float *x1, float *x2,
                                                      int T) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (int64_t)T * E) return;
    const int64_t t = i / E, r = i % E;
    float m = dout[(int64_t)pair_of[t * KUSED] * E + r] * wts[t * KUSED];
    for (int j = 1; j < KUSED; j++) {
        const float p = dout[(int64_t)pair_of[t * KUSED + j] * E + r] * wts[t * KUSED + j];
        m = m + p;
    }
    const float s = sh[i] * sg[t];
    const float f = m + s;
    x2[i] = f + x1[i];
}

// ---- MTP entry for seeding -----------------------------------------------------------------
// row t: [rms_norm(embd(tok)) * enorm ; rms_norm(h) * hnorm] quantised (K = 2 n_embd), as the
// decode's entry prologue (engine.rs:2362-2390); the embedding goes to x (replay source) first
__global__ __launch_bounds__(PT) void entry_in_kernel(Q8W emb, const uint32_t *toks, const float *h, float *x,
                                                      const float *enorm, const float *hnorm, float eps, int8_t *xq,
                                                      uint16_t *xd) {
    __shared__ NormScratch ns;
    const int64_t t = blockIdx.x;
    float v[EPT];
    embed8(emb, toks[t], v);
    store8(x + t * E, v);
    __syncthreads();
    rms_norm_mul_e(v, x + t * E, enorm, eps, ns);
    quant8(v, xq + t * 2 * E + EPT * threadIdx.x, xd + t * (2 * E / 32) + (EPT * threadIdx.x) / 32);
    const float *hr = h + t * E;
    load8(hr, v);
    rms_norm_mul_e(v, hr, hnorm, eps, ns);
    quant8(v, xq + t * 2 * E + E + EPT * threadIdx.x, xd + t * (2 * E / 32) + (E + EPT * threadIdx.x) / 32);
}

}  // namespace pf

// ---- host ----------------------------------------------------------------------------------------

int Engine::pf_alloc(int T) {
    if (T <= pfb.cap) return 0;
    try {
        const size_t np = (size_t)T * KUSED;
        pfb.x = alloc<float>((size_t)T * E);
        pfb.x1 = alloc<float>((size_t)T * E);
        pfb.xn = alloc<float>((size_t)T * E);
        pfb.hin = alloc<float>((size_t)T * E);
        pfb.xq = alloc<int8_t>((size_t)T * 2 * E);
        pfb.xd = alloc<uint16_t>((size_t)T * (2 * E / 32));
        pfb.proj = alloc<float>((size_t)T * DN_ROWS);
        pfb.cy = alloc<float>((size_t)T * NCH);
        pfb.gg = alloc<float>((size_t)T * NVH);
        pfb.gb = alloc<float>((size_t)T * NVH);
        pfb.o = alloc<float>((size_t)T * DIN);
        pfb.oq = alloc<int8_t>((size_t)T * DIN);
        pfb.od = alloc<uint16_t>((size_t)T * (DIN / 32));
        pfb.qh = alloc<uint16_t>((size_t)T * NH * HD);
        pfb.lg = alloc<float>((size_t)T * NEXP);
        pfb.sg = alloc<float>((size_t)T);
        pfb.ids = alloc<int32_t>(np);
        pfb.wts = alloc<float>(np);
        pfb.mo = alloc<int32_t>(pf::MO_WORDS);
        pfb.ptok = alloc<int32_t>(np);
        pfb.pair_of = alloc<int32_t>(np);
        pfb.max_tiles = (int)(np / 64 + NEXP);
        pfb.tiles = alloc<int4>((size_t)pfb.max_tiles);
        pfb.gu = alloc<float>(np * 2 * FF);
        pfb.hq = alloc<int8_t>(np * FF);
        pfb.hd = alloc<uint16_t>(np * (FF / 32));
        pfb.dout = alloc<float>(np * E);
        pfb.sh = alloc<float>((size_t)T * E);
        pfb.tok = alloc<uint32_t>((size_t)T);
        pfb.cap = T;
    } catch (...) {
        set_err("out of device memory for the prefill buffers");
        return -3;
    }
    return 0;
}

// dynamic LDS of the prefill attention for score rows of kv_cap positions: the kv-head-shared kernel
// where its 8 rows fit, else the per-head kernel
int Engine::pf_attn_lds(int kv_cap) {
    const bool gqa = (size_t)kv_cap * pf::AQ_BYTES_PER_POS <= (size_t)pf::AQ_LDS_MAX;
    const size_t lds = (size_t)kv_cap * (gqa ? pf::AQ_BYTES_PER_POS : 6);
    if (lds > 160 * 1024 - 4096) {
        set_err("prefill attention: context too long for the LDS-resident score row");
        return -1;
    }
    int &have = gqa ? pfb.attn_lds_gqa : pfb.attn_lds;
    if ((int)lds > have) {
        const void *f = gqa ? (const void *)pf::attn_gqa_kernel : (const void *)pf::attn_kernel;
        if (hipFuncSetAttribute(f, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) != hipSuccess) return -2;
        have = (int)lds;
    }
    return 0;
}

// One chunk of T tokens at positions pos .. pos + T - 1 through every layer; h_out (optional, host)
// receives every token's h_nextn; the last token's logits go to lane 0's logits, its h_nextn to
// lane 0's hidden state.
int Engine::pf_chunk(const uint32_t *toks, int T, float *h_out) {
    using namespace pf;
    const int p0 = pos, n_ctx = m.n_ctx;
    const float eps = m.eps;
    int kv_cap = (p0 + T + 255) / 256 * 256;
    if (kv_cap > n_ctx) kv_cap = n_ctx;
    int rc = pf_attn_lds(kv_cap);
    if (rc) return rc;
    if (hipMemcpyAsync(pfb.tok, toks, (size_t)T * 4, hipMemcpyHostToDevice, st) != hipSuccess) return -2;
    const int64_t conv_slot = (int64_t)m.n_rec * NCH * (KC - 1), ssm_slot = (int64_t)m.n_rec * NVH * HV * HV;
    const int np = T * KUSED;
    auto gemm = [&](const Q8W &w, const int8_t *xq, const uint16_t *xd, int64_t k, float *y, int64_t ldy, const float *res,
                    int64_t nt) {
        GemmArgs g{};
        g.wq = w.q; g.wd = w.d; g.xq = xq; g.xd = xd; g.y = y; g.res = res;
        g.nr = w.rows; g.nt = nt; g.k = k; g.ldy = ldy; g.ldr = res ? E : 0;
        probe(K_PF_GEMM);
        const int r = gemm_launch(g, 0, st);
        probe(K_PF_GEMM);
        return r;
    };
    auto grouped = [&](const Q8W &w, int64_t rows, int64_t k, const int8_t *xq, const uint16_t *xd, const int32_t *xrow,
                       float *y) {
        GemmArgs g{};
        g.wq = w.q; g.wd = w.d; g.xq = xq; g.xd = xd; g.y = y;
        g.nr = rows; g.nt = np; g.k = k; g.ldy = rows;
        g.tiles = pfb.tiles; g.wq_stride = rows * k; g.wd_stride = rows * (k / 32); g.xrow = xrow;
        g.tile_count = pfb.mo + MO_NT;
        probe(K_PF_GEMM); probe(K_PF_EXPERT);
        const int r = gemm_launch(g, pfb.max_tiles, st);
        probe(K_PF_EXPERT); probe(K_PF_GEMM);
        return r;
    };
    for (int il = 0; il < d.n_layer; il++) {
        const LayerW &w = L[il];
        // input norm + Q8_0 (layer 0: the token embeddings, also the residual)
        hipLaunchKernelGGL(norm_quant_kernel, dim3(T), dim3(PT), 0, st, m.tok_embd, il == 0 ? pfb.tok : nullptr, pfb.x,
                           w.attn_norm, eps, pfb.xq, pfb.xd, (int64_t)E, nullptr);
        if ((rc = gemm(w.proj, pfb.xq, pfb.xd, E, pfb.proj, DN_ROWS, nullptr, T))) return rc;
        if (!w.att) {
            float *cs = m.conv_state + (int64_t)cur * conv_slot + (int64_t)w.index * NCH * (KC - 1);
            float *ss = m.ssm_state + (int64_t)cur * ssm_slot + (int64_t)w.index * NVH * HV * HV;
            hipLaunchKernelGGL(conv_kernel, dim3(NCH / 256, T), dim3(256), 0, st, pfb.proj, T, w.conv, cs, pfb.cy);
            hipLaunchKernelGGL(conv_state_kernel, dim3(NCH / 256), dim3(256), 0, st, pfb.proj, T, cs);
            hipLaunchKernelGGL(dn_prep_kernel, dim3(T, 8), dim3(256), 0, st, pfb.cy, pfb.proj, w.dt_bias, w.ssm_a, eps,
                               pfb.gg, pfb.gb);
            probe(K_PF_DELTA);
            hipLaunchKernelGGL(delta_kernel, dim3(NVH * 8), dim3(256), 0, st, pfb.cy, pfb.gg, pfb.gb, ss, pfb.o, T);
            probe(K_PF_DELTA);
            hipLaunchKernelGGL(gated_norm_kernel, dim3(T, NVH / 4), dim3(256), 0, st, pfb.o, pfb.proj, w.ssm_norm, eps,
                               pfb.oq, pfb.od);
        } else {
            uint16_t *kcl = m.kcache + (int64_t)w.index * NKV * n_ctx * HD;
            uint16_t *vtl = m.vcache + (int64_t)w.index * NKV * HD * n_ctx;
            hipLaunchKernelGGL(attn_prep_kernel, dim3(T, 5), dim3(256), 0, st, pfb.proj, w.q_norm, w.k_norm, m.rope, p0,
                               eps, pfb.qh, kcl, vtl, n_ctx, 0);
            probe(K_PF_ATTN);
            if ((size_t)kv_cap * AQ_BYTES_PER_POS <= (size_t)AQ_LDS_MAX)
                hipLaunchKernelGGL(attn_gqa_kernel, dim3(T, NKV), dim3(256), (size_t)kv_cap * AQ_BYTES_PER_POS, st, pfb.qh, kcl, vtl,
                                   pfb.proj, p0, n_ctx, kv_cap, pfb.o);
            else
                hipLaunchKernelGGL(attn_kernel, dim3(T, NH), dim3(256), (size_t)kv_cap * 6, st, pfb.qh, kcl, vtl, pfb.proj,
                                   p0, n_ctx, kv_cap, pfb.o);
            probe(K_PF_ATTN);
            if ((rc = quantize_q8_0(pfb.o, (int64_t)T * MIX_W, pfb.oq, pfb.od, st))) return rc;
        }
        // mixer output projection + residual
        if ((rc = gemm(w.out, pfb.oq, pfb.od, MIX_W, pfb.x1, E, pfb.x, T))) return rc;
        // post-attention norm: Q8_0 for the experts, f32 for the router
        hipLaunchKernelGGL(norm_quant_kernel, dim3(T), dim3(PT), 0, st, m.tok_embd, nullptr, pfb.x1, w.post_norm, eps,
                           pfb.xq, pfb.xd, (int64_t)E, pfb.xn);
        hipLaunchKernelGGL(router_kernel, dim3((T + RT_TB - 1) / RT_TB, (RT_NR + RT_TB - 1) / RT_TB), dim3(256), 0, st,
                           pfb.xn, w.router, w.shexp_gate, T, pfb.lg, pfb.sg);
        hipLaunchKernelGGL(route_kernel, dim3((T + 3) / 4), dim3(256), 0, st, pfb.lg, T, pfb.ids, pfb.wts,
                           b.counters + CNT_ERR_TIE);
        // shared expert over all tokens
        if ((rc = gemm(w.shexp_gu, pfb.xq, pfb.xd, E, pfb.gu, 2 * FFSH, nullptr, T))) return rc;
        hipLaunchKernelGGL(swiglu_quant_kernel, dim3(T), dim3(256), 0, st, pfb.gu, pfb.hq, pfb.hd);
        if ((rc = gemm(w.shexp_down, pfb.hq, pfb.hd, FFSH, pfb.sh, E, nullptr, T))) return rc;
        // routed experts: pairs grouped by expert, 64-pair tiles built on the device
        if (hipMemsetAsync(pfb.mo, 0, NEXP * 4, st) != hipSuccess) return -2;
        hipLaunchKernelGGL(moe_count_kernel, dim3((np + 255) / 256), dim3(256), 0, st, pfb.ids, np, pfb.mo);
        hipLaunchKernelGGL(moe_tiles_kernel, dim3(1), dim3(NEXP), 0, st, pfb.mo, pfb.tiles);
        hipLaunchKernelGGL(moe_scatter_kernel, dim3((np + 255) / 256), dim3(256), 0, st, pfb.ids, np, pfb.mo, pfb.ptok,
                           pfb.pair_of);
        if ((rc = grouped(w.exp_gu, 2 * FF, E, pfb.xq, pfb.xd, pfb.ptok, pfb.gu))) return rc;
        hipLaunchKernelGGL(swiglu_quant_kernel, dim3(np), dim3(256), 0, st, pfb.gu, pfb.hq, pfb.hd);
        if ((rc = grouped(w.exp_down, E, FF, pfb.hq, pfb.hd, nullptr, pfb.dout))) return rc;
        hipLaunchKernelGGL(combine_kernel, dim3((unsigned)(((int64_t)T * E + 255) / 256)), dim3(256), 0, st, pfb.dout,
                           pfb.pair_of, pfb.wts, pfb.sh, pfb.sg, pfb.x1, pfb.x, T);
        if (hipGetLastError() != hipSuccess) return -2;
    }
    // h_nextn of every token (output norm of x2), the LM head of the last token
    hipLaunchKernelGGL(norm_quant_kernel, dim3(T), dim3(PT), 0, st, m.tok_embd, nullptr, pfb.x, m.out_norm, eps, pfb.xq,
                       pfb.xd, (int64_t)E, pfb.xn);
    // the LM head of one token is a weight stream: the lane GEMV (HBM-bound), not the GEMM
    rc = oxe_hip_gemv_q8_0(E, m.output.rows, 1, m.output.q, m.output.d, pfb.xq + (int64_t)(T - 1) * E,
                           pfb.xd + (int64_t)(T - 1) * (E / 32), b.logits, nullptr, st);
    if (rc != 1) return rc == 0 ? -1 : rc;   // 1: done (oxe_vl_gemv's convention)
    if (hipMemcpyAsync(b.hid, pfb.xn + (int64_t)(T - 1) * E, (size_t)E * 4, hipMemcpyDeviceToDevice, st) != hipSuccess)
        return -2;
    if (h_out && hipMemcpyAsync(h_out, pfb.xn, (size_t)T * E * 4, hipMemcpyDeviceToHost, st) != hipSuccess) return -2;
    if (hipStreamSynchronize(st) != hipSuccess || hipGetLastError() != hipSuccess) return -2;
    pos = p0 + T;
    return 0;
}

int Engine::prefill(const uint32_t *toks, int n, uint32_t *next, float *h_all) {
    if (n < 1 || pos + n > m.n_ctx || !toks_ok(toks, n)) return -1;
    if (kq) {
        // the batched pass's GEMMs take Q8_0 matrices: a model with K-quant / F32 matrices runs the
        // decode runs two positions at a time (every position's state and h_nextn are the same)
        uint32_t g[OXE_NL] = {};
        for (int c0 = 0; c0 < n; c0 += OXE_NL) {
            const int c = std::min(OXE_NL, n - c0);
            int rc = verify(toks + c0, c, g);
            if (!rc) rc = commit(c);
            if (rc) return rc;
            for (int i = 0; i < c && h_all; i++)
                if ((rc = hidden_host(i, h_all + (size_t)(c0 + i) * E))) return rc;
        }
        if (next) *next = g[(n - 1) % OXE_NL];
        return 0;
    }
    int rc = pf_alloc(std::min(n, PF_CHUNK));
    if (rc) return rc;
    pend_n = 0;
    for (int c0 = 0; c0 < n; c0 += PF_CHUNK) {
        const int c = std::min(PF_CHUNK, n - c0);
        if ((rc = pf_chunk(toks + c0, c, h_all ? h_all + (size_t)c0 * E : nullptr))) return rc;
    }
    // greedy pick of the last token: the first strict maximum, NaN never wins, all -inf -> 0
    // (engine.rs:1969-1987)
    std::vector<float> lg(d.n_vocab);
    if (hipMemcpy(lg.data(), b.logits, (size_t)d.n_vocab * 4, hipMemcpyDeviceToHost) != hipSuccess) return -2;
    uint32_t best = 0;
    float bv = -__builtin_inff();
    for (int i = 0; i < d.n_vocab; i++)
        if (lg[i] > bv) {
            bv = lg[i];
            best = (uint32_t)i;
        }
    if (next) *next = best;
    return 0;
}

// MTP KV seeding of the pairs (toks[i], hs[i]) at positions pos0 + i, in batches (the decode's
// mtp_seed for any number of pairs): entry eh_proj, then the MTP layer's K and V rows.
int Engine::seed_batched(const uint32_t *toks, int n, int pos0, const float *hs) {
    using namespace pf;
    if (n < 1 || pos0 < 0 || pos0 + n > m.n_ctx || !toks_ok(toks, n) || !hs) return -1;
    const LayerW &w = L[d.n_layer];
    if (m.tok_embd_r.type != 8 || w.kq_proj()) {
        // the batched kernels below read the Q8_0 token embedding and the MTP layer's Q8_0
        // projection; a model with either in other blocks seeds through the seeding runs, OXE_NL
        // pairs at a time (every pair's K / V rows depend on that pair only)
        for (int c0 = 0; c0 < n; c0 += OXE_NL) {
            const int c = std::min(OXE_NL, n - c0);
            if (int rc = mtp_seed(toks + c0, c, pos0 + c0, hs + (size_t)c0 * E)) return rc;
        }
        return 0;
    }
    int rc = pf_alloc(std::min(n, PF_CHUNK));
    if (rc) return rc;
    uint16_t *kcl = m.kcache + (int64_t)w.index * NKV * m.n_ctx * HD;
    uint16_t *vtl = m.vcache + (int64_t)w.index * NKV * HD * m.n_ctx;
    for (int c0 = 0; c0 < n; c0 += PF_CHUNK) {
        const int T = std::min(PF_CHUNK, n - c0);
        if (hipMemcpyAsync(pfb.tok, toks + c0, (size_t)T * 4, hipMemcpyHostToDevice, st) != hipSuccess) return -2;
        if (hipMemcpyAsync(pfb.hin, hs + (size_t)c0 * E, (size_t)T * E * 4, hipMemcpyHostToDevice, st) != hipSuccess)
            return -2;
        hipLaunchKernelGGL(entry_in_kernel, dim3(T), dim3(PT), 0, st, m.tok_embd, pfb.tok, pfb.hin, pfb.x, w.enorm, w.hnorm,
                           m.eps, pfb.xq, pfb.xd);
        GemmArgs g{};
        g.wq = w.eh_proj.q; g.wd = w.eh_proj.d; g.xq = pfb.xq; g.xd = pfb.xd; g.y = pfb.x1;
        g.nr = E; g.nt = T; g.k = 2 * E; g.ldy = E;
        if ((rc = gemm_launch(g, 0, st))) return rc;
        hipLaunchKernelGGL(norm_quant_kernel, dim3(T), dim3(PT), 0, st, m.tok_embd, nullptr, pfb.x1, w.attn_norm, m.eps,
                           pfb.xq, pfb.xd, (int64_t)E, nullptr);
        GemmArgs k{};
        k.wq = w.proj.q + (int64_t)AT_K * E; k.wd = w.proj.d + (int64_t)AT_K * (E / 32);
        k.xq = pfb.xq; k.xd = pfb.xd; k.y = pfb.proj + AT_K;
        k.nr = AT_ROWS - AT_K; k.nt = T; k.k = E; k.ldy = DN_ROWS;
        if ((rc = gemm_launch(k, 0, st))) return rc;
        hipLaunchKernelGGL(attn_prep_kernel, dim3(T, 5), dim3(256), 0, st, pfb.proj, w.q_norm, w.k_norm, m.rope,
                           pos0 + c0, m.eps, pfb.qh, kcl, vtl, m.n_ctx, 1);
    }
    if (hipStreamSynchronize(st) != hipSuccess || hipGetLastError() != hipSuccess) return -2;
    return 0;
}

}  // namespace oxe

extern "C" {

// Routing of n_rows rows of n_expert (= 256) router logits: softmax, top-8 (libstdc++ std::sort order
// on ties), weights renormalised by their clamped sum. Replaces Engine::route (engine.rs:3414-3429)
// over oxe_soft_max_f32 and oxe_argsort_top_k_f32 (crates/kernels-sys/src/lib.rs:129-130).
int oxe_hip_route_f32(const float *logits, int64_t n_rows, int32_t *ids, float *w, uint32_t *tie_count, void *stream) {
    if (n_rows <= 0 || n_rows > (int64_t)1 << 30 || !logits || !ids || !w || !tie_count) return -1;
    hipLaunchKernelGGL(oxe::pf::route_kernel, dim3((unsigned)((n_rows + 3) / 4)), dim3(256), 0, (hipStream_t)stream, logits,
                       (int)n_rows, ids, w, tie_count);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// A batched prefill with HIP events around every launch of one kernel kind (12 every matrix-core
// GEMM, 13 the grouped expert GEMMs, 14 attention, 15 the delta rule): *total_us = their summed
// duration, *n = launches timed. Diagnostic for the prefill roofline (no counterpart in the
// reference).
int oxe_engine_prefill_probe(oxe_engine *e, const uint32_t *toks, int n, int kind, float *total_us, int *n_launch) {
    oxe::Engine *g = (oxe::Engine *)e;
    if (n < 1 || !g->toks_ok(toks, n) || g->pos + n > g->m.n_ctx || kind < 12 || kind > 15 || !total_us || !n_launch)
        return -1;
    g->probe_kind = kind;
    g->probe_used = 0;
    uint32_t next;
    const int rc = g->prefill(toks, n, &next, nullptr);
    g->probe_kind = -1;
    if (rc) return rc;
    double tot = 0.0;
    int cnt = 0;
    for (size_t i = 0; i + 1 < g->probe_used; i += 2) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, g->probe_ev[i], g->probe_ev[i + 1]) != hipSuccess) return -2;
        tot += ms;
        cnt++;
    }
    *total_us = (float)(tot * 1000.0);
    *n_launch = cnt;
    return 0;
}

}  // extern "C"
