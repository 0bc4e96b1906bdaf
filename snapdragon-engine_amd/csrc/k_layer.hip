// Mixer-side decode kernels of one layer, and the model entry / exit:
//   proj   - attn_norm + Q8_0 quantize (workgroup prologue) + the layer's input projections in one
//            weight pass (delta-net: [qkv | z | beta | alpha], attention: [q+gate | k | v], V rows
//            also written to the V^T cache)                   engine.rs:2394-2449, 2614-2703
//   dn     - delta-net recurrence: causal conv + silu, l2 norms, gates, the delta rule on the
//            128x128 state held in registers, then (last workgroup of a head) the gated RMS norm
//            and the Q8_0 quantization of the head's output   engine.rs:2450-2569
//   out    - ssm_out / attn_output GEMV + residual             engine.rs:2573-2609
//   kwrite - k_norm + RoPE + f16 K rows of the run's positions engine.rs:2707-2739
//   entry  - MTP entry eh_proj . [enorm(embd); hnorm(h)]       engine.rs:2362-2390
//   head   - output_norm + LM head GEMV + first-strict-max argmax engine.rs:3630-3715, 1969-1987
#include "oxe_gemv.h"
#include "oxe_model_kernels.h"
#include "oxe_prologue.h"

namespace oxe {

using namespace shp;

__global__ void set_run_kernel(RunCtl *ctl, RunCtl v) { *ctl = v; }
void launch_set_run(RunCtl *ctl, const RunCtl &v, hipStream_t st) {
    hipLaunchKernelGGL(set_run_kernel, dim3(1), dim3(1), 0, st, ctl, v);
}

// ------------------------------------------------------------------------------------------------
// proj: per workgroup, the lanes' normalised + quantised input in LDS, then GEMV tiles.
struct ProjArgs {
    const float *x;
    Q8W emb;            // layer 0: x = embd(tok) (emb.q != null)
    const float *embf;  // layer 0 of a K-quant embedding: the lanes' dequantised rows [NL][E]
    float *x_store;     // workgroup 0 stores the embedded input here (the residual of layer 0)
    const float *norm_w;
    float eps;
    Q8W w;
    int64_t tile0, ntiles;  // tiles [tile0, ntiles) of R rows (MTP seeding: the K and V rows only)
    float *out;         // [NL][out_ld]
    int64_t out_ld;
    int64_t v_row0;     // attention: rows >= v_row0 are V rows (-1: none)
    uint16_t *vt;       // V^T of this layer [NKV*HD][vt_ld]
    int64_t vt_ld;
};

template <int NL>
__global__ __launch_bounds__(GEMV_THREADS) void proj_kernel(const RunCtl *__restrict__ ctl, ProjArgs a) {
    constexpr int R = GemvR<E>::R;
    __shared__ int8_t s_xq[NL][E];
    __shared__ uint16_t s_xd[NL][E / 32];
    __shared__ NormScratch ns;
    __shared__ GemvSmem<E, R, NL> sm;
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        if (l < nl) {
            float v[EPT];
            const bool emb_in = a.emb.q || a.embf;
            if (emb_in) {
                if (a.embf) load8(a.embf + (int64_t)l * E, v);
                else embed8(a.emb, ctl->tok[l], v);
                if (blockIdx.x == 0 && a.x_store) store8(a.x_store + (int64_t)l * E, v);
            } else {
                load8(a.x + (int64_t)l * E, v);
            }
            // replay source for the exact-sum fallback: the stored input (embedding) or x
            const float *xg = emb_in ? nullptr : a.x + (int64_t)l * E;
            if (!xg) {
                // the embedded row is not in memory for every workgroup: recompute on demand
                __shared__ float s_emb[E];
                store8(s_emb, v);
                __syncthreads();
                rms_norm_mul_e(v, s_emb, a.norm_w, a.eps, ns);
            } else {
                rms_norm_mul_e(v, xg, a.norm_w, a.eps, ns);
            }
            quant8(v, &s_xq[l][EPT * t], &s_xd[l][(EPT * t) / 32]);
        } else {
            *(uint2 *)&s_xq[l][EPT * t] = make_uint2(0, 0);
            if ((t & 3) == 0) s_xd[l][(EPT * t) / 32] = 0;
        }
    }
    __syncthreads();
    const int8_t *xq[NL];
    const uint16_t *xd[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) { xq[l] = s_xq[l]; xd[l] = s_xd[l]; }
    const int pos0 = ctl->pos0;
    for (int64_t tile = a.tile0 + blockIdx.x; tile < a.ntiles; tile += gridDim.x) {
        const int64_t row0 = tile * R;
        gemv_tile<E, R, NL>(a.w.q, a.w.d, row0, a.w.rows, xq, xd, sm);
        if (t < NL * R) {
            const int l = t / R, r = t % R;
            const int64_t row = row0 + r;
            if (l < nl && row < a.w.rows) {
                const float v = sm.out[l][r];
                a.out[l * a.out_ld + row] = v;
                if (a.vt && row >= a.v_row0) a.vt[(row - a.v_row0) * a.vt_ld + pos0 + l] = f2h(v);
            }
        }
    }
}

static unsigned grid_for(int64_t ntiles, int64_t cap) { return (unsigned)(ntiles < cap ? ntiles : cap); }

void launch_proj(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const float *x, bool embed, float *x_store,
                 const ActBufs &b, hipStream_t st, int64_t row_begin) {
    ProjArgs a{};
    a.x = x;
    if (embed && m.tok_embd_r.type != 8) a.embf = b.emb;
    else if (embed) a.emb = m.tok_embd;
    a.x_store = x_store;
    a.norm_w = w.attn_norm;
    a.eps = m.eps;
    a.w = w.proj;
    a.tile0 = row_begin / GemvR<E>::R;
    a.ntiles = (w.proj.rows + GemvR<E>::R - 1) / GemvR<E>::R;
    a.out = b.proj;
    a.out_ld = DN_ROWS;
    a.v_row0 = -1;
    if (w.att) {
        a.v_row0 = AT_V;
        a.vt = m.vcache + (int64_t)w.index * NKV * HD * m.n_ctx;
        a.vt_ld = m.n_ctx;
    }
    hipLaunchKernelGGL(proj_kernel<OXE_NL>, dim3(grid_for(a.ntiles - a.tile0, 1024)), dim3(GEMV_THREADS), 0, st, ctl, a);
}

// ------------------------------------------------------------------------------------------------
// delta-net recurrence. Workgroup = one value head vh (1024 threads: 64 row groups x 16 lanes, two
// state rows per row group). Lane c of a row owns state elements i = c + 16 s (s = 0..7), which is
// exactly chain c of ggml_vec_dot_f32's 16 accumulation chains (element i -> accumulator
// (i mod 16) / 4, lane i mod 4), so each row dot is 8 FMAs per lane and the NEON reduction tree
// (a0+a2, a1+a3, a0+a1, then (l0+l1)+(l2+l3)) is the shuffle sequence xor 8, 4, 1, 2. The head's
// 128 outputs stay in LDS for the gated RMS norm and the Q8_0 quantization of the mixer output.
struct DnArgs {
    const float *proj;      // [NL][DN_ROWS]
    const float *conv_w;    // [NCH][KC]
    float *conv_state;      // this layer's slot 0; slot stride conv_slot
    int64_t conv_slot;
    float *ssm;             // this layer's slot 0; slot stride ssm_slot
    int64_t ssm_slot;
    const float *ssm_a, *dt_bias, *ssm_norm;
    float eps;
    int8_t *oq;             // [NL][DIN]
    uint16_t *od;           // [NL][DIN/32]
    float *o32;             // optional: the gated outputs in f32 [NL][DIN] (a K-quant ssm_out)
};

constexpr int DN_THREADS = 1024;

OXE_DEV float dot16_tree(float acc) {
    acc = acc + shfl_xor_f(acc, 8);
    acc = acc + shfl_xor_f(acc, 4);
    acc = acc + shfl_xor_f(acc, 1);
    acc = acc + shfl_xor_f(acc, 2);
    return acc;
}

// causal conv step of one channel (oxe_ssm_conv_step_f32, oxe_ops.cpp:175-201, nc = 4): the four
// products are rounded, then added in order to sumf = +0
OXE_DEV float conv4(float s0, float s1, float s2, float xn, const float *c) {
    const float p0 = s0 * c[0], p1 = s1 * c[1], p2 = s2 * c[2], p3 = xn * c[3];
    float sumf = 0.0f;
    sumf = sumf + p0;
    sumf = sumf + p1;
    sumf = sumf + p2;
    sumf = sumf + p3;
    return sumf;
}

template <int NL>
__global__ __launch_bounds__(DN_THREADS) void dn_kernel(const RunCtl *__restrict__ ctl, DnArgs a) {
    __shared__ float s_q[NL][DS], s_k[NL][DS], s_v[NL][HV], s_o[NL][HV];
    __shared__ float s_g[NL], s_b[NL];
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
    const int vh = blockIdx.x, kh = vh % NKH;
    const int cur = ctl->cur;
    // prefetch this thread's two state rows (slot cur) while the conv runs
    const int rg = t >> 4, c = t & 15;
    float r[2][8];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const float *src = a.ssm + (int64_t)cur * a.ssm_slot + ((int64_t)vh * HV + rg + 64 * h) * HV;
#pragma unroll
        for (int s = 0; s < 8; s++) r[h][s] = src[c + 16 * s];
    }
    // 1. conv + silu of the channels this head reads: q and k of key head kh, v of head vh. Lane l
    //    continues from lane l-1's window and writes slot (cur + l + 1); the q/k channel states are
    //    written by the workgroup of value head kh (the other value head sharing them only reads).
    if (t < 3 * DS) {
        int ch;
        bool writer;
        if (t < DS) { ch = kh * DS + t; writer = vh < NKH; }
        else if (t < 2 * DS) { ch = NKH * DS + kh * DS + (t - DS); writer = vh < NKH; }
        else { ch = 2 * NKH * DS + vh * HV + (t - 2 * DS); writer = true; }
        const float *cw = a.conv_w + (int64_t)ch * KC;
        const float *st = a.conv_state + (int64_t)cur * a.conv_slot + (int64_t)ch * (KC - 1);
        float s0 = st[0], s1 = st[1], s2 = st[2];
        for (int l = 0; l < nl; l++) {
            const float xn = a.proj[(int64_t)l * DN_ROWS + ch];
            const float y = v_silu(conv4(s0, s1, s2, xn, cw));
            s0 = s1; s1 = s2; s2 = xn;
            if (writer) {
                float *dst = a.conv_state + (int64_t)((cur + l + 1) % OXE_NSLOTS) * a.conv_slot + (int64_t)ch * (KC - 1);
                dst[0] = s0; dst[1] = s1; dst[2] = s2;
            }
            if (t < DS) s_q[l][t] = y;
            else if (t < 2 * DS) s_k[l][t - DS] = y;
            else s_v[l][t - 2 * DS] = y;
        }
    }
    __syncthreads();
    // 2. l2 norms of q and k per lane (oxe_gdn_l2_norm_f32: rms_norm with eps/n, then * 1/sqrt(n)),
    //    one wave per (lane, q|k) vector; the gates (engine.rs:2509-2524) on wave 4
    {
        const int w = t >> 6, lane = t & 63;
        if (w < 2 * NL && (w >> 1) < nl) {
            const int l = w >> 1;
            float *x = (w & 1) ? s_k[l] : s_q[l];
            const float a0 = x[lane], a1 = x[lane + 64];
            const float nf = (float)DS;
            const float mean = wave_mean_sq_128(a0, a1, x);
            const float scale = 1.0f / sqrtf(mean + a.eps / nf);
            const float s2 = 1.0f / sqrtf(nf);
            x[lane] = (a0 * scale) * s2;
            x[lane + 64] = (a1 * scale) * s2;
        }
        if (w == 2 * NL && lane < nl) {
            const float ab = a.proj[(int64_t)lane * DN_ROWS + DN_ALPHA + vh] + a.dt_bias[vh];
            s_g[lane] = oxe_libm::expf_c(softplus_c(ab) * a.ssm_a[vh]);   // e^g of the step
            s_b[lane] = sigmoid_c(a.proj[(int64_t)lane * DN_ROWS + DN_BETA + vh]);
        }
    }
    __syncthreads();
    // 3. delta rule (oxe_gated_delta_net_step_f32_x4_from, oxe_ops.cpp:268-345) on rows rg, rg + 64
    const float scale = 1.0f / sqrtf((float)HV);
    for (int l = 0; l < nl; l++) {
        const float eg = s_g[l], beta = s_b[l];
#pragma unroll
        for (int h = 0; h < 2; h++) {
            const int j = rg + 64 * h;
            float acc = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                r[h][s] = r[h][s] * eg;
                acc = __builtin_fmaf(r[h][s], s_k[l][c + 16 * s], acc);
            }
            const float s1 = dot16_tree(acc);
            const float delta = (s_v[l][j] - s1) * beta;
            acc = 0.0f;
#pragma unroll
            for (int s = 0; s < 8; s++) {
                r[h][s] = __builtin_fmaf(s_k[l][c + 16 * s], delta, r[h][s]);
                acc = __builtin_fmaf(r[h][s], s_q[l][c + 16 * s], acc);
            }
            const float s2 = dot16_tree(acc);
            float *dst = a.ssm + (int64_t)((cur + l + 1) % OXE_NSLOTS) * a.ssm_slot + ((int64_t)vh * HV + j) * HV;
#pragma unroll
            for (int s = 0; s < 8; s++) dst[c + 16 * s] = r[h][s];
            if (c == 0) s_o[l][j] = s2 * scale;
        }
    }
    __syncthreads();
    // 4. gated RMS norm with z (engine.rs:2560-2566: o = rms_norm(out) * ssm_norm * silu(z)) and the
    //    Q8_0 quantization of the head's 128 outputs, one wave per lane
    {
        const int w = t >> 6, lane = t & 63;
        if (w < nl) {
            const int l = w;
            const float x0 = s_o[l][lane], x1 = s_o[l][lane + 64];
            const float mean = wave_mean_sq_128(x0, x1, s_o[l]);
            const float sc = 1.0f / sqrtf(mean + a.eps);
            const float *z = a.proj + (int64_t)l * DN_ROWS + DN_Z + vh * HV;
            const float o0 = ((x0 * sc) * a.ssm_norm[lane]) * v_silu(z[lane]);
            const float o1 = ((x1 * sc) * a.ssm_norm[lane + 64]) * v_silu(z[lane + 64]);
            if (a.o32) {
                a.o32[(int64_t)l * DIN + vh * HV + lane] = o0;
                a.o32[(int64_t)l * DIN + vh * HV + lane + 64] = o1;
            }
            // Q8_0 blocks of 32: lanes 0..31 hold blocks 0 (o0) and 2 (o1), lanes 32..63 blocks 1 and 3
            float m0 = __builtin_fabsf(o0), m1 = __builtin_fabsf(o1);
            for (int mm = 16; mm >= 1; mm >>= 1) {
                m0 = fmaxf(m0, shfl_xor_f(m0, mm));
                m1 = fmaxf(m1, shfl_xor_f(m1, mm));
            }
            const float d0 = m0 / 127.0f, d1 = m1 / 127.0f;
            const float id0 = d0 != 0.0f ? 1.0f / d0 : 0.0f, id1 = d1 != 0.0f ? 1.0f / d1 : 0.0f;
            int8_t *q = a.oq + (int64_t)l * DIN + vh * HV;
            q[lane] = (int8_t)(int32_t)__builtin_rintf(o0 * id0);
            q[lane + 64] = (int8_t)(int32_t)__builtin_rintf(o1 * id1);
            uint16_t *d = a.od + (int64_t)l * (DIN / 32) + vh * (HV / 32);
            if (lane == 0) { d[0] = f2h(d0); d[2] = f2h(d1); }
            if (lane == 32) { d[1] = f2h(d0); d[3] = f2h(d1); }
        }
    }
}

void launch_dn(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st, float *o32) {
    DnArgs a{};
    a.proj = b.proj;
    a.conv_w = w.conv;
    a.conv_slot = (int64_t)m.n_rec * NCH * (KC - 1);
    a.conv_state = m.conv_state + (int64_t)w.index * NCH * (KC - 1);
    a.ssm_slot = (int64_t)m.n_rec * NVH * HV * HV;
    a.ssm = m.ssm_state + (int64_t)w.index * NVH * HV * HV;
    a.ssm_a = w.ssm_a;
    a.dt_bias = w.dt_bias;
    a.ssm_norm = w.ssm_norm;
    a.eps = m.eps;
    a.oq = b.oq;
    a.od = b.od;
    a.o32 = o32;
    hipLaunchKernelGGL(dn_kernel<OXE_NL>, dim3(NVH), dim3(DN_THREADS), 0, st, ctl, a);
}

// ------------------------------------------------------------------------------------------------
// out: GEMV over the quantised mixer output + residual x1 = out + x
struct EpiResidual {
    const RunCtl *ctl;
    float *y;          // [NL][E]
    const float *res;  // [NL][E]
    template <int NL, int R>
    OXE_DEV void tile(int64_t row0, int nvalid, const float (&out)[NL][R]) const {
        const int nl = ctl->nl;
        for (int i = threadIdx.x; i < NL * R; i += GEMV_THREADS) {
            const int l = i / R, r = i % R;
            if (l < nl && r < nvalid) y[(int64_t)l * E + row0 + r] = out[l][r] + res[(int64_t)l * E + row0 + r];
        }
    }
};

template <int NL>
__global__ __launch_bounds__(GEMV_THREADS) void out_kernel(const RunCtl *__restrict__ ctl, Q8W w, const int8_t *oq,
                                                           const uint16_t *od, EpiResidual epi) {
    constexpr int K = MIX_W, R = GemvR<K>::R;
    __shared__ GemvSmem<K, R, NL> sm;
    if (!ctl->active) return;
    const int8_t *xq[NL];
    const uint16_t *xd[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) { xq[l] = oq + (int64_t)l * K; xd[l] = od + (int64_t)l * (K / 32); }
    const int64_t row0 = (int64_t)blockIdx.x * R;
    gemv_tile<K, R, NL>(w.q, w.d, row0, w.rows, xq, xd, sm);
    epi.template tile<NL, R>(row0, R, sm.out);
}

void launch_out(const RunCtl *ctl, const LayerW &w, const float *x, const ActBufs &b, hipStream_t st) {
    EpiResidual epi{ctl, b.x1, x};
    hipLaunchKernelGGL(out_kernel<OXE_NL>, dim3((unsigned)(E / GemvR<MIX_W>::R)), dim3(GEMV_THREADS), 0, st, ctl,
                       w.out, b.oq, b.od, epi);
}

// ------------------------------------------------------------------------------------------------
// kwrite: K rows of the run's positions (write_k, engine.rs:2707-2739): k = rope(rms_norm(kraw) *
// k_norm) -> f16 K cache [att][kv head][pos][HD]. Workgroup (lane, kv head), one wave per job.
__global__ __launch_bounds__(64) void kwrite_kernel(const RunCtl *__restrict__ ctl, const float *proj,
                                                    const float *k_norm, const float *rope, uint16_t *kc, int n_ctx,
                                                    float eps) {
    __shared__ float s_k[HD];
    if (!ctl->active) return;
    const int l = blockIdx.x / NKV, kvh = blockIdx.x % NKV, lane = threadIdx.x;
    if (l >= ctl->nl) return;
    const int pos = ctl->pos0 + l;
    const float *kr = proj + (int64_t)l * DN_ROWS + AT_K + kvh * HD;
    float v[4];
#pragma unroll
    for (int i = 0; i < 4; i++) v[i] = kr[lane + 64 * i];
    const float mean = wave_mean_sq_256(v, kr);
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int i = 0; i < 4; i++) s_k[lane + 64 * i] = (v[i] * scale) * k_norm[lane + 64 * i];
    __syncthreads();
    rope_neox_lds(s_k, rope + (int64_t)pos * NROT, lane);
    __syncthreads();
    uint16_t *dst = kc + ((int64_t)kvh * n_ctx + pos) * HD;
#pragma unroll
    for (int i = 0; i < 4; i++) dst[lane + 64 * i] = f2h(s_k[lane + 64 * i]);
}

void launch_kwrite(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st) {
    uint16_t *kc = m.kcache + (int64_t)w.index * NKV * m.n_ctx * HD;
    hipLaunchKernelGGL(kwrite_kernel, dim3(OXE_NL * NKV), dim3(64), 0, st, ctl, b.proj, w.k_norm, m.rope, kc, m.n_ctx,
                       m.eps);
}

// ------------------------------------------------------------------------------------------------
// entry (MTP): x2[l] = eh_proj . quantize([rms_norm(embd(tok), enorm); rms_norm(h, hnorm)])
template <int NL>
__global__ __launch_bounds__(GEMV_THREADS) void entry_kernel(const RunCtl *__restrict__ ctl, Q8W emb, const float *embf,
                                                             Q8W w, const float *enorm, const float *hnorm,
                                                             const float *hid, float *x2, float eps) {
    constexpr int K = 2 * E, R = GemvR<K>::R;
    __shared__ int8_t s_xq[NL][K];
    __shared__ uint16_t s_xd[NL][K / 32];
    __shared__ float s_emb[E];
    __shared__ NormScratch ns;
    __shared__ GemvSmem<K, R, NL> sm;
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        if (l < nl) {
            float v[EPT];
            if (embf) load8(embf + (int64_t)l * E, v);   // a K-quant embedding's dequantised row
            else embed8(emb, ctl->tok[l], v);
            store8(s_emb, v);
            __syncthreads();
            rms_norm_mul_e(v, s_emb, enorm, eps, ns);
            quant8(v, &s_xq[l][EPT * t], &s_xd[l][(EPT * t) / 32]);
            const float *h = hid + (int64_t)ctl->hin_sel[l] * E;
            load8(h, v);
            rms_norm_mul_e(v, h, hnorm, eps, ns);
            quant8(v, &s_xq[l][E + EPT * t], &s_xd[l][(E + EPT * t) / 32]);
            __syncthreads();
        } else {
            *(uint2 *)&s_xq[l][EPT * t] = make_uint2(0, 0);
            *(uint2 *)&s_xq[l][E + EPT * t] = make_uint2(0, 0);
            if ((t & 3) == 0) { s_xd[l][(EPT * t) / 32] = 0; s_xd[l][(E + EPT * t) / 32] = 0; }
        }
    }
    __syncthreads();
    const int8_t *xq[NL];
    const uint16_t *xd[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) { xq[l] = s_xq[l]; xd[l] = s_xd[l]; }
    for (int64_t tile = blockIdx.x; tile < E / R; tile += gridDim.x) {
        gemv_tile<K, R, NL>(w.q, w.d, tile * R, w.rows, xq, xd, sm);
        if (t < NL * R) {
            const int l = t / R, r = t % R;
            if (l < nl) x2[(int64_t)l * E + tile * R + r] = sm.out[l][r];
        }
    }
}

void launch_entry(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st,
                  const float *emb) {
    hipLaunchKernelGGL(entry_kernel<OXE_NL>, dim3(E / GemvR<2 * E>::R), dim3(GEMV_THREADS), 0, st, ctl, m.tok_embd, emb,
                       w.eh_proj, w.enorm, w.hnorm, b.hid, b.x2, m.eps);
}

// ------------------------------------------------------------------------------------------------
// head: xn = rms_norm(x2) * norm -> h_nextn (hid[l]); logits = LM head GEMV; argmax = first strict
// maximum in row order, values above -inf only (NaN never wins), else row 0. Each workgroup keeps
// its running first strict maximum over ascending rows; the global pick is an atomic max of
// (ordered value << 32 | ~row), i.e. the largest value, then the smallest row.
OXE_DEV uint32_t ordered_bits(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

template <int NL>
__global__ __launch_bounds__(GEMV_THREADS) void head_kernel(const RunCtl *__restrict__ ctl, const float *x2,
                                                            const float *norm_w, float eps, Q8W w, int64_t ntiles,
                                                            float *hid, float *logits,
                                                            unsigned long long *amax_key, const uint32_t *ids) {
    constexpr int R = GemvR<E>::R;
    __shared__ int8_t s_xq[NL][E];
    __shared__ uint16_t s_xd[NL][E / 32];
    __shared__ NormScratch ns;
    __shared__ GemvSmem<E, R, NL> sm;
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x, mask = ctl->head_mask;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        if (l < nl) {
            float v[EPT];
            load8(x2 + (int64_t)l * E, v);
            rms_norm_mul_e(v, x2 + (int64_t)l * E, norm_w, eps, ns);
            if (blockIdx.x == 0) store8(hid + (int64_t)l * E, v);
            quant8(v, &s_xq[l][EPT * t], &s_xd[l][(EPT * t) / 32]);
        } else {
            *(uint2 *)&s_xq[l][EPT * t] = make_uint2(0, 0);
            if ((t & 3) == 0) s_xd[l][(EPT * t) / 32] = 0;
        }
    }
    if (mask == 0) return;
    __syncthreads();
    const int8_t *xq[NL];
    const uint16_t *xd[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) { xq[l] = s_xq[l]; xd[l] = s_xd[l]; }
    float best = -__builtin_inff();
    int64_t bi = -1;
    for (int64_t tile = blockIdx.x; tile < ntiles; tile += gridDim.x) {
        const int64_t row0 = tile * R;
        gemv_tile<E, R, NL>(w.q, w.d, row0, w.rows, xq, xd, sm);
        if (logits && t < NL * R) {
            const int l = t / R, r = t % R;
            if (l < nl && row0 + r < w.rows) logits[l * w.rows + row0 + r] = sm.out[l][r];
        }
        if (t < NL && t < nl && (mask >> t) & 1) {
            for (int r = 0; r < R && row0 + r < w.rows; r++) {
                const float v = sm.out[t][r];
                if (v > best) { best = v; bi = row0 + r; }
            }
        }
    }
    if (t < NL && t < nl && ((mask >> t) & 1) && bi >= 0) {
        // a restricted draft head's rows are ascending token ids (ids[row]): the first maximum by
        // row is the first by id
        const uint32_t id = ids ? ids[bi] : (uint32_t)bi;
        const unsigned long long key = ((unsigned long long)ordered_bits(best) << 32) | (0xffffffffu - id);
        atomicMax(&amax_key[t], key);
    }
}

void launch_head(const RunCtl *ctl, const ModelRt &m, const float *norm_w, const ActBufs &b, bool store_logits,
                 hipStream_t st, const Q8W *w, const uint32_t *ids) {
    const Q8W &hw = w ? *w : m.output;
    const int64_t ntiles = (hw.rows + GemvR<E>::R - 1) / GemvR<E>::R;
    hipLaunchKernelGGL(head_kernel<OXE_NL>, dim3(grid_for(ntiles, 2048)), dim3(GEMV_THREADS), 0, st, ctl, b.x2,
                       norm_w, m.eps, hw, ntiles, b.hid, store_logits ? b.logits : nullptr, b.amax_key, ids);
}

}  // namespace oxe

namespace oxe {
// V^T entries of rejected positions [p0, p1) of the main attention layers back to +0 (zero_v,
// crates/model/src/engine.rs:1616-1638), so later full-length V^T . p dots see a fresh cache.
__global__ void zero_v_kernel(uint16_t *vt, int64_t rows, int n_ctx, int p0, int p1) {
    const int64_t r = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (r < rows)
        for (int p = p0; p < p1; p++) vt[r * n_ctx + p] = 0;
}
void launch_zero_v(const ModelRt &m, int n_att_main, int p0, int p1, hipStream_t st) {
    if (p1 <= p0) return;
    const int64_t rows = (int64_t)n_att_main * shp::NKV * shp::HD;
    hipLaunchKernelGGL(zero_v_kernel, dim3((unsigned)((rows + 255) / 256)), dim3(256), 0, st, m.vcache, rows, m.n_ctx, p0, p1);
}
}  // namespace oxe
