// GQA decode attention for 1-2 lanes, FA-off numerics of the reference (oxe_attn_head_f16,
// crates/kernels-sys/csrc/oxe_ops.cpp:465-493; tiled form 595-662, 725-770):
//   score(p) = ggml_vec_dot_f16(K_p, f16(q))  for p <= pos (4 x 8 fp16 FMA chains + F16x8 reduce)
//   softmax over n_kv = min(n_ctx, max(256, pad256(pos + 1))) with scale 1/16 and the -inf mask
//   out_d    = ggml_vec_dot_f16(V^T_d, f16(p)) over all n_kv positions (masked p = +0)
//   o        = out * sigmoid(gate)
// Two kernels: `scores` (workgroup = kv head x 64 positions: each K row is loaded once for the
// 8 query heads of its group and both lanes) and `pv` (workgroup = kv head x lane x 32 output
// dims: the softmax of the group's 8 heads, then V^T . p with each V^T row loaded once for the 8
// heads), which also applies the gate and quantises the 32-dim Q8_0 block it owns.
// fp16 FMAs use v_pk_fma_f16 (IEEE fused, one binary16 rounding = vfmaq_f16); the accumulator
// of chain (j, l) takes positions 32 s + 8 j + l in increasing s, as in the reference.
#include "oxe_model_kernels.h"
#include "oxe_prologue.h"

namespace oxe {

using namespace shp;
typedef _Float16 h2 __attribute__((ext_vector_type(2)));

OXE_DEV h2 u2h2(uint32_t u) { return __builtin_bit_cast(h2, u); }
OXE_DEV uint32_t h22u(h2 v) { return __builtin_bit_cast(uint32_t, v); }

// GGML_F16x8_REDUCE of the 4 accumulators held by the 4 lanes j of a quad (lane bits 0-1), then
// the f32 widening and vaddvq: returns the dot in every lane of the quad.
OXE_DEV float f16x8_reduce_quad(h2 a[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) a[i] = a[i] + u2h2(__shfl_xor(h22u(a[i]), 2, 64));   // a0+a2, a1+a3
#pragma unroll
    for (int i = 0; i < 4; i++) a[i] = a[i] + u2h2(__shfl_xor(h22u(a[i]), 1, 64));   // a0+a1
    // halves: a[0] = (l0, l1), a[1] = (l2, l3), a[2] = (l4, l5), a[3] = (l6, l7)
    const float t0 = (float)a[0].x + (float)a[2].x;
    const float t1 = (float)a[0].y + (float)a[2].y;
    const float t2 = (float)a[1].x + (float)a[3].x;
    const float t3 = (float)a[1].y + (float)a[3].y;
    return (t0 + t1) + (t2 + t3);
}

// ------------------------------------------------------------------------------------------------
struct ScoreArgs {
    const float *proj;      // [NL][DN_ROWS]: q+gate rows per head
    const float *q_norm;
    const float *rope;      // [n_ctx][NROT]
    const uint16_t *kc;     // this layer's K cache [NKV][n_ctx][HD]
    float *scores;          // [NL][NH][n_ctx]
    int n_ctx;
    float eps;
};

constexpr int SC_POS = 64;  // positions per workgroup

template <int NL>
__global__ __launch_bounds__(256) void scores_kernel(const RunCtl *__restrict__ ctl, ScoreArgs a) {
    __shared__ uint16_t s_q[NL * GQA][HD];
    __shared__ float s_tmp[4][HD];
    if (!ctl->active) return;
    const int nl = ctl->nl, pos0 = ctl->pos0, t = threadIdx.x;
    const int kvh = blockIdx.x % NKV, chunk = blockIdx.x / NKV;
    const int pmax = pos0 + nl - 1;
    if (chunk * SC_POS > pmax) return;
    // q = rope(rms_norm(q_raw) * q_norm) -> f16, one wave per (lane, head) vector, 4 at a time
    {
        const int w = t >> 6, lane = t & 63;
        for (int k = 0; k < NL * GQA / 4; k++) {
            const int job = w + 4 * k, l = job / GQA, hh = job % GQA, h = kvh * GQA + hh;
            float *x = s_tmp[w];
            if (l < nl) {
                const float *q = a.proj + (int64_t)l * DN_ROWS + h * 2 * HD;
                float v[4];
#pragma unroll
                for (int i = 0; i < 4; i++) v[i] = q[lane + 64 * i];
                const float mean = wave_mean_sq_256(v, q);
                const float scale = 1.0f / sqrtf(mean + a.eps);
#pragma unroll
                for (int i = 0; i < 4; i++) x[lane + 64 * i] = (v[i] * scale) * a.q_norm[lane + 64 * i];
            }
            __syncthreads();
            if (l < nl) rope_neox_lds(x, a.rope + (int64_t)(pos0 + l) * NROT, lane);
            __syncthreads();
#pragma unroll
            for (int i = 0; i < 4; i++) s_q[job][lane + 64 * i] = l < nl ? f2h(x[lane + 64 * i]) : (uint16_t)0;
            __syncthreads();
        }
    }
    const int p = chunk * SC_POS + (t >> 2), j = t & 3;
    if (p > pmax) return;
    const uint16_t *krow = a.kc + ((int64_t)kvh * a.n_ctx + p) * HD;
    h2 acc[NL * GQA][4];
#pragma unroll
    for (int q = 0; q < NL * GQA; q++)
#pragma unroll
        for (int i = 0; i < 4; i++) acc[q][i] = h2{(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
    for (int s = 0; s < HD / 32; s++) {
        const uint4 kv = *(const uint4 *)(krow + 32 * s + 8 * j);
        const h2 k0 = u2h2(kv.x), k1 = u2h2(kv.y), k2 = u2h2(kv.z), k3 = u2h2(kv.w);
#pragma unroll
        for (int q = 0; q < NL * GQA; q++) {
            const uint4 qv = *(const uint4 *)(&s_q[q][32 * s + 8 * j]);
            acc[q][0] = __builtin_elementwise_fma(k0, u2h2(qv.x), acc[q][0]);
            acc[q][1] = __builtin_elementwise_fma(k1, u2h2(qv.y), acc[q][1]);
            acc[q][2] = __builtin_elementwise_fma(k2, u2h2(qv.z), acc[q][2]);
            acc[q][3] = __builtin_elementwise_fma(k3, u2h2(qv.w), acc[q][3]);
        }
    }
#pragma unroll
    for (int q = 0; q < NL * GQA; q++) {
        const float sc = f16x8_reduce_quad(acc[q]);
        const int l = q / GQA, h = kvh * GQA + q % GQA;
        if (j == 0 && l < nl && p <= pos0 + l) a.scores[((int64_t)l * NH + h) * a.n_ctx + p] = sc;
    }
}

void launch_scores(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st) {
    ScoreArgs a{};
    a.proj = b.proj;
    a.q_norm = w.q_norm;
    a.rope = m.rope;
    a.kc = m.kcache + (int64_t)w.index * NKV * m.n_ctx * HD;
    a.scores = b.scores;
    a.n_ctx = m.n_ctx;
    a.eps = m.eps;
    const unsigned grid = (unsigned)(NKV * ((m.n_ctx + SC_POS - 1) / SC_POS));
    hipLaunchKernelGGL(scores_kernel<OXE_NL>, dim3(grid), dim3(256), 0, st, ctl, a);
}

// ------------------------------------------------------------------------------------------------
struct PvArgs {
    const float *proj;      // gates
    const float *scores;    // [NL][NH][n_ctx]
    const uint16_t *vt;     // this layer's V^T [NKV*HD][n_ctx]
    int8_t *oq;             // [NL][MIX_W]
    uint16_t *od;
    float *o32;             // optional: the gated outputs in f32 [NL][MIX_W] (a K-quant attn_output)
    int n_ctx;
};

constexpr int PV_D = 32;            // output dims per workgroup (one Q8_0 block of one head)
constexpr int PV_MAX_KV = 8192;     // LDS holds the head's f16 probabilities for n_kv <= this

// workgroup (kv head kvh, lane l, 32-dim chunk, head hh of the GQA group): 256 workgroups, the
// chunk's V^T rows shared through the cache by the group's 8 heads
template <int NL>
__global__ __launch_bounds__(256) void pv_kernel(const RunCtl *__restrict__ ctl, PvArgs a) {
    extern __shared__ uint16_t s_dyn[];
    uint16_t *s_p = s_dyn;                                        // [n_kv]
    float *s_e = (float *)(s_dyn + ((a.n_ctx + 1) & ~1));         // [n_kv]
    __shared__ float s_gs[PV_MAX_KV / 4];
    __shared__ double s_red[8];
    __shared__ float s_o[PV_D];
    if (!ctl->active) return;
    const int t = threadIdx.x;
    const int hh = blockIdx.x % GQA;
    const int dchunk = (blockIdx.x / GQA) % (HD / PV_D);
    const int l = (blockIdx.x / (GQA * (HD / PV_D))) % NL;
    const int kvh = blockIdx.x / (GQA * (HD / PV_D) * NL);
    if (l >= ctl->nl) return;
    const int pos = ctl->pos0 + l;
    int n_kv = (pos + 1 + 255) / 256 * 256;
    if (n_kv < 256) n_kv = 256;
    if (n_kv > a.n_ctx) n_kv = a.n_ctx;
    const float scale = 1.0f / sqrtf((float)HD);
    const int h = kvh * GQA + hh;
    // softmax of the head's row (oxe_soft_max_f32, oxe_ops.cpp:101-115)
    {
        const float *sc = a.scores + ((int64_t)l * NH + h) * a.n_ctx;
        float mx = -__builtin_inff();
        for (int i = t; i < n_kv; i += 256) {
            const float wv = i <= pos ? sc[i] * scale : -__builtin_inff();
            s_e[i] = wv;
            mx = (mx > wv) ? mx : wv;
        }
        __shared__ float s_mx[8];
        mx = block_max_f<256>(mx, s_mx);
        double part = 0.0;
        for (int i0 = 0; i0 < n_kv; i0 += 256) {
            const int i = i0 + t;
            const float e = i < n_kv ? v_expf(s_e[i] - mx) : 0.0f;
            if (i < n_kv) s_e[i] = e;
            float g = e + shfl_xor_f(e, 1);       // (v0 + v1), (v2 + v3)
            g = g + shfl_xor_f(g, 2);             // (v0 + v1) + (v2 + v3)
            if ((t & 3) == 0 && i < n_kv) {
                s_gs[i >> 2] = g;
                part += (double)g;
            }
        }
        const double P = block_sum_d<256>(part, s_red);
        float f;
        if (!bracket_ok_recip(P, P, n_kv / 4, &f)) {
            if (t == 0) {
                double s = 0.0;
                for (int g = 0; g < n_kv / 4; g++) s += (double)s_gs[g];
                s_red[0] = s;
            }
            __syncthreads();
            f = (float)(1.0 / s_red[0]);
            __syncthreads();
        }
        for (int i = t; i < n_kv; i += 256) s_p[i] = f2h(s_e[i] * f);
        __syncthreads();
    }
    // V^T . p: thread = (dim d, chain octet j) of ggml_vec_dot_f16 (threads >= 128 idle)
    const int j = t & 3, d = (t >> 2) & (PV_D - 1);
    const int dg = dchunk * PV_D + d;
    if (t < 4 * PV_D) {
        const uint16_t *vrow = a.vt + (int64_t)(kvh * HD + dg) * a.n_ctx;
        h2 acc[4];
#pragma unroll
        for (int i = 0; i < 4; i++) acc[i] = h2{(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll 4
        for (int s = 0; s < n_kv / 32; s++) {
            const uint4 vv = *(const uint4 *)(vrow + 32 * s + 8 * j);
            const uint4 pv = *(const uint4 *)(&s_p[32 * s + 8 * j]);
            acc[0] = __builtin_elementwise_fma(u2h2(vv.x), u2h2(pv.x), acc[0]);
            acc[1] = __builtin_elementwise_fma(u2h2(vv.y), u2h2(pv.y), acc[1]);
            acc[2] = __builtin_elementwise_fma(u2h2(vv.z), u2h2(pv.z), acc[2]);
            acc[3] = __builtin_elementwise_fma(u2h2(vv.w), u2h2(pv.w), acc[3]);
        }
        const float out = f16x8_reduce_quad(acc);
        if (j == 0) {
            const float gate = a.proj[(int64_t)l * DN_ROWS + h * 2 * HD + HD + dg];
            s_o[d] = out * sigmoid_c(gate);
            if (a.o32) a.o32[(int64_t)l * MIX_W + h * HD + dg] = s_o[d];
        }
    }
    __syncthreads();
    if (t == 0) {
        const int64_t off = (int64_t)l * MIX_W + h * HD + dchunk * PV_D;
        quant_block_q8_0(s_o, a.oq + off, a.od + off / 32);
    }
}

void launch_pv(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st, float *o32) {
    PvArgs a{};
    a.o32 = o32;
    a.proj = b.proj;
    a.scores = b.scores;
    a.vt = m.vcache + (int64_t)w.index * NKV * HD * m.n_ctx;
    a.oq = b.oq;
    a.od = b.od;
    a.n_ctx = m.n_ctx;
    const size_t lds = (size_t)((m.n_ctx + 1) & ~1) * 2 + (size_t)m.n_ctx * 4;
    static size_t configured = 0;
    if (lds > configured) {
        (void)hipFuncSetAttribute((const void *)pv_kernel<OXE_NL>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        configured = lds;
    }
    hipLaunchKernelGGL(pv_kernel<OXE_NL>, dim3(NKV * OXE_NL * (HD / PV_D) * GQA), dim3(256), lds, st, ctl, a);
}

}  // namespace oxe
