// MoE FFN of one layer for 1-2 lanes (reference crates/model/src/engine.rs:3372-3624):
//   router  - post_attention_norm + quantize (prologue); router logits (f32 dots in ggml_vec_dot_f32
//             order), the shared-expert gate sigmoid(dot), the shared expert's gate/up GEMV + swiglu
//   experts - routing (softmax, top-8, renormalised weights, union of the lanes' experts) in every
//             workgroup, then gate/up GEMV + swiglu of (union expert, 16-row tile) units
//   down    - per 8 output rows: the down GEMV of every union expert and of the shared expert (all
//             weight loads issued before any arithmetic), then the reference's combine order
//             m = d0 w0; m += dj wj; f = m + dsh * g; x2 = f + x1
#include "oxe_gemv.h"
#include "oxe_model_kernels.h"
#include "oxe_prologue.h"

namespace oxe {

using namespace shp;

// ------------------------------------------------------------------------------------------------
constexpr int RT_ROW_WG = NEXP / 16;       // 16 router workgroups of 16 rows
constexpr int RT_SH_WG = 1;                // shared-gate dot
constexpr int RT_GU_TILES = 2 * FFSH / 16; // 64 shared gate/up tiles

struct RouterArgs {
    const float *x1;
    const float *post_norm;
    float eps;
    const float *router;      // [NEXP][E]
    const float *shexp_gate;  // [E]
    Q8W shexp_gu;
    float *router_lg;         // [NL][NEXP]
    float *sh_gate;           // [NL]
    float *hsh;               // [NL][FFSH]
    int8_t *xq;               // [NL][2E] (first E used)
    uint16_t *xd;
    float *xn;                // [NL][E]
};

template <int NL>
__global__ __launch_bounds__(256) void router_kernel(const RunCtl *__restrict__ ctl, RouterArgs a) {
    constexpr int R = GemvR<E>::R;
    __shared__ float s_xn[NL][E];
    __shared__ int8_t s_xq[NL][E];
    __shared__ uint16_t s_xd[NL][E / 32];
    __shared__ NormScratch ns;
    __shared__ GemvSmem<E, R, NL> sm;
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        float v[EPT];
        if (l < nl) {
            load8(a.x1 + (int64_t)l * E, v);
            rms_norm_mul_e(v, a.x1 + (int64_t)l * E, a.post_norm, a.eps, ns);
        } else {
#pragma unroll
            for (int i = 0; i < EPT; i++) v[i] = 0.0f;
        }
        store8(s_xn[l], v);
        quant8(v, &s_xq[l][EPT * t], &s_xd[l][(EPT * t) / 32]);
        if (blockIdx.x == 0) {
            store8(a.xn + (int64_t)l * E, v);
            *(uint2 *)(a.xq + (int64_t)l * 2 * E + EPT * t) = *(const uint2 *)&s_xq[l][EPT * t];
        }
    }
    __syncthreads();
    if (blockIdx.x == 0 && t < NL * (E / 32)) a.xd[(t / (E / 32)) * (2 * E / 32) + t % (E / 32)] = s_xd[t / (E / 32)][t % (E / 32)];
    const int b = blockIdx.x;
    if (b < RT_ROW_WG + RT_SH_WG) {
        // f32 dots in ggml_vec_dot_f32 order: lane c of a 16-lane group runs chain c (elements
        // c + 16 s); xor 8, 4, 1, 2 is the NEON reduction tree
        const int c = t & 15, rr = t >> 4;
        const bool sh = b == RT_ROW_WG;
        if (sh && rr > 0) return;
        const float *w = sh ? a.shexp_gate : a.router + (int64_t)(b * 16 + rr) * E;
        float acc[NL];
#pragma unroll
        for (int l = 0; l < NL; l++) acc[l] = 0.0f;
        for (int s = 0; s < E / 16; s++) {
            const float wv = w[c + 16 * s];
#pragma unroll
            for (int l = 0; l < NL; l++) acc[l] = __builtin_fmaf(wv, s_xn[l][c + 16 * s], acc[l]);
        }
#pragma unroll
        for (int l = 0; l < NL; l++) {
            float v = acc[l];
            v = v + shfl_xor_f(v, 8);
            v = v + shfl_xor_f(v, 4);
            v = v + shfl_xor_f(v, 1);
            v = v + shfl_xor_f(v, 2);
            if (c == 0 && l < nl) {
                if (sh) a.sh_gate[l] = sigmoid_c(v);
                else a.router_lg[l * NEXP + b * 16 + rr] = v;
            }
        }
        return;
    }
    // shared expert gate/up tile: rows 16*tile .. (8 gate rows then 8 up rows) -> 8 h values
    const int tile = b - RT_ROW_WG - RT_SH_WG;
    const int8_t *xq[NL];
    const uint16_t *xd[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) { xq[l] = s_xq[l]; xd[l] = s_xd[l]; }
    gemv_tile<E, R, NL>(a.shexp_gu.q, a.shexp_gu.d, (int64_t)tile * R, a.shexp_gu.rows, xq, xd, sm);
    if (t < NL * 8) {
        const int l = t / 8, r = t % 8;
        if (l < nl) a.hsh[l * FFSH + tile * 8 + r] = v_silu(sm.out[l][r]) * sm.out[l][8 + r];
    }
}

void launch_router(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st) {
    RouterArgs a{};
    a.x1 = b.x1;
    a.post_norm = w.post_norm;
    a.eps = m.eps;
    a.router = w.router;
    a.shexp_gate = w.shexp_gate;
    a.shexp_gu = w.shexp_gu;
    a.router_lg = b.router_lg;
    a.sh_gate = b.sh_gate;
    a.hsh = b.hsh;
    a.xq = b.xq;
    a.xd = b.xd;
    a.xn = b.xn;
    hipLaunchKernelGGL(router_kernel<OXE_NL>, dim3(RT_ROW_WG + RT_SH_WG + RT_GU_TILES), dim3(256), 0, st, ctl, a);
}

// ------------------------------------------------------------------------------------------------
// Routing of one lane (engine.rs:3414-3429) by 256 threads (thread t = expert t):
//   probs = oxe_soft_max_f32(logits, scale 1, no mask); ids = oxe_argsort_top_k_f32(probs, 8)
//   w_j = probs[ids_j]; s = clamp(ggml_vec_sum_f32(w), 6.103515625e-5, inf); w_j /= s
// Ties among the 9 largest probabilities (where the reference falls back to std::sort) are
// counted in *tie_cnt; the order used is then descending value, ascending index.
struct RouteSmem {
    float p[NEXP];
    float gs[NEXP / 4];
    double red[8];
    float mx[8];
    int32_t ids[OXE_NL][KUSED];
    float w[OXE_NL][KUSED];
    int32_t uni[OXE_MAX_UNION];
    int32_t n_uni;
    int32_t tie;
};

template <int NL>
OXE_DEV void route_all(const RunCtl *ctl, const float *router_lg, RouteSmem &rs, uint32_t *tie_cnt, bool count_ties) {
    const int nl = ctl->nl, t = threadIdx.x;
    if (t == 0) rs.tie = 0;
    if (t < OXE_NL * KUSED) { rs.ids[t / KUSED][t % KUSED] = 0; rs.w[t / KUSED][t % KUSED] = 0.0f; }
    __syncthreads();
    for (int l = 0; l < nl; l++) {
        const float wp = router_lg[l * NEXP + t] * 1.0f;
        const float mx = block_max_f<256>(wp, rs.mx);
        const float e = v_expf(wp - mx);
        float g = e + shfl_xor_f(e, 1);
        g = g + shfl_xor_f(g, 2);
        if ((t & 3) == 0) rs.gs[t >> 2] = g;
        const double P = block_sum_d<256>((t & 3) == 0 ? (double)g : 0.0, rs.red);
        float f;
        if (!bracket_ok_recip(P, P, NEXP / 4, &f)) {
            if (t == 0) {
                double s = 0.0;
                for (int i = 0; i < NEXP / 4; i++) s += (double)rs.gs[i];
                rs.red[0] = s;
            }
            __syncthreads();
            f = (float)(1.0 / rs.red[0]);
            __syncthreads();
        }
        const float pt = e * f;
        rs.p[t] = pt;
        __syncthreads();
        int rank = 0;
        bool eq = false;
        for (int u = 0; u < NEXP; u++) {
            const float pu = rs.p[u];
            rank += (pu > pt) || (pu == pt && u < t);
            eq |= (pu == pt) && (u != t);
        }
        if (rank <= KUSED && (eq || pt != pt)) rs.tie = 1;
        if (rank < KUSED) { rs.ids[l][rank] = t; rs.w[l][rank] = pt; }
        __syncthreads();
        if (t == 0) {
            double s = 0.0;
            for (int j = 0; j < KUSED; j++) s += (double)rs.w[l][j];
            float sf = (float)s;
            sf = sf < __builtin_inff() ? sf : __builtin_inff();
            sf = sf > 6.103515625e-5f ? sf : 6.103515625e-5f;
            for (int j = 0; j < KUSED; j++) rs.w[l][j] = rs.w[l][j] / sf;
        }
        __syncthreads();
    }
    if (t == 0) {
        // union of the lanes' experts in first-use order, lane-major (engine.rs:3458-3475)
        int n = 0;
        for (int l = 0; l < nl; l++)
            for (int j = 0; j < KUSED; j++) {
                const int e = rs.ids[l][j];
                bool seen = false;
                for (int u = 0; u < n; u++) seen |= rs.uni[u] == e;
                if (!seen) rs.uni[n++] = e;
            }
        rs.n_uni = n;
        if (count_ties && rs.tie) atomicAdd(tie_cnt, 1u);
    }
    __syncthreads();
}

OXE_DEV int slot_of(const RouteSmem &rs, int l, int e) {
    for (int j = 0; j < KUSED; j++)
        if (rs.ids[l][j] == e) return j;
    return -1;
}

struct ExpertArgs {
    const float *router_lg;
    const int8_t *xq;         // [NL][2E]
    const uint16_t *xd;       // [NL][2E/32]
    Q8W exp_gu;               // [NEXP][2FF][E]
    float *hexp;              // [NL][KUSED][FF]
    int32_t *route_ids;
    float *route_w;
    int32_t *uni;
    uint32_t *tie_cnt;
};

constexpr int EX_TILES = 2 * FF / 16;  // 64 tiles of 16 rows (8 gate + 8 up) per expert

template <int NL>
__global__ __launch_bounds__(256) void experts_kernel(const RunCtl *__restrict__ ctl, ExpertArgs a) {
    constexpr int R = GemvR<E>::R;
    __shared__ RouteSmem rs;
    __shared__ GemvSmem<E, R, NL> sm;
    if (!ctl->active) return;
    route_all<NL>(ctl, a.router_lg, rs, a.tie_cnt, blockIdx.x == 0);
    const int nl = ctl->nl, t = threadIdx.x;
    if (blockIdx.x == 0) {
        if (t < NL * KUSED) {
            const int l = t / KUSED, j = t % KUSED;
            if (l < nl) { a.route_ids[t] = rs.ids[l][j]; a.route_w[t] = rs.w[l][j]; }
        }
        if (t < OXE_MAX_UNION) a.uni[1 + t] = t < rs.n_uni ? rs.uni[t] : -1;
        if (t == 0) a.uni[0] = rs.n_uni;
    }
    const int u = blockIdx.x / EX_TILES, tile = blockIdx.x % EX_TILES;
    if (u >= rs.n_uni) return;
    const int e = rs.uni[u];
    const int8_t *xq[NL];
    const uint16_t *xd[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) { xq[l] = a.xq + (int64_t)l * 2 * E; xd[l] = a.xd + (int64_t)l * (2 * E / 32); }
    const int64_t rows = 2 * FF;
    gemv_tile<E, R, NL>(a.exp_gu.q + (int64_t)e * rows * E, a.exp_gu.d + (int64_t)e * rows * (E / 32), (int64_t)tile * R,
                        rows, xq, xd, sm);
    if (t < NL * 8) {
        const int l = t / 8, r = t % 8;
        if (l < nl) {
            const int j = slot_of(rs, l, e);
            if (j >= 0) a.hexp[((int64_t)l * KUSED + j) * FF + tile * 8 + r] = v_silu(sm.out[l][r]) * sm.out[l][8 + r];
        }
    }
}

void launch_experts(const RunCtl *ctl, const LayerW &w, const ActBufs &b, hipStream_t st) {
    ExpertArgs a{};
    a.router_lg = b.router_lg;
    a.xq = b.xq;
    a.xd = b.xd;
    a.exp_gu = w.exp_gu;
    a.hexp = b.hexp;
    a.route_ids = b.route_ids;
    a.route_w = b.route_w;
    a.uni = b.uni;
    a.tie_cnt = b.counters + CNT_ERR_TIE;
    hipLaunchKernelGGL(experts_kernel<OXE_NL>, dim3(OXE_MAX_UNION * EX_TILES), dim3(256), 0, st, ctl, a);
}

// ------------------------------------------------------------------------------------------------
// down + combine: workgroup = 8 output rows. Units u = 0..15 are the union experts, u = 16 the
// shared expert. K = 512: one 16-byte code chunk per thread per unit (32 chunks x 8 rows).
constexpr int DW_R = 8;
constexpr int DW_U = OXE_MAX_UNION + 1;
constexpr int DW_NB = FF / 32;        // 16 blocks per row
constexpr int DW_WDS = DW_NB / 2 + 1; // padded scale row (words)

struct DownArgs {
    const int32_t *uni;
    const int32_t *route_ids;
    const float *route_w;
    const float *sh_gate;
    const float *hexp;        // [NL][KUSED][FF]
    const float *hsh;         // [NL][FFSH]
    Q8W exp_down;             // [NEXP][E][FF]
    Q8W shexp_down;           // [E][FFSH]
    const float *x1;
    float *x2;
    unsigned long long *amax_key;
};

template <int NL>
__global__ __launch_bounds__(256) void down_kernel(const RunCtl *__restrict__ ctl, DownArgs a) {
    __shared__ int8_t s_hq[NL][KUSED + 1][FF];
    __shared__ uint16_t s_hd[NL][KUSED + 1][DW_NB];
    __shared__ uint32_t s_wd[DW_U][DW_R * DW_WDS];
    __shared__ int32_t s_isum[DW_U][NL][DW_R][DW_NB + 1];
    __shared__ float s_dn[NL][KUSED + 1][DW_R];
    __shared__ int32_t s_e[DW_U], s_slot[DW_U][NL];
    __shared__ float s_w[NL][KUSED], s_sg[NL];
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * DW_R;
    if (blockIdx.x == 0 && t < NL) a.amax_key[t] = 0ull;  // the LM head that follows starts clean
    int nu = a.uni[0];
    nu = nu < 0 ? 0 : (nu > OXE_MAX_UNION ? OXE_MAX_UNION : nu);
    // phase 1: every weight load of the workgroup first (the dominant HBM traffic)
    const int c = t & 31, r = t >> 5;
    uint4 wv[DW_U];
#pragma unroll
    for (int u = 0; u < DW_U; u++) {
        const int e = u < OXE_MAX_UNION ? (u < nu ? a.uni[1 + u] : -1) : 0;
        if (u == OXE_MAX_UNION || e >= 0) {
            const int8_t *base = u < OXE_MAX_UNION ? a.exp_down.q + (int64_t)e * E * FF : a.shexp_down.q;
            wv[u] = *(const uint4 *)(base + (row0 + r) * FF + 16 * c);
        } else {
            wv[u] = make_uint4(0, 0, 0, 0);
        }
    }
    for (int i = t; i < DW_U * DW_R * (DW_NB / 2); i += 256) {
        const int u = i / (DW_R * (DW_NB / 2)), k = i % (DW_R * (DW_NB / 2)), rr = k / (DW_NB / 2), b2 = k % (DW_NB / 2);
        const int e = u < OXE_MAX_UNION ? (u < nu ? a.uni[1 + u] : -1) : 0;
        uint32_t v = 0;
        if (u == OXE_MAX_UNION || e >= 0) {
            const uint16_t *sb = u < OXE_MAX_UNION ? a.exp_down.d + (int64_t)e * E * DW_NB : a.shexp_down.d;
            v = *(const uint32_t *)(sb + (row0 + rr) * DW_NB + 2 * b2);
        }
        s_wd[u][rr * DW_WDS + b2] = v;
    }
    // routing results of the experts kernel, and the lanes' activations quantised into LDS
    if (t < DW_U) {
        const int e = t < OXE_MAX_UNION ? (t < nu ? a.uni[1 + t] : -1) : 0;
        s_e[t] = e;
        for (int l = 0; l < NL; l++) {
            int j = -1;
            if (l < nl) {
                if (t == OXE_MAX_UNION) j = KUSED;
                else if (e >= 0)
                    for (int jj = 0; jj < KUSED; jj++)
                        if (a.route_ids[l * KUSED + jj] == e) j = jj;
            }
            s_slot[t][l] = j;
        }
    }
    if (t < NL * KUSED) s_w[t / KUSED][t % KUSED] = t / KUSED < nl ? a.route_w[t] : 0.0f;
    if (t < NL) s_sg[t] = t < nl ? a.sh_gate[t] : 0.0f;
    for (int i = t; i < NL * (KUSED + 1) * DW_NB; i += 256) {
        const int l = i / ((KUSED + 1) * DW_NB), j = (i / DW_NB) % (KUSED + 1), b = i % DW_NB;
        if (l < nl) {
            const float *src = j < KUSED ? a.hexp + ((int64_t)l * KUSED + j) * FF + 32 * b : a.hsh + (int64_t)l * FFSH + 32 * b;
            quant_block_q8_0(src, &s_hq[l][j][32 * b], &s_hd[l][j][b]);
        } else {
            for (int k = 0; k < 32; k++) s_hq[l][j][32 * b + k] = 0;
            s_hd[l][j][b] = 0;
        }
    }
    __syncthreads();
    // phase 2: block dots (exact int32), halves of a block meet by a lane shuffle
#pragma unroll
    for (int u = 0; u < DW_U; u++) {
        if (u < OXE_MAX_UNION && u >= nu) continue;  // uniform across the workgroup
#pragma unroll
        for (int l = 0; l < NL; l++) {
            const int j = s_slot[u][l] < 0 ? 0 : s_slot[u][l];
            const uint4 xa = *(const uint4 *)&s_hq[l][j][16 * c];
            int32_t s = dot16(wv[u], xa, 0);
            s += shfl_xor_i(s, 1);
            if ((c & 1) == 0) s_isum[u][l][r][c >> 1] = s;
        }
    }
    __syncthreads();
    // phase 3: serial fp32 chains per (unit, lane, row)
    for (int i = t; i < DW_U * NL * DW_R; i += 256) {
        const int u = i / (NL * DW_R), l = (i / DW_R) % NL, rr = i % DW_R;
        if (u < OXE_MAX_UNION && u >= nu) continue;
        const int j = s_slot[u][l];
        if (j < 0) continue;
        const uint16_t *sw = (const uint16_t *)&s_wd[u][rr * DW_WDS];
        float acc = 0.0f;
#pragma unroll
        for (int b = 0; b < DW_NB; b++)
            acc = __builtin_fmaf((float)s_isum[u][l][rr][b], h2f(s_hd[l][j][b]) * h2f(sw[b]), acc);
        s_dn[l][j][rr] = acc;
    }
    __syncthreads();
    // phase 4: combine in slot order (engine.rs:3591-3601)
    if (t < NL * DW_R) {
        const int l = t / DW_R, rr = t % DW_R;
        if (l < nl) {
            float m = s_dn[l][0][rr] * s_w[l][0];
            for (int j = 1; j < KUSED; j++) {
                const float p = s_dn[l][j][rr] * s_w[l][j];
                m = m + p;
            }
            const float s = s_dn[l][KUSED][rr] * s_sg[l];
            const float f = m + s;
            a.x2[(int64_t)l * E + row0 + rr] = f + a.x1[(int64_t)l * E + row0 + rr];
        }
    }
}

void launch_down(const RunCtl *ctl, const LayerW &w, const ActBufs &b, hipStream_t st) {
    DownArgs a{};
    a.uni = b.uni;
    a.route_ids = b.route_ids;
    a.route_w = b.route_w;
    a.sh_gate = b.sh_gate;
    a.hexp = b.hexp;
    a.hsh = b.hsh;
    a.exp_down = w.exp_down;
    a.shexp_down = w.shexp_down;
    a.x1 = b.x1;
    a.x2 = b.x2;
    a.amax_key = b.amax_key;
    hipLaunchKernelGGL(down_kernel<OXE_NL>, dim3(E / DW_R), dim3(256), 0, st, ctl, a);
}

}  // namespace oxe
