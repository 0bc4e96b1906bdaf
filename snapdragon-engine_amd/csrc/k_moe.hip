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
#include "oxe_route.h"

namespace oxe {

using namespace shp;

// ------------------------------------------------------------------------------------------------
constexpr int RT_ROWS = 8;                  // router rows per workgroup (staged in LDS)
constexpr int RT_ROW_WG = NEXP / RT_ROWS;   // 32 router workgroups
constexpr int RT_SH_WG = 1;                 // shared-gate dot
constexpr int RT_GU_TILES = 2 * FFSH / 16;  // 64 shared gate/up tiles
constexpr int RT_LDW = E + 16;              // padded LDS row of a staged router row

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
    extern __shared__ float s_w[];  // [RT_ROWS][RT_LDW] staged f32 rows (router / shared-gate workgroups)
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x, b = blockIdx.x;
    const bool dot_wg = b < RT_ROW_WG + RT_SH_WG;
    const bool sh = b == RT_ROW_WG;
    // f32 rows first: their loads are in flight during the norm prologue
    float4 wv[RT_ROWS * E / 4 / 256];
    if (dot_wg) {
#pragma unroll
        for (int i = 0; i < RT_ROWS * E / 4 / 256; i++) {
            const int idx = t + 256 * i, rr = idx / (E / 4);
            if (sh && rr > 0) { wv[i] = make_float4(0, 0, 0, 0); continue; }
            const float *row = sh ? a.shexp_gate : a.router + (int64_t)(b * RT_ROWS + rr) * E;
            wv[i] = *(const float4 *)(row + 4 * (idx % (E / 4)));
        }
    }
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
        if (b == 0) {
            store8(a.xn + (int64_t)l * E, v);
            *(uint2 *)(a.xq + (int64_t)l * 2 * E + EPT * t) = *(const uint2 *)&s_xq[l][EPT * t];
        }
    }
    if (dot_wg) {
#pragma unroll
        for (int i = 0; i < RT_ROWS * E / 4 / 256; i++) {
            const int idx = t + 256 * i, rr = idx / (E / 4);
            *(float4 *)&s_w[rr * RT_LDW + 4 * (idx % (E / 4))] = wv[i];
        }
    }
    __syncthreads();
    if (b == 0 && t < NL * (E / 32)) a.xd[(t / (E / 32)) * (2 * E / 32) + t % (E / 32)] = s_xd[t / (E / 32)][t % (E / 32)];
    if (dot_wg) {
        // f32 dots in ggml_vec_dot_f32 order (vec.cpp:104-125): lane c of a 16-lane group runs chain
        // c (elements c + 16 s); xor 8, 4, 1, 2 is the NEON reduction tree
        const int c = t & 15, rr = t >> 4;
        if (rr >= RT_ROWS || (sh && rr > 0)) return;
        const float *w = &s_w[rr * RT_LDW];
        float acc[NL];
#pragma unroll
        for (int l = 0; l < NL; l++) acc[l] = 0.0f;
#pragma unroll 8
        for (int s = 0; s < E / 16; s++) {
            const float x = w[c + 16 * s];
#pragma unroll
            for (int l = 0; l < NL; l++) acc[l] = __builtin_fmaf(x, s_xn[l][c + 16 * s], acc[l]);
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
                else a.router_lg[l * NEXP + b * RT_ROWS + rr] = v;
            }
        }
        return;
    }
    // shared expert gate/up tile: rows 16*tile .. (8 gate rows then 8 up rows) -> 8 h values
    __shared__ GemvSmem<E, R, NL> sm;
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
    const size_t lds = (size_t)RT_ROWS * RT_LDW * 4;
    static bool configured = false;
    if (!configured) {
        (void)hipFuncSetAttribute((const void *)router_kernel<OXE_NL>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
        configured = true;
    }
    // a K-quant shared gate / up runs in the MoE's K-quant kernels instead of these tiles
    const int tiles = w.sh_gate_r.type == 8 ? RT_GU_TILES : 0;
    hipLaunchKernelGGL(router_kernel<OXE_NL>, dim3(RT_ROW_WG + RT_SH_WG + tiles), dim3(256), lds, st, ctl, a);
}

// routing of every lane (one wave each) and the union of the lanes' experts in first-use order,
// lane-major (engine.rs:3414-3475)
struct RouteArgs {
    const float *router_lg;
    int32_t *route_ids;       // [NL][KUSED]
    float *route_w;           // [NL][KUSED]
    int32_t *uni;             // [1 + OXE_MAX_UNION]
    uint32_t *tie_cnt;
};

template <int NL>
__global__ __launch_bounds__(64 * NL) void route_kernel(const RunCtl *__restrict__ ctl, RouteArgs a) {
    __shared__ RouteOut ro;
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x, w = t >> 6;
    if (t == 0) ro.tie = 0;
    __syncthreads();
    if (w < nl) route_wave(a.router_lg + w * NEXP, w, ro);
    __syncthreads();
    if (t < 64) {
        // union in first-use order, lane-major: entry t = (lane t/8, rank t%8) is new when no earlier
        // entry holds the same expert; its slot is the number of new entries before it
        const int e = t < nl * KUSED ? ro.ids[t / KUSED][t % KUSED] : -1;
        bool isnew = e >= 0;
#pragma unroll
        for (int u = 0; u < NL * KUSED; u++) {
            const int o = __shfl(e, u);
            isnew &= !(u < t && o == e);
        }
        const unsigned long long mask = __ballot(isnew);
        const int n = __popcll(mask);
        if (isnew) a.uni[1 + __popcll(mask & ((1ull << t) - 1))] = e;
        if (t >= n && t < OXE_MAX_UNION) a.uni[1 + t] = -1;
        if (t == 0) {
            a.uni[0] = n;
            if (ro.tie) atomicAdd(a.tie_cnt, 1u);
        }
    }
    if (t < NL * KUSED && t / KUSED < nl) {
        a.route_ids[t] = ro.ids[t / KUSED][t % KUSED];
        a.route_w[t] = ro.w[t / KUSED][t % KUSED];
    }
}

void launch_route(const RunCtl *ctl, const ActBufs &b, hipStream_t st) {
    RouteArgs a{b.router_lg, b.route_ids, b.route_w, b.uni, b.counters + CNT_ERR_TIE};
    hipLaunchKernelGGL(route_kernel<OXE_NL>, dim3(1), dim3(64 * OXE_NL), 0, st, ctl, a);
}

struct ExpertArgs {
    const int8_t *xq;         // [NL][2E]
    const uint16_t *xd;       // [NL][2E/32]
    Q8W exp_gu;               // [NEXP][2FF][E]
    float *hexp;              // [NL][KUSED][FF]
    const int32_t *route_ids;
    const int32_t *uni;
    uint32_t *stats;          // [0] sum of union sizes, [1] launches
};

constexpr int EX_TILES = 2 * FF / 16;  // 64 tiles of 16 rows (8 gate + 8 up) per expert

template <int NL>
__global__ __launch_bounds__(256) void experts_kernel(const RunCtl *__restrict__ ctl, ExpertArgs a) {
    constexpr int R = GemvR<E>::R;
    __shared__ GemvSmem<E, R, NL> sm;
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
    const int u = blockIdx.x / EX_TILES, tile = blockIdx.x % EX_TILES;
    const int nu = a.uni[0];
    if (blockIdx.x == 0 && t == 0) {
        atomicAdd(a.stats, (uint32_t)nu);   // expert units streamed (algorithmic bytes)
        atomicAdd(a.stats + 1, 1u);
    }
    if (u >= nu) return;
    int e = a.uni[1 + u];
    e = e < 0 ? 0 : (e >= NEXP ? NEXP - 1 : e);
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
            int j = -1;
            for (int jj = 0; jj < KUSED; jj++)
                if (a.route_ids[l * KUSED + jj] == e) j = jj;
            if (j >= 0) a.hexp[((int64_t)l * KUSED + j) * FF + tile * 8 + r] = v_silu(sm.out[l][r]) * sm.out[l][8 + r];
        }
    }
}

void launch_experts(const RunCtl *ctl, const LayerW &w, const ActBufs &b, hipStream_t st) {
    ExpertArgs a{};
    a.xq = b.xq;
    a.xd = b.xd;
    a.exp_gu = w.exp_gu;
    a.hexp = b.hexp;
    a.route_ids = b.route_ids;
    a.uni = b.uni;
    a.stats = b.counters + CNT_UNI_SUM;
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
