// Routing of the MoE router's logits (crates/model/src/engine.rs:3414-3429), one wave per lane;
// shared by the per-phase kernels and the fused run kernel.
#pragma once
#include "oxe_common.h"
#include "oxe_engine.h"
#include "oxe_shape.h"

namespace oxe {

using namespace shp;

// Routing of one lane by one wave (engine.rs:3414-3429), lane tl holding experts 4tl..4tl+3:
//   probs = oxe_soft_max_f32(logits, scale 1, no mask)   (oxe_ops.cpp:101-115): x*1, max, v_expf in
//           groups of 4 with the group sum (v0+v1)+(v2+v3) added in double, scale by f32(1/sum)
//   ids   = oxe_argsort_top_k_f32(probs, 8)              (oxe_ops.cpp:121-165)
//   w_j   = probs[ids_j] / clamp(ggml_vec_sum_f32(w), 6.103515625e-5, inf)
// The top 9 are taken by 9 wave arg-max rounds (largest value, then lowest index). When the 9 are
// not strictly decreasing or the 9th value repeats (where the reference runs std::sort), the
// lane's tie flag is set; the order used is then descending value, ascending index.
OXE_DEV float wave_max_f(float v) {
    for (int m = 32; m >= 1; m >>= 1) {
        const float o = shfl_xor_f(v, m);
        v = (v > o) ? v : o;
    }
    return v;
}
OXE_DEV int wave_min_i(int v) {
    for (int m = 32; m >= 1; m >>= 1) {
        const int o = shfl_xor_i(v, m);
        v = v < o ? v : o;
    }
    return v;
}
OXE_DEV int wave_sum_i(int v) {
    for (int m = 32; m >= 1; m >>= 1) v += shfl_xor_i(v, m);
    return v;
}

struct RouteOut {
    int32_t ids[OXE_NL][KUSED];
    float w[OXE_NL][KUSED];
    float gs[OXE_NL][NEXP / 4];
    int32_t tie;
};

OXE_DEV void route_wave(const float *lg, int l, RouteOut &ro) {
    const int tl = threadIdx.x & 63;
    float p[4];
#pragma unroll
    for (int k = 0; k < 4; k++) p[k] = lg[4 * tl + k] * 1.0f;
    float mx = p[0];
#pragma unroll
    for (int k = 1; k < 4; k++) mx = (mx > p[k]) ? mx : p[k];
    mx = wave_max_f(mx);
#pragma unroll
    for (int k = 0; k < 4; k++) p[k] = v_expf(p[k] - mx);
    const float g = (p[0] + p[1]) + (p[2] + p[3]);
    ro.gs[l][tl] = g;
    double P = (double)g;
    for (int m = 32; m >= 1; m >>= 1) P += shfl_xor_d(P, m);
    float f;
    if (!bracket_ok_recip(P, P, NEXP / 4, &f)) {
        double s = 0.0;
        for (int i = 0; i < NEXP / 4; i++) s += (double)ro.gs[l][i];
        f = (float)(1.0 / s);
    }
    bool nan = false;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        p[k] = p[k] * f;
        nan |= p[k] != p[k];
    }
    // top 9 by wave arg-max rounds
    unsigned taken = 0;  // bit k: expert 4tl+k already picked
    float vals[KUSED + 1];
    int ids[KUSED + 1];
#pragma unroll
    for (int r = 0; r <= KUSED; r++) {
        float bv = -__builtin_inff();
        int bi = 0x7fffffff;
#pragma unroll
        for (int k = 0; k < 4; k++)
            if (!((taken >> k) & 1) && (p[k] > bv || bi == 0x7fffffff)) { bv = p[k]; bi = 4 * tl + k; }
        const float m = wave_max_f(bv);
        const int i = wave_min_i(bv == m ? bi : 0x7fffffff);
        if ((i >> 2) == tl) taken |= 1u << (i & 3);
        vals[r] = m;
        ids[r] = i;
    }
    bool tie = false;
#pragma unroll
    for (int r = 1; r <= KUSED; r++) tie |= !(vals[r - 1] > vals[r]);
    int eq = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) eq += p[k] == vals[KUSED];
    eq = wave_sum_i(eq);
    tie |= eq != 1;
    tie |= wave_sum_i(nan ? 1 : 0) != 0;
    if (tl == 0) {
        double s = 0.0;
#pragma unroll
        for (int j = 0; j < KUSED; j++) s += (double)vals[j];
        float sf = (float)s;
        sf = sf < __builtin_inff() ? sf : __builtin_inff();
        sf = sf > 6.103515625e-5f ? sf : 6.103515625e-5f;
#pragma unroll
        for (int j = 0; j < KUSED; j++) {
            ro.ids[l][j] = ids[j];
            ro.w[l][j] = vals[j] / sf;
        }
        if (tie) ro.tie = 1;
    }
}

}  // namespace oxe
