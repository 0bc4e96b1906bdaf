// Routing of the MoE router's logits (crates/model/src/engine.rs:3414-3429), one wave per lane;
// shared by the per-phase kernels and the fused run kernel.
#pragma once
#include "oxe_common.h"
#include "oxe_engine.h"
#include "oxe_shape.h"
#include "oxe_stdsort.h"

namespace oxe {

using namespace shp;

// Routing of one lane by one wave (engine.rs:3414-3429), lane tl holding experts 4tl..4tl+3:
//   probs = oxe_soft_max_f32(logits, scale 1, no mask)   (oxe_ops.cpp:101-115): x*1, max, v_expf in
//           groups of 4 with the group sum (v0+v1)+(v2+v3) added in double, scale by f32(1/sum)
//   ids   = oxe_argsort_top_k_f32(probs, 8)              (oxe_ops.cpp:121-165)
//   w_j   = probs[ids_j] / clamp(ggml_vec_sum_f32(w), 6.103515625e-5, inf)
// Fast path: a radix select of the top 9, ranked directly when they are pairwise distinct. When
// the 9 largest are not strictly distinct, the 9th repeats, or a value is NaN (where the reference
// runs std::sort over all 256 indices with x[a] > x[b]), one thread of the wave runs libstdc++'s
// std::sort algorithm (oxe_stdsort.h) over the 256 probabilities in LDS, so tied experts come out in
// the reference's order; the lane's tie flag counts these runs.
struct RouteOut {
    int32_t ids[OXE_NL][KUSED];
    float w[OXE_NL][KUSED];
    float gs[OXE_NL][NEXP / 4];
    float sv[OXE_NL][KUSED + 1];     // the selected top 9 (value, expert) of the fast path
    int32_t si[OXE_NL][KUSED + 1];
    float vs[OXE_NL][KUSED + 1];     // values in rank order
    float pv[OXE_NL][NEXP];          // the tie path: probabilities, sorted expert indices, sort stack
    uint8_t sx[OXE_NL][NEXP];
    oxe_sort::Range stk[OXE_NL][OXE_SORT_STACK];
    int32_t tie;
};

OXE_DEV void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

OXE_DEV void route_wave(const float *lg, int l, RouteOut &ro) {
    const int tl = threadIdx.x & 63;
    float p[4];
#pragma unroll
    for (int k = 0; k < 4; k++) p[k] = lg[4 * tl + k] * 1.0f;
    float mx = p[0];
#pragma unroll
    for (int k = 1; k < 4; k++) mx = (mx > p[k]) ? mx : p[k];
    mx = wave_max_any(mx);
#pragma unroll
    for (int k = 0; k < 4; k++) p[k] = v_expf(p[k] - mx);
    const float g = (p[0] + p[1]) + (p[2] + p[3]);
    ro.gs[l][tl] = g;
    const double P = wave_sum_d_any((double)g);
    float f;
    if (!bracket_ok_recip(P, P, NEXP / 4, &f)) {
        wave_lds_sync();
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
    // Fast path: the probabilities are >= 0, so their bits order like their values. Radix-select
    // a bit pattern T with exactly 9 values >= T, from the high bits down (T keeps at least 9
    // values >= T at every step; the walk stops once exactly 9 are left). The probabilities are
    // <= 1, so bits 31 and 30 are clear and the walk starts at bit 29 (were one not, T would still
    // keep its invariant and the count test below decides). When exactly 9 values are >= T and
    // they are pairwise distinct, their order by value is the reference's (no ties), found by
    // ranking the 9 directly.
    bool fast = !__ballot(nan);
    if (fast) {
        uint32_t b[4];
#pragma unroll
        for (int k = 0; k < 4; k++) b[k] = __builtin_bit_cast(uint32_t, p[k]);
        uint32_t T = 0;
        int cntT = NEXP;
        for (int bit = 29; bit >= 0 && cntT != KUSED + 1; bit--) {
            const uint32_t cand = T | (1u << bit);
            int cnt = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) cnt += __popcll(__ballot(b[k] >= cand));
            if (cnt >= KUSED + 1) { T = cand; cntT = cnt; }
        }
        unsigned long long m[4];
        int nsel = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            m[k] = __ballot(b[k] >= T);
            nsel += __popcll(m[k]);
        }
        fast = nsel == KUSED + 1;
        if (fast) {
            const unsigned long long below = (1ull << tl) - 1;
            int base = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                if (b[k] >= T) {
                    const int slot = base + __popcll(m[k] & below);
                    ro.sv[l][slot] = p[k];
                    ro.si[l][slot] = 4 * tl + k;
                }
                base += __popcll(m[k]);
            }
            wave_lds_sync();
            int dup = 0;
            if (tl < KUSED + 1) {
                const float v = ro.sv[l][tl];
                const int id = ro.si[l][tl];
                int rank = 0;
#pragma unroll
                for (int j = 0; j < KUSED + 1; j++) {
                    const float o = ro.sv[l][j];
                    rank += (o > v) ? 1 : 0;
                    dup |= (j != tl && o == v) ? 1 : 0;
                }
                if (rank < KUSED) ro.ids[l][rank] = id;
                ro.vs[l][rank] = v;
                (void)id;
            }
            fast = !__ballot(dup != 0);
            wave_lds_sync();
        }
    }
    if (!fast) {
        // ties, NaN, or a repeated 9th value: std::sort of all 256 indices (oxe_ops.cpp:157-164)
        static_assert(NEXP == 256, "8-bit expert indices");
#pragma unroll
        for (int k = 0; k < 4; k++) {
            ro.pv[l][4 * tl + k] = p[k];
            ro.sx[l][4 * tl + k] = (uint8_t)(4 * tl + k);
        }
        wave_lds_sync();
        if (tl == 0) {
            oxe_sort::sort_desc(ro.sx[l], ro.pv[l], NEXP, ro.stk[l]);
            ro.tie = 1;
        }
        wave_lds_sync();
        if (tl <= KUSED) {
            const int e = ro.sx[l][tl];
            if (tl < KUSED) ro.ids[l][tl] = e;
            ro.vs[l][tl] = ro.pv[l][e];
        }
        wave_lds_sync();
    }
    // sum in rank order (every lane forms it), then lane j < 8 divides weight j
    double s = 0.0;
#pragma unroll
    for (int j = 0; j < KUSED; j++) s += (double)ro.vs[l][j];
    float sf = (float)s;
    sf = sf < __builtin_inff() ? sf : __builtin_inff();
    sf = sf > 6.103515625e-5f ? sf : 6.103515625e-5f;
    if (tl < KUSED) ro.w[l][tl] = ro.vs[l][tl] / sf;
}

}  // namespace oxe
