// K-quant kernels: the q8_K activation quantizer (quantize_row_q8_K) and the lane GEMVs over
// Q3_K / Q4_K / Q5_K / Q6_K weights (the reference's oxe_vl_gemv, crates/kernels-sys/csrc/
// oxe_vl.inc:78-107, types 3..6), bit for bit per (lane, row).
//
// Weights are the GGUF file's ggml blocks (no repack: the reference's 8-row interleave only serves
// its NEON SMMLA tiles). Integer parts are exact (codes repacked 4 per dword into v_dot4_i32_i8),
// so only the float chain per (lane, row), in the order and fusion the reference documents per
// type, fixes the bits; the kernel layout is free otherwise (see vl_gemv_kernel).
#include <algorithm>

#include "oxe_common.h"
#include "oxe_model_kernels.h"
#include "oxe_prologue.h"

#include <mutex>

namespace oxe {
namespace kq {

constexpr int QK = 256;
constexpr int Q8K_BYTES = 292;   // block_q8_K: float d, int8 qs[256], int16 bsums[16]
constexpr int Q8K_QS = 4, Q8K_BS = 260;
constexpr int MAX_LANES = 4;

// B: block bytes; R: integers per (unit, lane) that the chain reads (kept in LDS between the units
// and the chains, so a smaller R leaves room for more waves per CU)
template <int TY> struct BT;
template <> struct BT<3> { static constexpr int B = 110, R = 1; };
template <> struct BT<4> { static constexpr int B = 144, R = 5; };
template <> struct BT<5> { static constexpr int B = 176, R = 6; };
template <> struct BT<6> { static constexpr int B = 210, R = 1; };

OXE_DEV uint32_t ld32(const uint8_t *p) { return *(const uint32_t *)p; }
OXE_DEV uint16_t ld16(const uint8_t *p) { return *(const uint16_t *)p; }
// N dwords from a 2-byte aligned LDS address (Q3_K / Q6_K blocks are 110 / 210 bytes, so every other
// block of a row starts 2 bytes off a dword boundary): N + 1 aligned dword reads, then each dword
// cut out of a neighbouring pair (v_alignbyte_b32)
template <int N>
OXE_DEV void ld_run(const uint8_t *p, uint32_t (&out)[N]) {
    const uint32_t sh = (uint32_t)(uintptr_t)p & 3u;
    const uint32_t *a = (const uint32_t *)(p - sh);
    uint32_t w[N + 1];
#pragma unroll
    for (int i = 0; i <= N; i++) w[i] = a[i];
#pragma unroll
    for (int i = 0; i < N; i++) out[i] = __builtin_amdgcn_alignbyte(w[i + 1], w[i], sh);
}
// Activations in LDS: each q8_K block repacked as two halves (codes 128 h .. 128 h + 127 and their 8
// sums of 16), YH = 37 dwords apart (odd: the 16 threads of a row read one half each, at the same
// offset, on distinct banks), lanes YL(nb) dwords apart; the block scales in a separate array.
constexpr int YH = 37;
__host__ __device__ inline int y_lane_words(int nb) { return nb * 2 * YH; }
struct YView {
    const uint32_t *h;   // half (b, h) of lane 0
    int ls;              // lane stride in dwords
    OXE_DEV uint32_t q(int l, int j) const { return h[l * ls + j]; }   // code dword j (0..31)
    OXE_DEV int bsum(int l, int i) const { return (int)((const int16_t *)(h + l * ls + 32))[i]; }   // sum i (0..7)
};

// ---- quantize_row_q8_K_ref (vendor/ggml-subset/generated/quants_base.c:14-48) --------------------
// One wave per 256-value block; thread t holds values 4 t .. 4 t + 3. The block maximum is the
// first value of largest magnitude (the reference's strict > scan); iscale = -127 / max (f32
// division), codes = nearest_int(iscale * x) (the float add of 1.5 * 2^23: round half to even),
// clamped above at 127; bsums = sums of 16 codes; d = 1 / iscale. An all-zero block gets d = 0 and
// zero codes and sums.
// (xb: the block's 256 values; every lane of one wave)
OXE_DEV void q8K_block(const float *xb, int lane, uint8_t *__restrict__ yb) {
    const float4 v4 = *(const float4 *)(xb + 4 * lane);
    const float v[4] = {v4.x, v4.y, v4.z, v4.w};
    float am = 0.0f, mx = 0.0f;
    int idx = QK;
    for (int e = 0; e < 4; e++) {
        const float ax = fabsf(v[e]);
        if (ax > am) {
            am = ax;
            mx = v[e];
            idx = 4 * lane + e;
        }
    }
    for (int m = 32; m >= 1; m >>= 1) {
        const float oa = shfl_xor_f(am, m), om = shfl_xor_f(mx, m);
        const int oi = shfl_xor_i(idx, m);
        if (oa > am || (oa == am && oi < idx)) {
            am = oa;
            mx = om;
            idx = oi;
        }
    }
    int q[4] = {0, 0, 0, 0};
    float iscale = 0.0f;
    if (am != 0.0f) {
        iscale = -127.f / mx;
        for (int e = 0; e < 4; e++) {
            const float p = iscale * v[e];
            const float t = p + 12582912.f;
            const int r = (int)(__builtin_bit_cast(uint32_t, t) & 0x007fffffu) - 0x00400000;
            q[e] = r < 127 ? r : 127;
        }
    }
    *(uint32_t *)(yb + Q8K_QS + 4 * lane) =
        (uint32_t)(q[0] & 255) | (uint32_t)(q[1] & 255) << 8 | (uint32_t)(q[2] & 255) << 16 | (uint32_t)(q[3] & 255) << 24;
    int s = q[0] + q[1] + q[2] + q[3];
    s += shfl_xor_i(s, 1);
    s += shfl_xor_i(s, 2);
    if ((lane & 3) == 0) *(int16_t *)(yb + Q8K_BS + 2 * (lane >> 2)) = (int16_t)s;
    if (lane == 0) *(float *)yb = am != 0.0f ? 1 / iscale : 0.0f;
}

__global__ __launch_bounds__(256) void quant_q8_K_kernel(const float *__restrict__ x, int64_t nblk,
                                                         uint8_t *__restrict__ y) {
    const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblk) return;
    q8K_block(x + b * QK, threadIdx.x & 63, y + b * Q8K_BYTES);
}

// two buffers' blocks in one launch: blocks b < n0 of x0 into y0, then n1 of x1 into y1
__global__ __launch_bounds__(256) void quant_q8_K_two_kernel(const float *__restrict__ x0, int64_t n0,
                                                             uint8_t *__restrict__ y0, const float *__restrict__ x1,
                                                             int64_t n1, uint8_t *__restrict__ y1) {
    int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= n0 + n1) return;
    if (b < n0) {
        q8K_block(x0 + b * QK, threadIdx.x & 63, y0 + b * Q8K_BYTES);
    } else {
        b -= n0;
        q8K_block(x1 + b * QK, threadIdx.x & 63, y1 + b * Q8K_BYTES);
    }
}

// the q8_K blocks of a workgroup's [NL][E] rows held in LDS (256 threads: wave w takes blocks w,
// w + 4, ...), after the barrier that completes the rows
template <int NL>
OXE_DEV void q8K_rows_lds(const float (&rows)[NL][shp::E], uint8_t *__restrict__ y) {
    __syncthreads();
    for (int b = threadIdx.x >> 6; b < NL * shp::E / QK; b += 4)
        q8K_block(&rows[0][0] + b * QK, threadIdx.x & 63, y + (int64_t)b * Q8K_BYTES);
}

// ---- integers of one half block (unit h: weights 128 h .. 128 h + 127), every lane ---------------
// y: the lanes' halves h of this block position (YView); out[l * BT<TY>::R + ...]

// get_scale_min_k4 (quants_base.c:50-57)
OXE_DEV void scale_min_k4(int j, const uint8_t *q, int &d, int &m) {
    if (j < 4) {
        d = q[j] & 63;
        m = q[j + 4] & 63;
    } else {
        d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        m = (q[j + 4] >> 4) | ((q[j] >> 6) << 4);
    }
}

// Q4_K / Q5_K: for the unit's two 64-weight steps g: sc_lo * I_lo, sc_hi * I_hi (out[0..3]); Q4_K:
// out[4] = the unit's part of sum min_j * bsum32_j; Q5_K: out[4 + g'] = that sum per step
template <int TY, int NL>
OXE_DEV void unit_k45(const uint8_t *wb, YView y, int h, int *out) {
    constexpr int RES = BT<TY>::R;
    const uint8_t *sc = wb + 4;
    const uint8_t *qs = wb + (TY == 4 ? 16 : 48);
    const uint8_t *qh = wb + 16;
    int bias4[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) bias4[l] = 0;
#pragma unroll
    for (int gg = 0; gg < 2; gg++) {
        const int g = 2 * h + gg;
        int lo[NL], hi[NL];
#pragma unroll
        for (int l = 0; l < NL; l++) lo[l] = hi[l] = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t w = ld32(qs + 32 * g + 4 * i);
            uint32_t cl = w & 0x0F0F0F0Fu, ch = (w >> 4) & 0x0F0F0F0Fu;
            if (TY == 5) {
                const uint32_t hb = ld32(qh + 4 * i);
                cl |= ((hb >> (2 * g)) & 0x01010101u) << 4;
                ch |= ((hb >> (2 * g + 1)) & 0x01010101u) << 4;
            }
#pragma unroll
            for (int l = 0; l < NL; l++) {
                lo[l] = dot4(cl, y.q(l, 16 * gg + i), lo[l]);
                hi[l] = dot4(ch, y.q(l, 16 * gg + 8 + i), hi[l]);
            }
        }
        int s_lo, m_lo, s_hi, m_hi;
        scale_min_k4(2 * g, sc, s_lo, m_lo);
        scale_min_k4(2 * g + 1, sc, s_hi, m_hi);
#pragma unroll
        for (int l = 0; l < NL; l++) {
            out[l * RES + 2 * gg] = s_lo * lo[l];
            out[l * RES + 2 * gg + 1] = s_hi * hi[l];
            const int bias = m_lo * (y.bsum(l, 4 * gg) + y.bsum(l, 4 * gg + 1)) + m_hi * (y.bsum(l, 4 * gg + 2) + y.bsum(l, 4 * gg + 3));
            if (TY == 5) out[l * RES + 4 + gg] = bias;
            bias4[l] += bias;
        }
    }
    if (TY == 4)
#pragma unroll
        for (int l = 0; l < NL; l++) out[l * RES + 4] = bias4[l];
}

// Q6_K: the unit's part of I = sum_i scale_i * (16 codes - 32) . q8 (the -32 through the q8 sums)
template <int NL>
OXE_DEV void unit_q6(const uint8_t *wb, YView y, int n, int *out) {
    constexpr int RES = BT<6>::R;
    const int8_t *sc = (const int8_t *)(wb + 192);
    uint32_t qlw[16], qhw[8];   // ql[64 n .. 64 n + 63], qh[32 n .. 32 n + 31]
    ld_run<16>(wb + 64 * n, qlw);
    ld_run<8>(wb + 128 + 32 * n, qhw);
    int d[NL][8];
#pragma unroll
    for (int l = 0; l < NL; l++)
#pragma unroll
        for (int i = 0; i < 8; i++) d[l][i] = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t a = qlw[i], a2 = qlw[8 + i], hb = qhw[i];
        const uint32_t c0 = (a & 0x0F0F0F0Fu) | ((hb & 0x03030303u) << 4);
        const uint32_t c1 = (a2 & 0x0F0F0F0Fu) | (((hb >> 2) & 0x03030303u) << 4);
        const uint32_t c2 = ((a >> 4) & 0x0F0F0F0Fu) | (((hb >> 4) & 0x03030303u) << 4);
        const uint32_t c3 = ((a2 >> 4) & 0x0F0F0F0Fu) | (((hb >> 6) & 0x03030303u) << 4);
        const int s = i >> 2;   // which 16 of the 32
#pragma unroll
        for (int l = 0; l < NL; l++) {
            d[l][0 + s] = dot4(c0, y.q(l, i), d[l][0 + s]);
            d[l][2 + s] = dot4(c1, y.q(l, 8 + i), d[l][2 + s]);
            d[l][4 + s] = dot4(c2, y.q(l, 16 + i), d[l][4 + s]);
            d[l][6 + s] = dot4(c3, y.q(l, 24 + i), d[l][6 + s]);
        }
    }
#pragma unroll
    for (int l = 0; l < NL; l++) {
        int I = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) I += (int)sc[8 * n + i] * (d[l][i] - 32 * y.bsum(l, i));
        out[l * RES] = I;
    }
}

// q3k_raw_scales (repack_subset.cpp:575-587): raw 6-bit scale i of a Q3_K block
OXE_DEV int q3_raw(const uint8_t *s12, int i) {
    const int lo = i < 8 ? (s12[i] & 15) : (s12[i - 8] >> 4);
    const int hi = (s12[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
    return lo | hi << 4;
}

// Q3_K: the unit's part of isum = sum_i (raw_i - 32) * dot16_i, codes (low 2 bits | hmask bit << 2) - 4
template <int NL>
OXE_DEV void unit_q3(const uint8_t *wb, YView y, int n, int *out) {
    constexpr int RES = BT<3>::R;
    uint32_t qsw[8], hmw[8];   // qs[32 n .. 32 n + 31], hmask[0..31]
    ld_run<8>(wb + 32 + 32 * n, qsw);
    ld_run<8>(wb, hmw);
    int d[NL][8];
#pragma unroll
    for (int l = 0; l < NL; l++)
#pragma unroll
        for (int i = 0; i < 8; i++) d[l][i] = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t qw = qsw[i], hw = hmw[i];
        const int half = i >> 2;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t c = ((qw >> (2 * s)) & 0x03030303u) | (((hw >> (4 * n + s)) & 0x01010101u) << 2);
#pragma unroll
            for (int l = 0; l < NL; l++) d[l][2 * s + half] = dot4(c, y.q(l, 8 * s + i), d[l][2 * s + half]);
        }
    }
    int sc[8];
#pragma unroll
    for (int i = 0; i < 8; i++) sc[i] = q3_raw(wb + 96, 8 * n + i) - 32;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        int I = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) I += sc[i] * (d[l][i] - 4 * y.bsum(l, i));
        out[l * RES] = I;
    }
}

template <int TY, int NL>
OXE_DEV void unit(const uint8_t *wb, YView y, int h, int *out) {
    if (TY == 4 || TY == 5) unit_k45<TY, NL>(wb, y, h, out);
    else if (TY == 6) unit_q6<NL>(wb, y, h, out);
    else unit_q3<NL>(wb, y, h, out);
}

// ---- the reference's float chain over one block (units r0: weights 0..127, r1: 128..255) ---------
template <int TY>
OXE_DEV float chain(float acc, const uint8_t *wb, float dx, const int *r0, const int *r1) {
    if (TY == 4 || TY == 5) {
        // oxe_vl_q4k.inc:1-7 / oxe_vl_q5k.inc:6-12
        const float sbs = h2f(ld16(wb)) * dx, sbm = h2f(ld16(wb + 2)) * dx;
        const int *r[2] = {r0, r1};
        for (int u = 0; u < 2; u++)
            for (int gg = 0; gg < 2; gg++) {
                acc = fmaf(sbs, (float)r[u][2 * gg], acc);
                acc = fmaf(sbs, (float)r[u][2 * gg + 1], acc);
                if (TY == 5) {
                    const float t = sbm * (float)r[u][4 + gg];
                    acc = acc - t;
                }
            }
        if (TY == 4) {
            const float t = (float)(r0[4] + r1[4]) * sbm;
            acc = acc - t;
        }
        return acc;
    }
    if (TY == 6) {   // oxe_vl_q6k.inc:1-8, 107-113: unfused
        const float sbs = h2f(ld16(wb + 208)) * dx;
        const float t = (float)(r0[0] + r1[0]) * sbs;
        return acc + t;
    }
    // Q3_K, oxe_vl_q3k.inc:1-10: fused
    const float sbd = dx * h2f(ld16(wb + 108));
    return fmaf((float)(r0[0] + r1[0]), sbd, acc);
}

// ---- the lane GEMV --------------------------------------------------------------------------------
// s[l * nr + r] = W[r] . y[l]; w: nr rows of nb blocks (row bytes a multiple of 4, w 16-byte
// aligned); y: NL lanes of nb q8_K blocks. One wave per workgroup, persistent over groups of 4 rows
// (16 threads per row). Per group: the 4 rows' bytes (contiguous) go to LDS with 16-byte loads, the
// first PF x 1 KiB of them held in registers, two groups ahead (buffers a and b, alternating); then
// per chunk of up to 8 blocks thread (row ri, unit u) forms half block u % 2 of block u / 2 for
// every lane, and threads u < NL of each row run lane u's chain over the chunk's blocks in order.
// The register loads are unconditional (indices clamped into the group; a group past the end
// re-reads the last one and writes nothing): a load under a per-thread condition makes the
// compiler wait for every outstanding load before the first LDS store, which drains the second
// buffer (measured: 2-deep conditional 143.8 us, unconditional 130.6 us for the Q6_K LM head).
constexpr int GR = 4;     // rows per group
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));   // a plain vector (HIP's uint4 is a union
                                                              // type that keeps arrays of it in scratch)

__host__ __device__ inline int align16(int n) { return (n + 15) / 16 * 16; }

// the first PF x 1 KiB of group g's bytes (g < ngroups) into registers, non-temporal 16-byte loads
template <int PF>
OXE_DEV void pf_load(u32x4 (&pf)[PF], const uint8_t *w, int64_t g, int64_t nr, int row_bytes, int t) {
    const u32x4 *src = (const u32x4 *)(w + g * GR * row_bytes);
    const int n16 = (int)(min((int64_t)GR, nr - g * GR) * row_bytes) / 16;
#pragma unroll
    for (int j = 0; j < PF; j++) pf[j] = __builtin_nontemporal_load(src + min(t + 64 * j, n16 - 1));
}

// the consumer of an engine phase's GEMV, applied at its store (ctl null: lane u's value to s[u][r]):
// row r of lane u < ctl->nl, in an active run only, goes to dst[u][r] (lane stride ld), plus
// resid[u][r] when resid is given (one fp32 add, as a separate pass would make it), and as fp16 to
// the V^T cache row r at position pos0 + u when vt is given
struct KqEpi {
    const RunCtl *ctl = nullptr;
    float *dst = nullptr;
    int64_t ld = 0;
    const float *resid = nullptr;
    uint16_t *vt = nullptr;
    int64_t vt_ld = 0;
};

// up to four matrices of one type and row length over the same activation in one launch (a
// projection's parts): groups are numbered through the segments in order; segment i's rows go to
// dst at row offset off[i] (its lane values to s when there is no epilogue: one segment then), and
// segment vseg's also to V^T
constexpr int KQ_SEGS = 4;
struct KqSegs {
    int n = 0;
    int vseg = -1;
    int64_t ngroups = 0;
    const uint8_t *w[KQ_SEGS] = {};
    int64_t nr[KQ_SEGS] = {};
    int64_t g0[KQ_SEGS] = {};
    int64_t off[KQ_SEGS] = {};
};

struct SegRef {
    const uint8_t *w;
    int64_t nr, gl, off;   // rows, the group's index within the segment, row offset in dst
    bool v;
};

// the segment of group g (fixed indices only, so the table stays in the kernel arguments)
OXE_DEV SegRef seg_ref(const KqSegs &S, int64_t g) {
    SegRef r{S.w[0], S.nr[0], g, S.off[0], S.vseg == 0};
#pragma unroll
    for (int j = 1; j < KQ_SEGS; j++)
        if (j < S.n && g >= S.g0[j]) r = SegRef{S.w[j], S.nr[j], g - S.g0[j], S.off[j], S.vseg == j};
    return r;
}

// one group of 4 rows (g may be past the end: then nothing is written): its prefetched bytes (pf)
// and the rest to LDS, pf refilled with group g_next, then the units and the chains
template <int TY, int NL, int PF>
OXE_DEV void vl_group(u32x4 (&pf)[PF], int64_t g, int64_t g_next, const KqSegs &S, int nb, float *__restrict__ s,
                      const KqEpi &epi, uint8_t *wl, const uint32_t *yh, const float *yd, int *res) {
    constexpr int BB = BT<TY>::B;
    constexpr int RES = BT<TY>::R;
    constexpr int RS = (NL * RES) | 1;   // odd per-thread stride: no bank conflicts between threads
    const int row_bytes = nb * BB, ls = y_lane_words(nb);
    const int t = threadIdx.x, ri = t >> 4, u = t & 15;
    const int64_t ngroups = S.ngroups;
    const bool gin = g < ngroups;
    const SegRef sg = seg_ref(S, gin ? g : ngroups - 1);   // the group whose bytes pf holds
    const int64_t nr = sg.nr;
    const int sp = (int)(min((int64_t)GR, nr - sg.gl * GR) * row_bytes), n16 = sp / 16;
    const u32x4 *src = (const u32x4 *)(sg.w + sg.gl * GR * row_bytes);
    __syncthreads();   // the previous group's LDS reads are done
#pragma unroll
    for (int j = 0; j < PF; j++) ((u32x4 *)wl)[min(t + 64 * j, n16 - 1)] = pf[j];   // clamped: same bytes
    for (int i = t + 64 * PF; i < n16; i += 64) ((u32x4 *)wl)[i] = src[i];
    for (int i = n16 * 4 + t; i < sp / 4; i += 64) ((uint32_t *)wl)[i] = ((const uint32_t *)src)[i];   // tail
    __syncthreads();
    {
        const SegRef sn = seg_ref(S, g_next < ngroups ? g_next : ngroups - 1);
        pf_load(pf, sn.w, sn.gl, sn.nr, row_bytes, t);   // in flight meanwhile
    }
    const int64_t r = sg.gl * GR + ri;
    const bool live = gin && r < nr;
    float acc = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += 8) {
        const int kc = min(8, nb - b0);
        const int bi = b0 + (u >> 1);
        if ((u >> 1) < kc && live)
            unit<TY, NL>(wl + ri * row_bytes + bi * BB, YView{yh + (2 * bi + (u & 1)) * YH, ls}, u & 1, res + t * RS);
        __syncthreads();
        if (u < NL && live)
            for (int b = 0; b < kc; b++) {
                const int *r0 = res + (ri * 16 + 2 * b) * RS + u * RES;
                const int *r1 = res + (ri * 16 + 2 * b + 1) * RS + u * RES;
                acc = chain<TY>(acc, wl + ri * row_bytes + (b0 + b) * BB, yd[u * nb + b0 + b], r0, r1);
            }
        __syncthreads();
    }
    if (u < NL && live) {
        if (!epi.ctl) {
            s[(int64_t)u * nr + r] = acc;
        } else if (epi.ctl->active && u < epi.ctl->nl) {
            const int64_t i = (int64_t)u * epi.ld + sg.off + r;
            const float v = epi.resid ? acc + epi.resid[i] : acc;
            epi.dst[i] = v;
            if (sg.v && epi.vt) epi.vt[r * epi.vt_ld + epi.ctl->pos0 + u] = f2h(v);
        }
    }
}

template <int TY, int NL, int PF>
__global__ __launch_bounds__(64) void vl_gemv_kernel(KqSegs S, int nb, const uint8_t *__restrict__ y,
                                                     float *__restrict__ s, KqEpi epi) {
    constexpr int BB = BT<TY>::B;
    extern __shared__ __align__(16) uint8_t lds[];
    const int row_bytes = nb * BB;
    uint8_t *wl = lds;                                                   // [GR][row_bytes]
    uint32_t *yh = (uint32_t *)(lds + align16(GR * row_bytes));         // [NL][nb][2][YH]
    float *yd = (float *)(yh + NL * y_lane_words(nb));                   // [NL][nb]
    int *res = (int *)((uint8_t *)yh + align16(NL * nb * (2 * YH + 1) * 4));   // [64][(NL * R) | 1]
    const int t = threadIdx.x;
    const int64_t ngroups = S.ngroups, G = gridDim.x;
    // the lanes' q8_K blocks (lane l block b is block l nb + b) repacked into halves and scales
    for (int i = t; i < NL * nb * 2 * 36; i += 64) {
        const int wd = i % 36, hb = i / 36, h = hb & 1;
        const uint32_t *src = (const uint32_t *)(y + (int64_t)(hb >> 1) * Q8K_BYTES);
        yh[hb * YH + wd] = wd < 32 ? src[1 + 32 * h + wd] : src[65 + 4 * h + (wd - 32)];
    }
    for (int i = t; i < NL * nb; i += 64) yd[i] = *(const float *)(y + (int64_t)i * Q8K_BYTES);
    // two register buffers (fixed indices only: they stay in registers), groups g and g + G in
    // flight from the start; the scheduling barrier keeps buffer a's loads ahead of b's, so the
    // first LDS stores wait for a's only
    u32x4 pa[PF], pb[PF];
    if ((int64_t)blockIdx.x >= ngroups) return;
    {
        const SegRef sa = seg_ref(S, blockIdx.x), sb = seg_ref(S, min((int64_t)blockIdx.x + G, ngroups - 1));
        pf_load(pa, sa.w, sa.gl, sa.nr, row_bytes, t);
        __builtin_amdgcn_sched_barrier(0);
        pf_load(pb, sb.w, sb.gl, sb.nr, row_bytes, t);
    }
    for (int64_t g = blockIdx.x; g < ngroups; g += 2 * G) {
        vl_group<TY, NL, PF>(pa, g, g + 2 * G, S, nb, s, epi, wl, yh, yd, res);
        vl_group<TY, NL, PF>(pb, g + G, g + 3 * G, S, nb, s, epi, wl, yh, yd, res);
    }
}

size_t vl_gemv_lds(int bb, int rr, int nb, int nl) {
    return (size_t)align16(GR * nb * bb) + (size_t)align16(nl * nb * (2 * YH + 1) * 4) + (size_t)64 * ((nl * rr) | 1) * 4;
}

constexpr int KQ_MAX_DEV = 64;
template <int TY, int NL, int PF>
int vl_gemv_launch_pf(const KqSegs &S, int nb, const uint8_t *y, float *s, hipStream_t st, const KqEpi &epi) {
    constexpr int BB = BT<TY>::B;
    const size_t lds = vl_gemv_lds(BB, BT<TY>::R, nb, NL);
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= KQ_MAX_DEV) return -2;
    // per instantiation and device: the dynamic LDS the kernel is configured for (above 64 KiB it
    // needs the attribute; 160 KiB per CU), the CU count, and the occupancy per LDS size, each asked
    // of the runtime once (a query per launch would sit on the decode path)
    struct Cache {
        size_t configured = 65536;
        int ncu = 0;
        size_t lds[8] = {};
        int occ[8] = {};
    };
    static Cache cache[KQ_MAX_DEV];
    static std::mutex mu;
    int ncu = 256, occ = 0;
    {
        std::lock_guard<std::mutex> lk(mu);
        Cache &cc = cache[dev];
        if (lds > cc.configured) {
            if (hipFuncSetAttribute((const void *)vl_gemv_kernel<TY, NL, PF>, hipFuncAttributeMaxDynamicSharedMemorySize,
                                    (int)lds) != hipSuccess)
                return -2;
            cc.configured = lds;
        }
        if (cc.ncu == 0 && hipDeviceGetAttribute(&cc.ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
            cc.ncu = 256;
        ncu = cc.ncu;
        int slot = -1;
        for (int i = 0; i < 8 && slot < 0; i++)
            if (cc.lds[i] == lds || cc.lds[i] == 0) slot = i;
        if (slot >= 0 && cc.lds[slot] == lds) {
            occ = cc.occ[slot];
        } else {
            // exactly the waves a CU holds, by LDS and registers both: a grid beyond them leaves its
            // last waves to start after others finish, one below them leaves SIMDs short of a wave
            // (measured on the Q6_K LM head, 12 resident per CU: 11 per CU 131 us, 13 per CU 116 us,
            // 12 per CU 92.5 us)
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&occ, vl_gemv_kernel<TY, NL, PF>, 64, lds) != hipSuccess ||
                occ < 1)
                occ = (int)std::max<size_t>(1, (160 * 1024) / lds);
            if (slot >= 0) {
                cc.lds[slot] = lds;
                cc.occ[slot] = occ;
            }
        }
    }
    const int per_cu = std::min(16, occ);
    const int64_t grid = std::min<int64_t>(S.ngroups, (int64_t)ncu * per_cu);
    hipLaunchKernelGGL((vl_gemv_kernel<TY, NL, PF>), dim3((unsigned)grid), dim3(64), lds, st, S, nb, y, s, epi);
    return hipGetLastError() == hipSuccess ? 1 : -2;
}

// registers per prefetch buffer: the smallest of 2, 4, 8 KiB-per-wave steps that holds a whole group
// (the rest of a larger group is copied to LDS directly)
template <int TY, int NL>
int vl_gemv_launch(const KqSegs &S, int nb, const uint8_t *y, float *s, hipStream_t st, const KqEpi &epi) {
    const int n16 = GR * nb * BT<TY>::B / 16;
    if (n16 <= 128) return vl_gemv_launch_pf<TY, NL, 2>(S, nb, y, s, st, epi);
    if (n16 <= 256) return vl_gemv_launch_pf<TY, NL, 4>(S, nb, y, s, st, epi);
    return vl_gemv_launch_pf<TY, NL, 8>(S, nb, y, s, st, epi);
}

// one matrix [nr rows of nb blocks] as a one-segment table
inline KqSegs one_seg(const uint8_t *w, int64_t nr) {
    KqSegs S;
    S.n = 1;
    S.w[0] = w;
    S.nr[0] = nr;
    S.ngroups = (nr + GR - 1) / GR;
    return S;
}

template <int TY>
int vl_gemv_segs(const KqSegs &S, int nb, const uint8_t *y, int nl, float *s, hipStream_t st, const KqEpi &epi) {
    switch (nl) {
        case 1: return vl_gemv_launch<TY, 1>(S, nb, y, s, st, epi);
        case 2: return vl_gemv_launch<TY, 2>(S, nb, y, s, st, epi);
        case 3: return vl_gemv_launch<TY, 3>(S, nb, y, s, st, epi);
        default: return vl_gemv_launch<TY, 4>(S, nb, y, s, st, epi);
    }
}

template <int TY>
int vl_gemv_type(const uint8_t *w, int nb, int64_t nr, const uint8_t *y, int nl, float *s, hipStream_t st) {
    return vl_gemv_segs<TY>(one_seg(w, nr), nb, y, nl, s, st, KqEpi{});
}


// ==== K-quant and F32 matrices in the engine's per-phase runs ======================================
// (the reference's mv / mv_lanes over any qtype, crates/model/src/engine.rs:2270-2343; MoE phases
// engine.rs:3437-3625; LM head 3630-3715). Every (lane, row) value is the lane GEMV's: the same
// block units and float chain as vl_gemv_kernel, on the activation quantised as the weight's type
// asks (q8_K for K-quants, Q8_0 for Q8_0, the f32 vector itself for F32 rows).

// ggml type id (11..14) -> the units / chain of that type
template <int NL>
OXE_DEV void unit_rt(int type, const uint8_t *wb, YView y, int h, int *out) {
    switch (type) {
        case 11: unit<3, NL>(wb, y, h, out); break;
        case 12: unit<4, NL>(wb, y, h, out); break;
        case 13: unit<5, NL>(wb, y, h, out); break;
        default: unit<6, NL>(wb, y, h, out); break;
    }
}
OXE_DEV float chain_rt(int type, float acc, const uint8_t *wb, float dx, const int *r0, const int *r1) {
    switch (type) {
        case 11: return chain<3>(acc, wb, dx, r0, r1);
        case 12: return chain<4>(acc, wb, dx, r0, r1);
        case 13: return chain<5>(acc, wb, dx, r0, r1);
        default: return chain<6>(acc, wb, dx, r0, r1);
    }
}
OXE_DEV int res_of(int type) { return type == 12 ? BT<4>::R : type == 13 ? BT<5>::R : 1; }
constexpr int RES_MAX = 6;

// nblk q8_K blocks (292 bytes each, from y) into LDS as halves (YH words apart) and scales
OXE_DEV void stage_q8k(const uint8_t *y, int nblk, uint32_t *yh, float *yd) {
    for (int i = threadIdx.x; i < nblk * 2 * 36; i += blockDim.x) {
        const int wd = i % 36, hb = i / 36, h = hb & 1;
        const uint32_t *src = (const uint32_t *)(y + (int64_t)(hb >> 1) * Q8K_BYTES);
        yh[hb * YH + wd] = wd < 32 ? src[1 + 32 * h + wd] : src[65 + 4 * h + (wd - 32)];
    }
    for (int i = threadIdx.x; i < nblk; i += blockDim.x) yd[i] = *(const float *)(y + (int64_t)i * Q8K_BYTES);
}

OXE_DEV uint32_t ordered_bits(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// ---- F32 ssm_beta / ssm_alpha rows: x -> rms_norm * attn_norm (every workgroup, exact), then
// oxe_vec_dot_f32 per (row, lane) in ggml_vec_dot_f32's order (vec.cpp:104-125): lane c of a
// 16-lane group runs chain c over elements c + 16 s; xor 8, 4, 1, 2 is the NEON reduction tree.
// Workgroup b: rows 16 b .. 16 b + 15 of [beta rows | alpha rows]; outputs into the projection
// buffer at DN_BETA / DN_ALPHA, where the delta-net phase reads them.
template <int NL>
__global__ __launch_bounds__(256) void ba_f32_kernel(const RunCtl *__restrict__ ctl, const float *x, const float *norm_w,
                                                     float eps, const float *beta, const float *alpha, float *proj) {
    __shared__ float s_xn[NL][shp::E];
    __shared__ NormScratch ns;
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        float v[EPT];
        if (l < nl) {
            load8(x + (int64_t)l * shp::E, v);
            rms_norm_mul_e(v, x + (int64_t)l * shp::E, norm_w, eps, ns);
        } else {
#pragma unroll
            for (int i = 0; i < EPT; i++) v[i] = 0.0f;
        }
        store8(s_xn[l], v);
    }
    __syncthreads();
    const int c = t & 15, row = blockIdx.x * 16 + (t >> 4);
    const bool is_beta = row < shp::NVH;
    const float *w = (is_beta ? beta + (int64_t)row * shp::E : alpha + (int64_t)(row - shp::NVH) * shp::E);
    float acc[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) acc[l] = 0.0f;
#pragma unroll 32
    for (int s = 0; s < shp::E / 16; s++) {
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
        if (c == 0 && l < nl) proj[(int64_t)l * shp::DN_ROWS + (is_beta ? shp::DN_BETA + row : shp::DN_ALPHA + row - shp::NVH)] = v;
    }
}

// ---- MoE gate / up over K-quant matrices: workgroup (unit u, tile of 8 rows), u < OXE_MAX_UNION
// the union's expert u, u = OXE_MAX_UNION the shared expert. Thread (matrix t / 128: gate, up; row
// t / 16 % 8, half block t % 16) forms its half block's integers for every lane; threads t % 16 < NL
// then run lane t % 16's chain over the row's 8 blocks, gate and up at once; then silu(g) * u
// (ggml_v_silu, as swiglu) for every lane that routed to the expert (the shared expert: every lane).
struct KqGuArgs {
    const uint8_t *xk;          // [NL][E / 256] q8_K blocks of xn
    RawW gate, up, sh_gate, sh_up;
    const int32_t *uni, *route_ids;
    float *hexp;                // [NL][KUSED][FF]
    float *hsh;                 // [NL][FFSH]
    int do_exp, do_sh;
    uint32_t *stats;            // [0] sum of union sizes, [1] launches (as the Q8_0 experts phase counts)
};
constexpr int GU_NB = shp::E / QK;   // 8 blocks per row
constexpr int GU_R = 8;              // rows per workgroup
static_assert(GU_NB * 2 == 16 && shp::FF == shp::FFSH, "16 half blocks per row; one tiling for both");

template <int NL>
__global__ __launch_bounds__(256) void kq_gu_kernel(const RunCtl *__restrict__ ctl, KqGuArgs a) {
    constexpr int RS = (NL * RES_MAX) | 1;
    __shared__ uint32_t yh[NL * GU_NB * 2 * YH];
    __shared__ float yd[NL * GU_NB];
    __shared__ int res[256 * RS];
    __shared__ float s_gu[2][GU_R][NL];
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x, which = t >> 7, ri = (t >> 4) & (GU_R - 1), hu = t & 15;
    const int u = blockIdx.x / (shp::FF / GU_R), tile = blockIdx.x % (shp::FF / GU_R);
    const bool sh = u == OXE_MAX_UNION;
    if (a.do_exp && blockIdx.x == 0 && t == 0) {
        atomicAdd(a.stats, (uint32_t)a.uni[0]);
        atomicAdd(a.stats + 1, 1u);
    }
    if (sh ? !a.do_sh : !a.do_exp) return;
    int e = 0;
    if (!sh) {
        int nu = a.uni[0];
        nu = nu < 0 ? 0 : (nu > OXE_MAX_UNION ? OXE_MAX_UNION : nu);
        if (u >= nu) return;
        e = a.uni[1 + u];
        e = e < 0 ? 0 : (e >= shp::NEXP ? shp::NEXP - 1 : e);
    }
    stage_q8k(a.xk, NL * GU_NB, yh, yd);
    __syncthreads();
    const int row = tile * GU_R + ri;
    {
        const RawW &W = sh ? (which ? a.sh_up : a.sh_gate) : (which ? a.up : a.gate);
        const int type = W.type, rs = res_of(type);
        const int64_t rb = raw_row_bytes(W);
        const uint8_t *wr = W.w + ((int64_t)e * W.rows + row) * rb;
        unit_rt<NL>(type, wr + (hu >> 1) * kq_block_bytes(type), YView{yh + (2 * (hu >> 1) + (hu & 1)) * YH, GU_NB * 2 * YH},
                    hu & 1, res + t * RS);
        __syncthreads();
        if (hu < NL) {
            float acc = 0.0f;
            for (int b = 0; b < GU_NB; b++) {
                const int *r0 = res + ((t & ~15) + 2 * b) * RS + hu * rs, *r1 = res + ((t & ~15) + 2 * b + 1) * RS + hu * rs;
                acc = chain_rt(type, acc, wr + b * kq_block_bytes(type), yd[hu * GU_NB + b], r0, r1);
            }
            s_gu[which][ri][hu] = acc;
        }
        __syncthreads();
    }
    if (which == 0 && hu < NL && hu < nl) {
        const float h = v_silu(s_gu[0][ri][hu]) * s_gu[1][ri][hu];
        if (sh) {
            a.hsh[(int64_t)hu * shp::FFSH + row] = h;
        } else {
            int j = -1;
            for (int jj = 0; jj < shp::KUSED; jj++)
                if (a.route_ids[hu * shp::KUSED + jj] == e) j = jj;
            if (j >= 0) a.hexp[((int64_t)hu * shp::KUSED + j) * shp::FF + row] = h;
        }
    }
}

// ---- MoE down + combine with any mix of K-quant and Q8_0 down matrices: workgroup = 16 output
// rows; units 0..nu-1 the union's experts, unit OXE_MAX_UNION the shared expert. Each (unit, lane,
// row) value is that matrix's row dot with the lane's h (slot j of the lane's top-k, or the shared
// h): K-quants on h's q8_K blocks (2 per row of 512), four units per pass with 64 threads each
// (row, half block); Q8_0 on h quantised to Q8_0 in LDS, one thread per (unit, lane, row) running
// the block chain. Then the reference's combine (engine.rs:3591-3601):
// m = d0 w0; m += dj wj; f = m + dsh * g; x2 = f + x1.
struct KqDownArgs {
    const int32_t *uni, *route_ids;
    const float *route_w, *sh_gate;
    const float *hexp, *hsh;        // f32 h (Q8_0 matrices quantise it here)
    const uint8_t *hk, *hshk;       // q8_K blocks of h (K-quant matrices)
    Q8W exp_down, shexp_down;
    RawW exp_down_r, sh_down_r;
    const float *x1;
    float *x2;
    unsigned long long *amax_key;
};
constexpr int DN_R = 8;                      // output rows per workgroup (E / 8 = 256 workgroups)
constexpr int DN_NB = shp::FF / QK;          // 2 blocks per down row
constexpr int DN_U = OXE_MAX_UNION + 1;
constexpr int DN_A = shp::KUSED + 1;         // activation rows per lane: the k slots, then the shared h

template <int NL>
__global__ __launch_bounds__(256) void kq_down_kernel(const RunCtl *__restrict__ ctl, KqDownArgs a) {
    constexpr int RS = (NL * RES_MAX) | 1;   // odd per-thread stride of the unit integers
    __shared__ uint32_t yh[NL * DN_A * DN_NB * 2 * YH];
    __shared__ float yd[NL * DN_A * DN_NB];
    __shared__ int8_t s_q[NL * DN_A][shp::FF];
    __shared__ uint16_t s_d[NL * DN_A][shp::FF / 32];
    __shared__ int res[256 * RS];
    __shared__ float s_dn[NL][DN_A][DN_R];
    __shared__ int32_t s_e[DN_U], s_slot[DN_U][NL];
    __shared__ float s_w[NL][shp::KUSED], s_sg[NL];
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
    const int64_t row0 = (int64_t)blockIdx.x * DN_R;
    if (blockIdx.x == 0 && t < NL) a.amax_key[t] = 0ull;   // the LM head that follows starts clean
    int nu = a.uni[0];
    nu = nu < 0 ? 0 : (nu > OXE_MAX_UNION ? OXE_MAX_UNION : nu);
    const bool exp_kq = a.exp_down_r.type != 8, sh_kq = a.sh_down_r.type != 8;
    if (t < DN_U) {
        const int e = t < OXE_MAX_UNION ? (t < nu ? a.uni[1 + t] : -1) : 0;
        s_e[t] = e < 0 ? 0 : (e < shp::NEXP ? e : shp::NEXP - 1);   // slots below compare the unclamped id
        for (int l = 0; l < NL; l++) {
            int j = -1;
            if (l < nl) {
                if (t == OXE_MAX_UNION) j = shp::KUSED;
                else if (e >= 0)
                    for (int jj = 0; jj < shp::KUSED; jj++)
                        if (a.route_ids[l * shp::KUSED + jj] == e) j = jj;
            }
            s_slot[t][l] = j;
        }
    }
    if (t < NL * shp::KUSED) s_w[t / shp::KUSED][t % shp::KUSED] = t / shp::KUSED < nl ? a.route_w[t] : 0.0f;
    if (t < NL) s_sg[t] = t < nl ? a.sh_gate[t] : 0.0f;
    // activations: activation row ar = l * DN_A + j (j = KUSED: the shared h)
    if (exp_kq || sh_kq) {
        for (int l = 0; l < NL; l++) {
            if (exp_kq) stage_q8k(a.hk + (int64_t)l * shp::KUSED * DN_NB * Q8K_BYTES, shp::KUSED * DN_NB,
                                  yh + l * DN_A * DN_NB * 2 * YH, yd + l * DN_A * DN_NB);
            if (sh_kq) stage_q8k(a.hshk + (int64_t)l * DN_NB * Q8K_BYTES, DN_NB, yh + (l * DN_A + shp::KUSED) * DN_NB * 2 * YH,
                                 yd + (l * DN_A + shp::KUSED) * DN_NB);
        }
    }
    if (!exp_kq || !sh_kq) {
        for (int i = t; i < NL * DN_A * (shp::FF / 32); i += 256) {
            const int ar = i / (shp::FF / 32), b = i % (shp::FF / 32), l = ar / DN_A, j = ar % DN_A;
            const bool want = j < shp::KUSED ? !exp_kq : !sh_kq;
            if (want && l < nl) {
                const float *src = j < shp::KUSED ? a.hexp + ((int64_t)l * shp::KUSED + j) * shp::FF + 32 * b
                                                  : a.hsh + (int64_t)l * shp::FFSH + 32 * b;
                quant_block_q8_0(src, &s_q[ar][32 * b], &s_d[ar][b]);
            }
        }
    }
    __syncthreads();
    // K-quant units, eight per pass: thread (unit u0 + t / 32, row t / 4 % 8, half block t % 4) forms
    // its half block's integers for every lane with a slot there; threads t % 4 < NL then run lane
    // t % 4's chain over the row's two blocks
    static_assert(DN_R == 8, "thread mapping of the K-quant units");
    {
        const int p = t >> 5, rr = (t >> 2) & 7, hu = t & 3;
        for (int u0 = 0; u0 < DN_U; u0 += 8) {
            const int u = u0 + p;
            const bool live = u < DN_U && (u == OXE_MAX_UNION ? sh_kq : (exp_kq && u < nu));
            const RawW &W = u == OXE_MAX_UNION ? a.sh_down_r : a.exp_down_r;
            const int type = W.type, rs = res_of(type), bb = kq_block_bytes(type);
            const uint8_t *wr = live ? W.w + ((int64_t)s_e[u] * W.rows + row0 + rr) * raw_row_bytes(W) : nullptr;
            if (live)
                for (int l = 0; l < NL; l++) {
                    const int j = s_slot[u][l];
                    if (j >= 0)
                        unit_rt<1>(type, wr + (hu >> 1) * bb, YView{yh + ((l * DN_A + j) * DN_NB * 2 + hu) * YH, 0}, hu & 1,
                                   res + t * RS + l * rs);
                }
            __syncthreads();
            if (live && hu < NL && s_slot[u][hu] >= 0) {
                const int ar = hu * DN_A + s_slot[u][hu];
                float acc = 0.0f;
                for (int b = 0; b < DN_NB; b++) {
                    const int *r0 = res + ((t & ~3) + 2 * b) * RS + hu * rs, *r1 = res + ((t & ~3) + 2 * b + 1) * RS + hu * rs;
                    acc = chain_rt(type, acc, wr + b * bb, yd[ar * DN_NB + b], r0, r1);
                }
                s_dn[hu][s_slot[u][hu]][rr] = acc;
            }
            __syncthreads();
        }
    }
    // Q8_0 units: one thread per (unit, lane, row), the block chain of the Q8_0 GEMV
    for (int i = t; i < DN_U * NL * DN_R; i += 256) {
        const int u = i / (NL * DN_R), l = (i / DN_R) % NL, rr = i % DN_R;
        const bool sh = u == OXE_MAX_UNION;
        if (sh ? sh_kq : (exp_kq || u >= nu)) continue;
        const int j = s_slot[u][l];
        if (j < 0) continue;
        const int64_t row = row0 + rr;
        const int8_t *wq = sh ? a.shexp_down.q + row * shp::FFSH : a.exp_down.q + ((int64_t)s_e[u] * shp::E + row) * shp::FF;
        const uint16_t *wd = sh ? a.shexp_down.d + row * (shp::FFSH / 32)
                                : a.exp_down.d + ((int64_t)s_e[u] * shp::E + row) * (shp::FF / 32);
        const int ar = l * DN_A + j;
        float acc = 0.0f;
        for (int b = 0; b < shp::FF / 32; b++) {
            int32_t s = 0;
#pragma unroll
            for (int k = 0; k < 8; k++)
                s = dot4(*(const uint32_t *)(wq + 32 * b + 4 * k), *(const uint32_t *)&s_q[ar][32 * b + 4 * k], s);
            acc = __builtin_fmaf((float)s, h2f(s_d[ar][b]) * h2f(wd[b]), acc);
        }
        s_dn[l][j][rr] = acc;
    }
    __syncthreads();
    if (t < NL * DN_R) {
        const int l = t / DN_R, rr = t % DN_R;
        if (l < nl) {
            float m = s_dn[l][0][rr] * s_w[l][0];
            for (int j = 1; j < shp::KUSED; j++) {
                const float pp = s_dn[l][j][rr] * s_w[l][j];
                m = m + pp;
            }
            const float sv = s_dn[l][shp::KUSED][rr] * s_sg[l];
            const float f = m + sv;
            a.x2[(int64_t)l * shp::E + row0 + rr] = f + a.x1[(int64_t)l * shp::E + row0 + rr];
        }
    }
}

// ---- LM head over a K-quant matrix: the normed x2 (h_nextn) of every lane, q8_K blocks of it, the
// lane GEMV into the logits, then the first strict maximum per wanted lane (NaN never wins; all
// -inf: no key, argmax 0), packed as the per-phase head packs it: (ordered value << 32) | ~row.
template <int NL>
__global__ __launch_bounds__(256) void kq_head_norm_kernel(const RunCtl *__restrict__ ctl, const float *x2,
                                                           const float *norm_w, float eps, float *hid, float *xn,
                                                           uint8_t *xk) {
    __shared__ NormScratch ns;
    __shared__ float s_n[NL][shp::E];
    if (!ctl->active) return;
    const int nl = ctl->nl, t = threadIdx.x;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        float v[EPT];
        if (l < nl) {
            load8(x2 + (int64_t)l * shp::E, v);
            rms_norm_mul_e(v, x2 + (int64_t)l * shp::E, norm_w, eps, ns);
            store8(hid + (int64_t)l * shp::E, v);
        } else {
#pragma unroll
            for (int i = 0; i < EPT; i++) v[i] = 0.0f;
        }
        store8(xn + (int64_t)l * shp::E, v);
        store8(s_n[l], v);
    }
    q8K_rows_lds<NL>(s_n, xk);   // the head GEMV's activation
}

template <int NL>
__global__ __launch_bounds__(1024) void kq_argmax_kernel(const RunCtl *__restrict__ ctl, const float *logits, int64_t nv,
                                                         unsigned long long *amax_key, const uint32_t *ids) {
    __shared__ unsigned long long red[16];
    if (!ctl->active) return;
    const int l = blockIdx.x, t = threadIdx.x;
    if (l >= ctl->nl || !((ctl->head_mask >> l) & 1)) return;
    float best = -__builtin_inff();
    int64_t bi = -1;
    for (int64_t r = t; r < nv; r += 1024) {
        const float v = logits[(int64_t)l * nv + r];
        if (v > best) { best = v; bi = r; }
    }
    // a restricted draft head's rows are ascending token ids: the first maximum by row is the first by id
    const uint32_t id = bi < 0 ? 0u : (ids ? ids[bi] : (uint32_t)bi);
    unsigned long long key = bi >= 0 ? ((unsigned long long)ordered_bits(best) << 32) | (0xffffffffu - id) : 0ull;
    for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(key, m, 64);
        key = o > key ? o : key;
    }
    if ((t & 63) == 0) red[t >> 6] = key;
    __syncthreads();
    if (t == 0) {
        unsigned long long k = 0ull;
        for (int i = 0; i < 16; i++) k = red[i] > k ? red[i] : k;
        if (k) atomicMax(&amax_key[l], k);
    }
}

// ---- K-quant mixer matrices and token embedding in the per-phase runs ----------------------------
// dequantize_row_q{3,4,5,6}_K (vendor/ggml-subset/generated/quants_base.c:80-230) of element i of
// one 256-weight block b (type 11..14), as the reference builds it: GCC's default contraction
// (crates/kernels-sys/build.rs:5-7) makes the Q4_K / Q5_K element (d * scale) * code - dmin * min
// one fused multiply-subtract; Q3_K and Q6_K are products in source order.
OXE_DEV float ld_f16u(const uint8_t *p) { return h2f((uint16_t)(p[0] | (p[1] << 8))); }
OXE_DEV float kq_elem(int type, const uint8_t *b, int i) {
    switch (type) {
        case 12:
        case 13: {
            const float d = ld_f16u(b), mn = ld_f16u(b + 2);
            const int c = i >> 6, hi = (i >> 5) & 1, l = i & 31;
            const uint8_t *q = b + (type == 12 ? 16 : 48) + 32 * c;
            int sc, mi;
            scale_min_k4(2 * c + hi, b + 4, sc, mi);
            int qq = hi ? (q[l] >> 4) : (q[l] & 0xF);
            if (type == 13 && (b[16 + l] & ((1 + hi) << (2 * c)))) qq += 16;
            return __builtin_fmaf(d * (float)sc, (float)qq, -(mn * (float)mi));
        }
        case 14: {
            const float d = ld_f16u(b + 208);
            const int n = i >> 7, r = i & 127, qd = r >> 5, l = r & 31;
            const uint8_t *ql = b + 64 * n, *qh = b + 128 + 32 * n;
            const int8_t sc = (int8_t)b[192 + 8 * n + (l >> 4) + 2 * qd];
            const int lo = (qd & 1) ? ql[l + 32] : ql[l];
            const int q = ((qd >> 1) ? (lo >> 4) : (lo & 0xF)) | (((qh[l] >> (2 * qd)) & 3) << 4);
            return d * (float)sc * (float)(q - 32);
        }
        default: {   // 11: Q3_K
            const float dall = ld_f16u(b + 108);
            const int n = i >> 7, r = i & 127, j = r >> 5, hf = (r >> 4) & 1, idx = (r & 15) + 16 * hf;
            const float dl = dall * (float)(q3_raw(b + 96, 8 * n + 2 * j + hf) - 32);
            const int code = (b[32 + 32 * n + idx] >> (2 * j)) & 3;
            return dl * (float)(code - ((b[idx] & (1 << (4 * n + j))) ? 0 : 4));
        }
    }
}

// the lanes' token rows of a K-quant embedding (engine.rs:2251-2256): workgroup l = lane
template <int NL>
__global__ __launch_bounds__(256) void kq_embed_kernel(const RunCtl *__restrict__ ctl, const uint8_t *w, int type,
                                                       int64_t row_bytes, float *out) {
    if (!ctl->active) return;
    const int l = blockIdx.x;
    if (l >= ctl->nl) return;
    const uint8_t *row = w + (int64_t)ctl->tok[l] * row_bytes;
    const int bb = kq_block_bytes(type);
    for (int i = threadIdx.x; i < shp::E; i += 256) out[(int64_t)l * shp::E + i] = kq_elem(type, row + (i / QK) * bb, i % QK);
}

// the lanes' projection input: xn = rms_norm(x) * attn_norm (oxe_ops.cpp:32-42), x the embedding
// (Q8_0 emb, or the dequantised rows embf; stored to x_store, the residual of layer 0) or x; lanes
// past the run's are zero
template <int NL>
__global__ __launch_bounds__(256) void kq_norm_kernel(const RunCtl *__restrict__ ctl, const float *x, Q8W emb,
                                                      const float *embf, float *x_store, const float *norm_w, float eps,
                                                      float *xn, uint8_t *xk) {
    __shared__ NormScratch ns;
    __shared__ float s_x[shp::E];
    __shared__ float s_n[NL][shp::E];
    if (!ctl->active) return;
    const int nl = ctl->nl;
#pragma unroll
    for (int l = 0; l < NL; l++) {
        float v[EPT];
        if (l < nl) {
            if (embf) load8(embf + (int64_t)l * shp::E, v);
            else if (emb.q) embed8(emb, ctl->tok[l], v);
            else load8(x + (int64_t)l * shp::E, v);
            if (x_store && (embf || emb.q)) store8(x_store + (int64_t)l * shp::E, v);
            store8(s_x, v);   // the replay source of the exact-sum fallback
            __syncthreads();
            rms_norm_mul_e(v, s_x, norm_w, eps, ns);
            __syncthreads();
        } else {
#pragma unroll
            for (int i = 0; i < EPT; i++) v[i] = 0.0f;
        }
        store8(xn + (int64_t)l * shp::E, v);
        store8(s_n[l], v);
    }
    q8K_rows_lds<NL>(s_n, xk);   // the GEMV's activation: q8_K blocks of xn
}

}  // namespace kq

int launch_ba_f32(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const float *x, const ActBufs &b, hipStream_t st) {
    hipLaunchKernelGGL(kq::ba_f32_kernel<OXE_NL>, dim3(2 * shp::NVH / 16), dim3(256), 0, st, ctl, x, w.attn_norm, m.eps,
                       (const float *)w.beta_r.w, (const float *)w.alpha_r.w, b.proj);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// q8_K blocks of nblk consecutive 256-value blocks of x (every lane of a [NL][n] buffer at once)
static void quant_k(const float *x, int64_t nblk, uint8_t *y, hipStream_t st) {
    hipLaunchKernelGGL(kq::quant_q8_K_kernel, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0, st, x, nblk, y);
}

int launch_kq_moe(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st) {
    (void)m;
    const bool exp_gu = w.exp_gate_r.type != 8, sh_gu = w.sh_gate_r.type != 8;
    if (exp_gu || sh_gu) quant_k(b.xn, (int64_t)OXE_NL * shp::E / kq::QK, b.xk, st);
    if (!exp_gu) launch_experts(ctl, w, b, st);
    if (exp_gu || sh_gu) {
        kq::KqGuArgs a{};
        a.xk = b.xk;
        a.gate = w.exp_gate_r;
        a.up = w.exp_up_r;
        a.sh_gate = w.sh_gate_r;
        a.sh_up = w.sh_up_r;
        a.uni = b.uni;
        a.route_ids = b.route_ids;
        a.hexp = b.hexp;
        a.hsh = b.hsh;
        a.do_exp = exp_gu;
        a.do_sh = sh_gu;
        a.stats = b.counters + CNT_UNI_SUM;
        hipLaunchKernelGGL(kq::kq_gu_kernel<OXE_NL>, dim3((OXE_MAX_UNION + 1) * (shp::FF / kq::GU_R)), dim3(256), 0, st, ctl, a);
    }
    {
        // h of the routed slots and of the shared expert, for whichever down matrices are K-quants
        const int64_t ne = w.exp_down_r.type != 8 ? (int64_t)OXE_NL * shp::KUSED * shp::FF / kq::QK : 0;
        const int64_t ns = w.sh_down_r.type != 8 ? (int64_t)OXE_NL * shp::FFSH / kq::QK : 0;
        if (ne + ns > 0)
            hipLaunchKernelGGL(kq::quant_q8_K_two_kernel, dim3((unsigned)((ne + ns + 3) / 4)), dim3(256), 0, st, b.hexp, ne,
                               b.hk, b.hsh, ns, b.hshk);
    }
    kq::KqDownArgs d{};
    d.uni = b.uni;
    d.route_ids = b.route_ids;
    d.route_w = b.route_w;
    d.sh_gate = b.sh_gate;
    d.hexp = b.hexp;
    d.hsh = b.hsh;
    d.hk = b.hk;
    d.hshk = b.hshk;
    d.exp_down = w.exp_down;
    d.shexp_down = w.shexp_down;
    d.exp_down_r = w.exp_down_r;
    d.sh_down_r = w.sh_down_r;
    d.x1 = b.x1;
    d.x2 = b.x2;
    d.amax_key = b.amax_key;
    hipLaunchKernelGGL(kq::kq_down_kernel<OXE_NL>, dim3(shp::E / kq::DN_R), dim3(256), 0, st, ctl, d);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_kq_head(const RunCtl *ctl, const ModelRt &m, const float *norm_w, const ActBufs &b, hipStream_t st,
                   const RawW *w, const uint32_t *ids) {
    hipLaunchKernelGGL(kq::kq_head_norm_kernel<OXE_NL>, dim3(1), dim3(256), 0, st, ctl, b.x2, norm_w, m.eps, b.hid, b.xn,
                       b.xk);
    const int nb = shp::E / kq::QK;
    const RawW &o = w ? *w : m.output_r;
    int rc;
    switch (o.type) {
        case 11: rc = kq::vl_gemv_type<3>(o.w, nb, o.rows, b.xk, OXE_NL, b.logits, st); break;
        case 12: rc = kq::vl_gemv_type<4>(o.w, nb, o.rows, b.xk, OXE_NL, b.logits, st); break;
        case 13: rc = kq::vl_gemv_type<5>(o.w, nb, o.rows, b.xk, OXE_NL, b.logits, st); break;
        default: rc = kq::vl_gemv_type<6>(o.w, nb, o.rows, b.xk, OXE_NL, b.logits, st); break;
    }
    if (rc != 1) return -2;
    hipLaunchKernelGGL(kq::kq_argmax_kernel<OXE_NL>, dim3(OXE_NL), dim3(1024), 0, st, ctl, b.logits, o.rows, b.amax_key, ids);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// the lane GEMV over a matrix of ggml type 11..14 (nb blocks per row), s[l * rows + r]; 1: done
static int vl_gemv_any(int type, const kq::KqSegs &S, int nb, const uint8_t *y, hipStream_t st, const kq::KqEpi &epi) {
    switch (type) {
        case 11: return kq::vl_gemv_segs<3>(S, nb, y, OXE_NL, nullptr, st, epi);
        case 12: return kq::vl_gemv_segs<4>(S, nb, y, OXE_NL, nullptr, st, epi);
        case 13: return kq::vl_gemv_segs<5>(S, nb, y, OXE_NL, nullptr, st, epi);
        case 14: return kq::vl_gemv_segs<6>(S, nb, y, OXE_NL, nullptr, st, epi);
        default: return 0;
    }
}

int launch_kq_embed(const RunCtl *ctl, const ModelRt &m, float *out, hipStream_t st) {
    const RawW &e = m.tok_embd_r;
    if (e.type < 11 || e.type > 14) return -1;
    hipLaunchKernelGGL(kq::kq_embed_kernel<OXE_NL>, dim3(OXE_NL), dim3(256), 0, st, ctl, e.w, e.type, raw_row_bytes(e), out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_kq_proj(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const float *x, bool embed, float *x_store,
                   const ActBufs &b, hipStream_t st, int64_t row_begin) {
    using namespace shp;
    const bool kemb = embed && m.tok_embd_r.type != 8;
    hipLaunchKernelGGL(kq::kq_norm_kernel<OXE_NL>, dim3(1), dim3(256), 0, st, ctl, x, embed && !kemb ? m.tok_embd : Q8W{},
                       kemb ? b.emb : nullptr, x_store, w.attn_norm, m.eps, b.xn, b.xk);
    struct Part {
        const RawW *r;
        int64_t off;
        bool v;
    };
    const Part dn[4] = {{&w.qkv_r, 0, false}, {&w.z_r, DN_Z, false}, {&w.beta_r, DN_BETA, false}, {&w.alpha_r, DN_ALPHA, false}};
    const Part at[3] = {{&w.q_r, 0, false}, {&w.k_r, AT_K, false}, {&w.v_r, AT_V, true}};
    const Part *ps = w.att ? at : dn;
    const int np = w.att ? 3 : 4;
    kq::KqEpi epi;       // the rows straight into the run's projection buffer (V rows also to V^T)
    epi.ctl = ctl;
    epi.dst = b.proj;
    epi.ld = DN_ROWS;
    epi.vt = w.att ? m.vcache + (int64_t)w.index * NKV * HD * m.n_ctx : nullptr;
    epi.vt_ld = m.n_ctx;
    // consecutive parts of one K-quant type share a launch
    kq::KqSegs S;
    int ty = 0;
    auto flush = [&]() {
        const int rc = S.n ? vl_gemv_any(ty, S, (int)(E / kq::QK), b.xk, st, epi) : 1;
        S = kq::KqSegs{};
        return rc == 1;
    };
    for (int i = 0; i < np; i++) {
        const RawW &r = *ps[i].r;
        if (ps[i].off < row_begin || r.type < 11 || r.type > 14) continue;   // F32 beta / alpha: launch_ba_f32
        if (S.n && r.type != ty && !flush()) return -2;
        ty = r.type;
        const int j = S.n++;
        S.w[j] = (const uint8_t *)r.w;
        S.nr[j] = r.rows;
        S.g0[j] = S.ngroups;
        S.off[j] = ps[i].off;
        if (ps[i].v) S.vseg = j;
        S.ngroups += (r.rows + kq::GR - 1) / kq::GR;
    }
    if (!flush()) return -2;
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int launch_kq_out(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const float *x, const ActBufs &b, hipStream_t st) {
    (void)m;
    using namespace shp;
    const RawW &r = w.out_r;
    quant_k(b.o32, (int64_t)OXE_NL * MIX_W / kq::QK, b.ok, st);
    kq::KqEpi epi;       // mixer_out's residual (engine.rs:2573-2609) at the store: x1 = out + x
    epi.ctl = ctl;
    epi.dst = b.x1;
    epi.ld = E;
    epi.resid = x;
    if (vl_gemv_any(r.type, kq::one_seg((const uint8_t *)r.w, E), (int)(MIX_W / kq::QK), b.ok, st, epi) != 1) return -2;
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace oxe

extern "C" {

int oxe_hip_quantize_row_q8_K(const float *x, int64_t k, int64_t nrows, void *y, void *stream) {
    if (!x || !y || k <= 0 || k % oxe::kq::QK != 0 || nrows <= 0) return -1;
    if (((uintptr_t)x & 15) != 0 || ((uintptr_t)y & 3) != 0) return -1;
    const int64_t nblk = k / oxe::kq::QK * nrows;
    hipLaunchKernelGGL(oxe::kq::quant_q8_K_kernel, dim3((unsigned)((nblk + 3) / 4)), dim3(256), 0,
                       (hipStream_t)stream, x, nblk, (uint8_t *)y);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int oxe_hip_vl_gemv(int type, int64_t k, int64_t nr, int nl, const void *w, const void *y, float *s, void *stream) {
    using namespace oxe::kq;
    if (nl < 1 || nl > MAX_LANES || nr <= 0 || k <= 0 || k % QK != 0 || k > 8192 || !w || !y || !s) return 0;
    if (((uintptr_t)w & 15) != 0 || ((uintptr_t)y & 3) != 0) return 0;
    const int nb = (int)(k / QK);
    const hipStream_t st = (hipStream_t)stream;
    const uint8_t *wb = (const uint8_t *)w, *yb = (const uint8_t *)y;
    switch (type) {
        case 4: return vl_gemv_type<4>(wb, nb, nr, yb, nl, s, st);
        case 5: return vl_gemv_type<5>(wb, nb, nr, yb, nl, s, st);
        // 110- and 210-byte blocks: rows of an even block count keep every 4-row group 16-byte aligned
        case 3: return nb % 2 ? 0 : vl_gemv_type<3>(wb, nb, nr, yb, nl, s, st);
        case 6: return nb % 2 ? 0 : vl_gemv_type<6>(wb, nb, nr, yb, nl, s, st);
        default: return 0;
    }
}

}  // extern "C"
