// K-quant kernels: the q8_K activation quantizer (quantize_row_q8_K) and the lane GEMVs over
// Q3_K / Q4_K / Q5_K / Q6_K weights (the reference's oxe_vl_gemv, crates/kernels-sys/csrc/
// oxe_vl.inc:78-107, types 3..6), bit for bit per (lane, row).
//
// Weights are the GGUF file's ggml blocks (no repack: the reference's 8-row interleave only serves
// its NEON SMMLA tiles). A workgroup of 256 threads owns rpw rows and walks k in chunks of kch
// blocks: the chunk's weight bytes and the lanes' q8_K blocks are staged in LDS with coalesced
// dword loads; thread (row, unit) forms the exact integers of one half block (128 weights) for
// every lane with v_dot4_i32_i8 (codes repacked 4 per dword); then one thread per (row, lane)
// runs the reference's float chain over the chunk's blocks in order. Integer parts are exact, so
// only the chain (the order and fusion the reference documents per type) fixes the bits.
#include "oxe_common.h"

namespace oxe {
namespace kq {

constexpr int QK = 256;
constexpr int Q8K_BYTES = 292;   // block_q8_K: float d, int8 qs[256], int16 bsums[16]
constexpr int Q8K_QS = 4, Q8K_BS = 260;
constexpr int NT = 256;          // threads per workgroup
constexpr int KCH = 8;           // blocks per chunk (at most)
constexpr int RES = 6;           // ints per (unit, lane)
constexpr int MAX_LANES = 4;

template <int TY> struct BT;
template <> struct BT<3> { static constexpr int B = 110; };
template <> struct BT<4> { static constexpr int B = 144; };
template <> struct BT<5> { static constexpr int B = 176; };
template <> struct BT<6> { static constexpr int B = 210; };

OXE_DEV uint32_t ld32(const uint8_t *p) { return *(const uint32_t *)p; }
OXE_DEV uint16_t ld16(const uint8_t *p) { return *(const uint16_t *)p; }
// 4 bytes at a 2-byte aligned LDS address (Q3_K / Q6_K blocks are 110 / 210 bytes, so every other
// block of a row starts 2 bytes off a dword boundary)
OXE_DEV uint32_t ld32h(const uint8_t *p) { return (uint32_t)ld16(p) | (uint32_t)ld16(p + 2) << 16; }
OXE_DEV int bsum16(const uint8_t *yb, int i) { return (int)*(const int16_t *)(yb + Q8K_BS + 2 * i); }

// ---- quantize_row_q8_K_ref (vendor/ggml-subset/generated/quants_base.c:14-48) --------------------
// One wave per 256-value block; thread t holds values 4 t .. 4 t + 3. The block maximum is the
// first value of largest magnitude (the reference's strict > scan); iscale = -127 / max (f32
// division), codes = nearest_int(iscale * x) (the float add of 1.5 * 2^23: round half to even),
// clamped above at 127; bsums = sums of 16 codes; d = 1 / iscale. An all-zero block gets d = 0 and
// zero codes and sums.
__global__ __launch_bounds__(256) void quant_q8_K_kernel(const float *__restrict__ x, int64_t nblk,
                                                         uint8_t *__restrict__ y) {
    const int lane = threadIdx.x & 63;
    const int64_t b = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (b >= nblk) return;
    const float4 v4 = *(const float4 *)(x + b * QK + 4 * lane);
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
    uint8_t *yb = y + b * Q8K_BYTES;
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

// ---- integers of one half block (unit h: weights 128 h .. 128 h + 127) for one lane -------------

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
template <int TY>
OXE_DEV void unit_k45(const uint8_t *wb, const uint8_t *yb, int h, int *out) {
    const uint8_t *sc = wb + 4;
    const uint8_t *qs = wb + (TY == 4 ? 16 : 48);
    const uint8_t *qh = wb + 16;
    const uint8_t *yq = yb + Q8K_QS;
    int bias4 = 0;
    for (int gg = 0; gg < 2; gg++) {
        const int g = 2 * h + gg;
        int lo = 0, hi = 0;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint32_t w = ld32(qs + 32 * g + 4 * i);
            uint32_t cl = w & 0x0F0F0F0Fu, ch = (w >> 4) & 0x0F0F0F0Fu;
            if (TY == 5) {
                const uint32_t hb = ld32(qh + 4 * i);
                cl |= ((hb >> (2 * g)) & 0x01010101u) << 4;
                ch |= ((hb >> (2 * g + 1)) & 0x01010101u) << 4;
            }
            lo = dot4(cl, ld32(yq + 64 * g + 4 * i), lo);
            hi = dot4(ch, ld32(yq + 64 * g + 32 + 4 * i), hi);
        }
        int s_lo, m_lo, s_hi, m_hi;
        scale_min_k4(2 * g, sc, s_lo, m_lo);
        scale_min_k4(2 * g + 1, sc, s_hi, m_hi);
        out[2 * gg] = s_lo * lo;
        out[2 * gg + 1] = s_hi * hi;
        const int bias = m_lo * (bsum16(yb, 4 * g) + bsum16(yb, 4 * g + 1)) +
                         m_hi * (bsum16(yb, 4 * g + 2) + bsum16(yb, 4 * g + 3));
        if (TY == 5) out[4 + gg] = bias;
        bias4 += bias;
    }
    if (TY == 4) out[4] = bias4;
}

// Q6_K: the unit's part of I = sum_i scale_i * (16 codes - 32) . q8 (the -32 through the q8 sums)
OXE_DEV void unit_q6(const uint8_t *wb, const uint8_t *yb, int n, int *out) {
    const uint8_t *ql = wb + 64 * n, *qh = wb + 128 + 32 * n;
    const int8_t *sc = (const int8_t *)(wb + 192);
    const uint8_t *yq = yb + Q8K_QS + 128 * n;
    int d[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t a = ld32h(ql + 4 * i), a2 = ld32h(ql + 32 + 4 * i), hb = ld32h(qh + 4 * i);
        const uint32_t c0 = (a & 0x0F0F0F0Fu) | ((hb & 0x03030303u) << 4);
        const uint32_t c1 = (a2 & 0x0F0F0F0Fu) | (((hb >> 2) & 0x03030303u) << 4);
        const uint32_t c2 = ((a >> 4) & 0x0F0F0F0Fu) | (((hb >> 4) & 0x03030303u) << 4);
        const uint32_t c3 = ((a2 >> 4) & 0x0F0F0F0Fu) | (((hb >> 6) & 0x03030303u) << 4);
        const int s = i >> 2;   // which 16 of the 32
        d[0 + s] = dot4(c0, ld32(yq + 4 * i), d[0 + s]);
        d[2 + s] = dot4(c1, ld32(yq + 32 + 4 * i), d[2 + s]);
        d[4 + s] = dot4(c2, ld32(yq + 64 + 4 * i), d[4 + s]);
        d[6 + s] = dot4(c3, ld32(yq + 96 + 4 * i), d[6 + s]);
    }
    int I = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) I += (int)sc[8 * n + i] * (d[i] - 32 * bsum16(yb, 8 * n + i));
    out[0] = I;
}

// q3k_raw_scales (repack_subset.cpp:575-587): raw 6-bit scale i of a Q3_K block
OXE_DEV int q3_raw(const uint8_t *s12, int i) {
    const int lo = i < 8 ? (s12[i] & 15) : (s12[i - 8] >> 4);
    const int hi = (s12[8 + (i & 3)] >> (2 * (i >> 2))) & 3;
    return lo | hi << 4;
}

// Q3_K: the unit's part of isum = sum_i (raw_i - 32) * dot16_i, codes (low 2 bits | hmask bit << 2) - 4
OXE_DEV void unit_q3(const uint8_t *wb, const uint8_t *yb, int n, int *out) {
    const uint8_t *hm = wb, *qs = wb + 32 + 32 * n;
    const uint8_t *yq = yb + Q8K_QS + 128 * n;
    int d[8] = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
    for (int i = 0; i < 8; i++) {
        const uint32_t qw = ld32h(qs + 4 * i), hw = ld32h(hm + 4 * i);
        const int half = i >> 2;
#pragma unroll
        for (int s = 0; s < 4; s++) {
            const uint32_t c = ((qw >> (2 * s)) & 0x03030303u) | (((hw >> (4 * n + s)) & 0x01010101u) << 2);
            d[2 * s + half] = dot4(c, ld32(yq + 32 * s + 4 * i), d[2 * s + half]);
        }
    }
    int I = 0;
#pragma unroll
    for (int i = 0; i < 8; i++) I += (q3_raw(wb + 96, 8 * n + i) - 32) * (d[i] - 4 * bsum16(yb, 8 * n + i));
    out[0] = I;
}

template <int TY>
OXE_DEV void unit(const uint8_t *wb, const uint8_t *yb, int h, int *out) {
    if (TY == 4 || TY == 5) unit_k45<TY>(wb, yb, h, out);
    else if (TY == 6) unit_q6(wb, yb, h, out);
    else unit_q3(wb, yb, h, out);
}

// ---- the reference's float chain over one block (units r0: weights 0..127, r1: 128..255) ---------
template <int TY>
OXE_DEV float chain(float acc, const uint8_t *wb, const uint8_t *yb, const int *r0, const int *r1) {
    const float dx = *(const float *)yb;
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
// s[l * nr + r] = W[r] . y[l]; w: nr rows of nb blocks; y: nl lanes of nb q8_K blocks. kch blocks
// per chunk (a power of two; every chunk's byte count and offset a multiple of 4), rpw = NT / (2 kch)
// rows per workgroup, thread (ri, u): row ri, unit u = half u % 2 of the chunk's block u / 2.
template <int TY>
__global__ __launch_bounds__(NT) void vl_gemv_kernel(const uint8_t *__restrict__ w, int nb, int64_t nr,
                                                     const uint8_t *__restrict__ y, int nl, float *__restrict__ s,
                                                     int kch) {
    constexpr int BB = BT<TY>::B;
    extern __shared__ __align__(16) uint8_t lds[];
    const int U = 2 * kch, rpw = NT / U;
    uint8_t *wl = lds;                                         // [rpw][kch * BB]
    uint8_t *yl = lds + (rpw * kch * BB + 15) / 16 * 16;       // [nl][kch][292]
    int *res = (int *)(yl + (nl * kch * Q8K_BYTES + 15) / 16 * 16);   // [NT][MAX_LANES][RES]
    const int t = threadIdx.x, ri = t / U, u = t % U;
    const int64_t row0 = (int64_t)blockIdx.x * rpw, r = row0 + ri;
    const int64_t row_bytes = (int64_t)nb * BB;
    float acc[2] = {0.0f, 0.0f};
    for (int b0 = 0; b0 < nb; b0 += kch) {
        const int kc = min(kch, nb - b0);
        const int seg = kc * BB / 4;
        for (int i = t; i < rpw * seg; i += NT) {
            const int rr = i / seg, o = i - rr * seg;
            if (row0 + rr < nr)
                ((uint32_t *)(wl + rr * kch * BB))[o] = ((const uint32_t *)(w + (row0 + rr) * row_bytes + (int64_t)b0 * BB))[o];
        }
        const int yseg = kc * Q8K_BYTES / 4;
        for (int i = t; i < nl * yseg; i += NT) {
            const int l = i / yseg, o = i - l * yseg;
            ((uint32_t *)(yl + l * kch * Q8K_BYTES))[o] = ((const uint32_t *)(y + ((int64_t)l * nb + b0) * Q8K_BYTES))[o];
        }
        __syncthreads();
        const int bi = u >> 1, h = u & 1;
        if (bi < kc && ri < rpw && r < nr)
            for (int l = 0; l < nl; l++)
                unit<TY>(wl + ri * kch * BB + bi * BB, yl + (l * kch + bi) * Q8K_BYTES, h, res + (t * MAX_LANES + l) * RES);
        __syncthreads();
        if (ri < rpw && r < nr)
            for (int j = 0; j < 2; j++) {
                const int l = u + j * U;
                if (l >= nl) continue;
                for (int b = 0; b < kc; b++) {
                    const int *r0 = res + ((ri * U + 2 * b) * MAX_LANES + l) * RES;
                    const int *r1 = res + ((ri * U + 2 * b + 1) * MAX_LANES + l) * RES;
                    acc[j] = chain<TY>(acc[j], wl + ri * kch * BB + b * BB, yl + (l * kch + b) * Q8K_BYTES, r0, r1);
                }
            }
        __syncthreads();
    }
    if (ri < rpw && r < nr)
        for (int j = 0; j < 2; j++) {
            const int l = u + j * U;
            if (l < nl) s[(int64_t)l * nr + r] = acc[j];
        }
}

size_t vl_gemv_lds(int bb, int kch, int nl) {
    const int rpw = NT / (2 * kch);
    return (size_t)(rpw * kch * bb + 15) / 16 * 16 + (size_t)(nl * kch * Q8K_BYTES + 15) / 16 * 16 +
           (size_t)NT * MAX_LANES * RES * 4;
}

template <int TY>
int vl_gemv_launch(const uint8_t *w, int nb, int64_t nr, const uint8_t *y, int nl, float *s, hipStream_t st) {
    constexpr int BB = BT<TY>::B;
    int kch = KCH;   // a power of two (so 2 kch divides the workgroup), at most nb
    while (kch > nb) kch >>= 1;
    const int rpw = NT / (2 * kch);
    const int64_t grid = (nr + rpw - 1) / rpw;
    if (grid > 0x7fffffff) return 0;
    const size_t lds = vl_gemv_lds(BB, kch, nl);
    hipLaunchKernelGGL(vl_gemv_kernel<TY>, dim3((unsigned)grid), dim3(NT), lds, st, w, nb, nr, y, nl, s, kch);
    return hipGetLastError() == hipSuccess ? 1 : -2;
}

}  // namespace kq
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
    if (nl < 1 || nl > MAX_LANES || nr <= 0 || k <= 0 || k % QK != 0 || k > 65536 || !w || !y || !s) return 0;
    if (((uintptr_t)w & 3) != 0 || ((uintptr_t)y & 3) != 0) return 0;
    const int nb = (int)(k / QK);
    const hipStream_t st = (hipStream_t)stream;
    const uint8_t *wb = (const uint8_t *)w, *yb = (const uint8_t *)y;
    switch (type) {
        case 4: return vl_gemv_launch<4>(wb, nb, nr, yb, nl, s, st);
        case 5: return vl_gemv_launch<5>(wb, nb, nr, yb, nl, s, st);
        // 110- and 210-byte blocks: dword staging needs an even block count
        case 3: return nb % 2 ? 0 : vl_gemv_launch<3>(wb, nb, nr, yb, nl, s, st);
        case 6: return nb % 2 ? 0 : vl_gemv_launch<6>(wb, nb, nr, yb, nl, s, st);
        default: return 0;
    }
}

}  // extern "C"
