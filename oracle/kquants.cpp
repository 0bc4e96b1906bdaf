// TEST INFRASTRUCTURE ONLY (see oxo.h): the K-quant activation quantizer and the K-quant lane GEMVs
// of the reference, restated per (lane, row) in the reference's float order.
//
// Blocks are ggml's (vendor/ggml-subset/generated/ggml-common.h:315-376): the GGUF file's bytes.
// The reference repacks them into 8-row interleaved blocks (block_q*_Kx8) for its NEON kernels;
// the repack moves bytes only, so every weight code, scale and min below is the same number.
#include <math.h>
#include <string.h>

#include "oxo.h"
#include "../include/oxe_model.h"

namespace {

constexpr int QK = 256;

struct BQ8K {   // block_q8_K, ggml-common.h:371-375
    float d;
    int8_t qs[QK];
    int16_t bsums[QK / 16];
};
static_assert(sizeof(BQ8K) == 292, "block_q8_K");

// nearest_int (vendor/ggml-subset/generated/quants_base.c:5-11): round half to even through the
// float add of 1.5 * 2^23
int nearest_int(float fval) {
    float val = fval + 12582912.f;
    int i;
    memcpy(&i, &val, sizeof(int));
    return (i & 0x007fffff) - 0x00400000;
}

// get_scale_min_k4 (quants_base.c:50-57): the 6-bit scale and min of sub-block j of a Q4_K / Q5_K block
void scale_min_k4(int j, const uint8_t *q, int *d, int *m) {
    if (j < 4) {
        *d = q[j] & 63;
        *m = q[j + 4] & 63;
    } else {
        *d = (q[j + 4] & 0xF) | ((q[j - 4] >> 6) << 4);
        *m = (q[j + 4] >> 4) | ((q[j - 0] >> 6) << 4);
    }
}

// q3k_raw_scales (repack_subset.cpp:575-587): the 16 raw 6-bit scales of a Q3_K block (scale = raw - 32)
void q3k_raw(const uint8_t *sc12, uint8_t raw[16]) {
    const uint32_t kmask1 = 0x03030303, kmask2 = 0x0f0f0f0f;
    uint32_t aux[4];
    memcpy(aux, sc12, 12);
    const uint32_t tmp = aux[2];
    aux[2] = ((aux[0] >> 4) & kmask2) | (((tmp >> 4) & kmask1) << 4);
    aux[3] = ((aux[1] >> 4) & kmask2) | (((tmp >> 6) & kmask1) << 4);
    aux[0] = (aux[0] & kmask2) | (((tmp >> 0) & kmask1) << 4);
    aux[1] = (aux[1] & kmask2) | (((tmp >> 2) & kmask1) << 4);
    memcpy(raw, aux, 16);
}

// the 32-value sums of the q8_K bsums (the reference's vpaddq_s16 of the 16-value sums)
int bsum32(const BQ8K &y, int j) { return (int16_t)(y.bsums[2 * j] + y.bsums[2 * j + 1]); }

// Q4_K (oxe_vl_q4k.inc:1-7, ggml_gemv_q4_K_8x8_q8_K dotprod branch): per 64-weight step sb,
//   acc = fma(d_w * d_x, f32(sc_lo * I_lo), acc); acc = fma(d_w * d_x, f32(sc_hi * I_hi), acc)
// and once per block acc = acc - f32(sum_j min_j * bsum32_j) * (dmin_w * d_x), unfused (vmlsq_f32).
float row_q4_K(const uint8_t *w, const BQ8K *y, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++, w += 144) {
        const float dw = oxo_f16_to_f32((uint16_t)(w[0] | w[1] << 8));
        const float dm = oxo_f16_to_f32((uint16_t)(w[2] | w[3] << 8));
        const uint8_t *sc = w + 4, *qs = w + 16;
        const float sbs = dw * y[b].d, sbm = dm * y[b].d;
        int32_t bias = 0;
        for (int sb = 0; sb < 4; sb++) {
            int s_lo, m_lo, s_hi, m_hi;
            scale_min_k4(2 * sb, sc, &s_lo, &m_lo);
            scale_min_k4(2 * sb + 1, sc, &s_hi, &m_hi);
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                lo += (qs[32 * sb + l] & 15) * y[b].qs[64 * sb + l];
                hi += (qs[32 * sb + l] >> 4) * y[b].qs[64 * sb + 32 + l];
            }
            acc = fmaf(sbs, (float)(s_lo * lo), acc);
            acc = fmaf(sbs, (float)(s_hi * hi), acc);
            bias += m_lo * bsum32(y[b], 2 * sb) + m_hi * bsum32(y[b], 2 * sb + 1);
        }
        const float t = (float)bias * sbm;
        acc = acc - t;
    }
    return acc;
}

// Q5_K (oxe_vl_q5k.inc:1-12, ggml_gemv_q5_K_8x8_q8_K): the 5th bit of a code is bit 2 sb (low
// sub-block) or 2 sb + 1 (high) of qh[l]; per step sb: fma lo, fma hi, then
// acc = acc - (dmin_w * d_x) * f32(min_lo * bsum_lo + min_hi * bsum_hi), unfused (vmlsq_f32).
float row_q5_K(const uint8_t *w, const BQ8K *y, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++, w += 176) {
        const float dw = oxo_f16_to_f32((uint16_t)(w[0] | w[1] << 8));
        const float dm = oxo_f16_to_f32((uint16_t)(w[2] | w[3] << 8));
        const uint8_t *sc = w + 4, *qh = w + 16, *qs = w + 48;
        const float sbs = dw * y[b].d, sbm = dm * y[b].d;
        for (int sb = 0; sb < 4; sb++) {
            int s_lo, m_lo, s_hi, m_hi;
            scale_min_k4(2 * sb, sc, &s_lo, &m_lo);
            scale_min_k4(2 * sb + 1, sc, &s_hi, &m_hi);
            int32_t lo = 0, hi = 0;
            for (int l = 0; l < 32; l++) {
                const int cl = (qs[32 * sb + l] & 15) | (((qh[l] >> (2 * sb)) & 1) << 4);
                const int ch = (qs[32 * sb + l] >> 4) | (((qh[l] >> (2 * sb + 1)) & 1) << 4);
                lo += cl * y[b].qs[64 * sb + l];
                hi += ch * y[b].qs[64 * sb + 32 + l];
            }
            acc = fmaf(sbs, (float)(s_lo * lo), acc);
            acc = fmaf(sbs, (float)(s_hi * hi), acc);
            const int32_t bias = m_lo * bsum32(y[b], 2 * sb) + m_hi * bsum32(y[b], 2 * sb + 1);
            const float t = sbm * (float)bias;
            acc = acc - t;
        }
    }
    return acc;
}

// Q6_K (oxe_vl_q6k.inc:1-8, ggml_gemv_q6_K_8x8_q8_K): I = sum over the 16 sub-blocks of
// scale_i * (16 codes - 32) . q8, exact int32; per block acc = acc + f32(I) * (d_w * d_x), unfused
// (vmlaq_f32, oxe_vl_q6k.inc:107-113).
float row_q6_K(const uint8_t *w, const BQ8K *y, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++, w += 210) {
        const uint8_t *ql = w, *qh = w + 128;
        const int8_t *sc = (const int8_t *)(w + 192);
        const float dw = oxo_f16_to_f32((uint16_t)(w[208] | w[209] << 8));
        const float sbs = dw * y[b].d;
        int32_t sub[16] = {0};
        for (int n = 0; n < 2; n++) {
            for (int l = 0; l < 32; l++) {
                const int e = 128 * n + l;
                const uint8_t lo = ql[64 * n + l], lo2 = ql[64 * n + 32 + l], h = qh[32 * n + l];
                const int q1 = ((lo & 15) | ((h & 3) << 4)) - 32;
                const int q2 = ((lo2 & 15) | (((h >> 2) & 3) << 4)) - 32;
                const int q3 = ((lo >> 4) | (((h >> 4) & 3) << 4)) - 32;
                const int q4 = ((lo2 >> 4) | (((h >> 6) & 3) << 4)) - 32;
                sub[(e + 0) / 16] += q1 * y[b].qs[e + 0];
                sub[(e + 32) / 16] += q2 * y[b].qs[e + 32];
                sub[(e + 64) / 16] += q3 * y[b].qs[e + 64];
                sub[(e + 96) / 16] += q4 * y[b].qs[e + 96];
            }
        }
        int32_t I = 0;
        for (int i = 0; i < 16; i++) I += sc[i] * sub[i];
        const float t = (float)I * sbs;
        acc = acc + t;
    }
    return acc;
}

// Q3_K (oxe_vl_q3k.inc:1-10, ggml_q3x8_dot_row_dotprod): code of element 128 n + 32 s + l =
// ((qs[32 n + l] >> 2 s) & 3) - (bit 4 n + s of hmask[l] ? 0 : 4); isum = sum over the 16
// sub-blocks of (raw_i - 32) * dot16_i; per block acc = fma(f32(isum), d_x * d_w, acc).
float row_q3_K(const uint8_t *w, const BQ8K *y, int nb) {
    float acc = 0.0f;
    for (int b = 0; b < nb; b++, w += 110) {
        const uint8_t *hm = w, *qs = w + 32;
        uint8_t raw[16];
        q3k_raw(w + 96, raw);
        const float dw = oxo_f16_to_f32((uint16_t)(w[108] | w[109] << 8));
        const float sbd = y[b].d * dw;
        int32_t sub[16] = {0};
        for (int n = 0; n < 2; n++)
            for (int s = 0; s < 4; s++)
                for (int l = 0; l < 32; l++) {
                    const int e = 128 * n + 32 * s + l;
                    const int q = ((qs[32 * n + l] >> (2 * s)) & 3) - (((hm[l] >> (4 * n + s)) & 1) ? 0 : 4);
                    sub[e / 16] += q * y[b].qs[e];
                }
        int32_t isum = 0;
        for (int i = 0; i < 16; i++) isum += (raw[i] - 32) * sub[i];
        acc = fmaf((float)isum, sbd, acc);
    }
    return acc;
}

}  // namespace

extern "C" {

// quantize_row_q8_K_ref (vendor/ggml-subset/generated/quants_base.c:14-48; on ARM the reference's
// quantize_row_q8_K is this function, ggml_subset.h:18-19)
void oxo_quantize_row_q8_K(const float *x, void *vy, int64_t k) {
    BQ8K *y = (BQ8K *)vy;
    for (int64_t i = 0; i < k / QK; i++, x += QK) {
        float max = 0, amax = 0;
        for (int j = 0; j < QK; ++j) {
            const float ax = fabsf(x[j]);
            if (ax > amax) {
                amax = ax;
                max = x[j];
            }
        }
        if (!amax) {
            y[i].d = 0;
            memset(y[i].qs, 0, QK);
            memset(y[i].bsums, 0, sizeof(y[i].bsums));   // the reference leaves them as they were
            continue;
        }
        const float iscale = -127.f / max;
        for (int j = 0; j < QK; ++j) {
            const float v = iscale * x[j];
            const int q = nearest_int(v);
            y[i].qs[j] = (int8_t)(q < 127 ? q : 127);
        }
        for (int j = 0; j < QK / 16; ++j) {
            int sum = 0;
            for (int ii = 0; ii < 16; ++ii) sum += y[i].qs[j * 16 + ii];
            y[i].bsums[j] = (int16_t)sum;
        }
        y[i].d = 1 / iscale;
    }
}

// dequantize_row_q{3,4,5,6}_K (vendor/ggml-subset/generated/quants_base.c:80-230), as the reference
// builds them: GCC with its default -ffp-contract=fast (crates/kernels-sys/build.rs:5-7), so the
// Q4_K / Q5_K element d1 * q - m1 is one fused multiply-subtract; Q3_K and Q6_K are products only.
// type: 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K. Returns 1, or 0 for another type.
int oxo_dequantize_row_kq(int type, const void *vx, float *y, int64_t k) {
    const uint8_t *x = (const uint8_t *)vx;
    const int64_t nb = k / QK;
    auto f16 = [](const uint8_t *p) { uint16_t h; memcpy(&h, p, 2); return oxo_f16_to_f32(h); };
    switch (type) {
        case 12: case 13: {
            const int bb = type == 12 ? 144 : 176;
            for (int64_t i = 0; i < nb; i++) {
                const uint8_t *b = x + i * bb;
                const float d = f16(b), mn = f16(b + 2);
                const uint8_t *sc = b + 4, *qh = b + 16, *q = b + (type == 12 ? 16 : 48);
                for (int j = 0, is = 0; j < QK; j += 64, is += 2) {
                    int s1, m1i, s2, m2i;
                    scale_min_k4(is, sc, &s1, &m1i);
                    scale_min_k4(is + 1, sc, &s2, &m2i);
                    const float d1 = d * (float)s1, m1 = mn * (float)m1i;
                    const float d2 = d * (float)s2, m2 = mn * (float)m2i;
                    const int u1 = 1 << (j / 32), u2 = 2 << (j / 32);
                    for (int l = 0; l < 32; ++l) {
                        const int qq = (q[l] & 0xF) + (type == 13 && (qh[l] & u1) ? 16 : 0);
                        *y++ = fmaf(d1, (float)qq, -m1);
                    }
                    for (int l = 0; l < 32; ++l) {
                        const int qq = (q[l] >> 4) + (type == 13 && (qh[l] & u2) ? 16 : 0);
                        *y++ = fmaf(d2, (float)qq, -m2);
                    }
                    q += 32;
                }
            }
            return 1;
        }
        case 14:
            for (int64_t i = 0; i < nb; i++) {
                const uint8_t *b = x + i * 210;
                const float d = f16(b + 208);
                const uint8_t *ql = b, *qh = b + 128;
                const int8_t *sc = (const int8_t *)(b + 192);
                for (int n = 0; n < QK; n += 128) {
                    for (int l = 0; l < 32; ++l) {
                        const int is = l / 16;
                        const int8_t q1 = (int8_t)((ql[l + 0] & 0xF) | (((qh[l] >> 0) & 3) << 4)) - 32;
                        const int8_t q2 = (int8_t)((ql[l + 32] & 0xF) | (((qh[l] >> 2) & 3) << 4)) - 32;
                        const int8_t q3 = (int8_t)((ql[l + 0] >> 4) | (((qh[l] >> 4) & 3) << 4)) - 32;
                        const int8_t q4 = (int8_t)((ql[l + 32] >> 4) | (((qh[l] >> 6) & 3) << 4)) - 32;
                        y[l + 0] = d * (float)sc[is + 0] * (float)q1;
                        y[l + 32] = d * (float)sc[is + 2] * (float)q2;
                        y[l + 64] = d * (float)sc[is + 4] * (float)q3;
                        y[l + 96] = d * (float)sc[is + 6] * (float)q4;
                    }
                    y += 128;
                    ql += 64;
                    qh += 32;
                    sc += 8;
                }
            }
            return 1;
        case 11:
            for (int64_t i = 0; i < nb; i++) {
                const uint8_t *b = x + i * 110;
                const float d_all = f16(b + 108);
                const uint8_t *q = b + 32, *hm = b;
                uint8_t raw[16];
                q3k_raw(b + 96, raw);
                int is = 0;
                uint8_t m = 1;
                for (int n = 0; n < QK; n += 128) {
                    int shift = 0;
                    for (int j = 0; j < 4; ++j) {
                        float dl = d_all * (float)(raw[is++] - 32);
                        for (int l = 0; l < 16; ++l) *y++ = dl * (float)((int)((q[l + 0] >> shift) & 3) - ((hm[l + 0] & m) ? 0 : 4));
                        dl = d_all * (float)(raw[is++] - 32);
                        for (int l = 0; l < 16; ++l) *y++ = dl * (float)((int)((q[l + 16] >> shift) & 3) - ((hm[l + 16] & m) ? 0 : 4));
                        shift += 2;
                        m <<= 1;
                    }
                    q += 32;
                }
            }
            return 1;
        default:
            return 0;
    }
}

// oxe_vl_gemv (crates/kernels-sys/csrc/oxe_vl.inc:78-107) per lane: s[l*nr + r] = row r of w
// (nb = k/256 blocks of the type, rows contiguous) . lane l of y (nb q8_K blocks per lane).
// type 3 Q3_K, 4 Q4_K, 5 Q5_K, 6 Q6_K. Returns 1, or 0 (nothing written) for another type.
int oxo_vl_gemv(int type, int64_t k, int64_t nr, int nl, const void *w, const void *y, float *s) {
    const int nb = (int)(k / QK);
    int bb;
    float (*row)(const uint8_t *, const BQ8K *, int);
    switch (type) {
        case 3: bb = 110; row = row_q3_K; break;
        case 4: bb = 144; row = row_q4_K; break;
        case 5: bb = 176; row = row_q5_K; break;
        case 6: bb = 210; row = row_q6_K; break;
        default: return 0;
    }
#pragma omp parallel for schedule(static) if (nr * nl > 64)
    for (int64_t r = 0; r < nr; r++)
        for (int l = 0; l < nl; l++)
            s[(int64_t)l * nr + r] = row((const uint8_t *)w + r * (int64_t)nb * bb, (const BQ8K *)y + (int64_t)l * nb, nb);
    return 1;
}

// Synthetic K-quant tensors for the tests' model files (not the reference's: its models come from
// files). Block i of tensor (seed, layer, kind), flat over [expert][row][k / 256], is filled with
// the 64-bit words oxe_rng(key, 32 i + j), then its fp16 fields are set from the scale key:
// Q4_K / Q5_K d in [0.0005, 0.004) and dmin = fp16(d * mean code) (7.5 for Q4_K, 15.5 for Q5_K, so
// the block's weights d * scale * code - dmin * min average about zero, as a trained model's do);
// Q6_K d in [0.00005, 0.0003); Q3_K d in [0.0005, 0.004). Codes, 6-bit scales and mins stay
// whatever the words hold (every bit pattern is a valid block).
// type: 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K (ggml ids). Returns the bytes written, or 0.
int64_t oxo_synth_kq(uint64_t seed, int layer, int kind, int type, int64_t expert, int64_t rows, int64_t k, uint8_t *out) {
    int bb;
    switch (type) {
        case 11: bb = 110; break;
        case 12: bb = 144; break;
        case 13: bb = 176; break;
        case 14: bb = 210; break;
        default: return 0;
    }
    if (k % QK != 0 || rows < 0 || expert < 0) return 0;
    const int64_t nb = rows * (k / QK);
    const uint64_t key = oxe_tensor_key(seed, layer, kind);
    const uint64_t skey = oxe_tensor_key(seed, layer, kind + OXE_T_SCALE_OFFSET);
    const uint64_t base = (uint64_t)expert * (uint64_t)nb;
    auto f16_in = [&](uint64_t i, float lo, float hi) {
        const float u = oxe_synth_unit(skey, i);
        const float t = u * (hi - lo);
        return oxe_f32_to_f16_rne(lo + t);
    };
#pragma omp parallel for schedule(static) if (nb > 4096)
    for (int64_t b = 0; b < nb; b++) {
        const uint64_t bi = base + (uint64_t)b;
        uint8_t *blk = out + b * bb;
        uint8_t tmp[256];
        for (int j = 0; j < 32; j++) {
            const uint64_t w = oxe_rng(key, 32 * bi + (uint64_t)j);
            memcpy(tmp + 8 * j, &w, 8);
        }
        memcpy(blk, tmp, bb);
        uint16_t h0, h1;
        switch (type) {
            case 12: case 13: {
                h0 = f16_in(2 * bi, 0.0005f, 0.004f);
                const float dv = oxo_f16_to_f32(h0) * (type == 12 ? 7.5f : 15.5f);
                h1 = oxe_f32_to_f16_rne(dv);
                memcpy(blk, &h0, 2);
                memcpy(blk + 2, &h1, 2);
                break;
            }
            case 14:
                h0 = f16_in(2 * bi, 0.00005f, 0.0003f);
                memcpy(blk + 208, &h0, 2);
                break;
            default:
                h0 = f16_in(2 * bi, 0.0005f, 0.004f);
                memcpy(blk + 108, &h0, 2);
                break;
        }
    }
    return nb * bb;
}

}  // extern "C"
