// On-device generation of the synthetic model (include/oxe_model.h): every weight is a pure
// function of (seed, tensor uid, element index), so the 36 GB model is built in HBM in
// milliseconds and the host oracle regenerates any slice of it independently.
#include "oxe_common.h"
#include "oxe_kernels.h"

#include <algorithm>

namespace oxe {

// Codes of dst rows [0, rows) x k: dst row r holds source row src_row(r) of expert `expert` of the
// tensor (flat index ((expert * src_rows + src_row) * k + i)). `il` interleaves two tensors per
// 16-row tile (8 rows of kind A then 8 rows of kind B) as the engine's gate/up layout: il == 1 ->
// dst row r takes tile t = r / 16, j = r % 16, source row t * 8 + (j % 8) of kind (j < 8 ? A : B).
struct SynthArgs {
    uint64_t key_a, skey_a, key_b, skey_b;
    oxe_synth_param p;
    int64_t rows, k, src_rows, expert;
    int il;
    int8_t *q;
    uint16_t *d;
};

OXE_DEV void synth_src(const SynthArgs &a, int64_t r, uint64_t *key, uint64_t *skey, int64_t *srow) {
    if (a.il) {
        const int64_t t = r / 16, j = r % 16;
        *srow = t * 8 + (j % 8);
        *key = j < 8 ? a.key_a : a.key_b;
        *skey = j < 8 ? a.skey_a : a.skey_b;
    } else {
        *srow = r;
        *key = a.key_a;
        *skey = a.skey_a;
    }
}

__global__ void synth_q8_kernel(SynthArgs a) {
    // one thread per 32-code block: 32 codes + its fp16 scale
    const int64_t nb = a.rows * (a.k / 32);
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = b / (a.k / 32), kb = b % (a.k / 32);
        uint64_t key, skey;
        int64_t srow;
        synth_src(a, r, &key, &skey, &srow);
        const uint64_t base = ((uint64_t)a.expert * a.src_rows + srow) * a.k + kb * 32;
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; i++) {
            const uint64_t rr = oxe_rng(key, (base >> 2) + i);  // base is a multiple of 32
            uint32_t u = 0;
#pragma unroll
            for (int j = 0; j < 4; j++) {
                const uint32_t s = (uint32_t)((rr >> (16 * j)) & 0xffffu);
                const int32_t c = (int32_t)((s * 255u) >> 16) - 127;
                u |= ((uint32_t)(c & 0xff)) << (8 * j);
            }
            w[i] = u;
        }
        uint4 *dst = (uint4 *)(a.q + r * a.k + kb * 32);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
        a.d[b] = oxe_synth_scale(skey, base / 32, a.p);
    }
}

__global__ void synth_f32_kernel(uint64_t key, int kind, int64_t n, float *out) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
        out[i] = oxe_synth_f32(key, (uint64_t)i, kind);
}

int synth_q8(uint64_t seed, int layer, int kind_a, int kind_b, int64_t rows, int64_t k, int64_t src_rows,
             int64_t expert, int8_t *q, uint16_t *d, hipStream_t st) {
    SynthArgs a;
    a.key_a = oxe_tensor_key(seed, layer, kind_a);
    a.skey_a = oxe_tensor_key(seed, layer, kind_a + OXE_T_SCALE_OFFSET);
    a.key_b = kind_b >= 0 ? oxe_tensor_key(seed, layer, kind_b) : 0;
    a.skey_b = kind_b >= 0 ? oxe_tensor_key(seed, layer, kind_b + OXE_T_SCALE_OFFSET) : 0;
    a.p = oxe_synth_param_of(kind_a);
    a.rows = rows;
    a.k = k;
    a.src_rows = src_rows;
    a.expert = expert;
    a.il = kind_b >= 0;
    a.q = q;
    a.d = d;
    const int64_t nb = rows * (k / 32);
    const unsigned grid = (unsigned)std::min<int64_t>((nb + 255) / 256, 65536);
    hipLaunchKernelGGL(synth_q8_kernel, dim3(grid), dim3(256), 0, st, a);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

// Synthetic K-quant tensors (the oracle's oxo_synth_kq, oracle/kquants.cpp, so a typed engine built
// on the device holds the oracle's typed weights): block i of tensor (seed, layer, kind), flat over
// [expert][row][k / 256], is the first bb bytes of the words oxe_rng(key, 32 i + j), j < 32, with
// its fp16 fields from the scale key: Q4_K / Q5_K d = fp16(lo + u (hi - lo)) in [0.0005, 0.004),
// dmin = fp16(d * mean code); Q6_K d in [0.00005, 0.0003); Q3_K d in [0.0005, 0.004). One thread
// per block.
__global__ void synth_kq_kernel(uint64_t key, uint64_t skey, int type, int bb, int64_t nb, uint8_t *out) {
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        uint8_t *blk = out + b * bb;
        for (int j = 0; j < 32; j++) {
            const uint64_t w = oxe_rng(key, 32 * (uint64_t)b + (uint64_t)j);
            for (int i = 0; i < 8 && 8 * j + i < bb; i++) blk[8 * j + i] = (uint8_t)(w >> (8 * i));
        }
        auto f16_in = [&](uint64_t i, float lo, float hi) {
            const float u = oxe_synth_unit(skey, i);
            const float t = u * (hi - lo);
            return oxe_f32_to_f16_rne(lo + t);
        };
        auto put16 = [&](int off, uint16_t h) {
            blk[off] = (uint8_t)h;
            blk[off + 1] = (uint8_t)(h >> 8);
        };
        if (type == 12 || type == 13) {
            const uint16_t h0 = f16_in(2 * (uint64_t)b, 0.0005f, 0.004f);
            put16(0, h0);
            put16(2, oxe_f32_to_f16_rne(h2f(h0) * (type == 12 ? 7.5f : 15.5f)));
        } else if (type == 14) {
            put16(208, f16_in(2 * (uint64_t)b, 0.00005f, 0.0003f));
        } else {
            put16(108, f16_in(2 * (uint64_t)b, 0.0005f, 0.004f));
        }
    }
}

// rows x k of a matrix in another type than Q8_0 (rows counts every expert of an expert tensor):
// K-quant blocks (ggml type 11..14) or F32 values (0)
int synth_raw(uint64_t seed, int layer, int kind, int type, int64_t rows, int64_t k, void *out, hipStream_t st) {
    if (type == 0) return synth_f32(seed, layer, kind, rows * k, (float *)out, st);
    const int bb = type == 11 ? 110 : type == 12 ? 144 : type == 13 ? 176 : type == 14 ? 210 : 0;
    if (!bb || k % 256) return -1;
    const int64_t nb = rows * (k / 256);
    const unsigned grid = (unsigned)std::min<int64_t>((nb + 255) / 256, 65536);
    hipLaunchKernelGGL(synth_kq_kernel, dim3(grid), dim3(256), 0, st, oxe_tensor_key(seed, layer, kind),
                       oxe_tensor_key(seed, layer, kind + OXE_T_SCALE_OFFSET), type, bb, nb, (uint8_t *)out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int synth_f32(uint64_t seed, int layer, int kind, int64_t n, float *out, hipStream_t st) {
    const unsigned grid = (unsigned)std::min<int64_t>((n + 255) / 256, 4096);
    hipLaunchKernelGGL(synth_f32_kernel, dim3(grid), dim3(256), 0, st, oxe_tensor_key(seed, layer, kind), kind, n, out);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

}  // namespace oxe
