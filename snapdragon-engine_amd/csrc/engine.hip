// The MI355X decode engine (host side): device arena allocation, synthetic weights, the run
// sequences of Engine::verify / commit / mtp_run / mtp_seed (crates/model/src/engine.rs:1991-2091)
// and the C ABI of include/oxe_amd.h. Every run is a fixed sequence of kernels on one stream; the
// run's lanes, positions and slots live in the device RunCtl, so the sequence needs no host value
// at launch time and can be captured once into a HIP graph.
#include "oxe_engine_host.h"

// ------------------------------------------------------------------------------------------------
// C ABI

using oxe::Engine;

extern "C" {

const char *oxe_last_error(void) { return oxe::g_last_error.c_str(); }

}  // extern "C"

namespace oxe {

// rows ids[0..n) of a row-major matrix (row_bytes per row, a multiple of 4) into dst, one thread per
// 4-byte word
__global__ void gather_rows_kernel(const uint8_t *src, int64_t row_bytes, const uint32_t *ids, int64_t n, uint8_t *dst) {
    const int64_t wpr = row_bytes / 4, nw = n * wpr;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nw; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t r = i / wpr, c = i % wpr;
        ((uint32_t *)dst)[i] = ((const uint32_t *)(src + (int64_t)ids[r] * row_bytes))[c];
    }
}

int Engine::set_draft_vocab(const uint32_t *ids, int n) {
    if (n < 0 || (n > 0 && !ids)) return -1;
    std::vector<uint32_t> v;
    for (int i = 0; i < n; i++)
        if (ids[i] < (uint32_t)d.n_vocab) v.push_back(ids[i]);
    if (n > 0 && v.empty()) {
        set_err("empty draft vocabulary");
        return -1;
    }
    std::sort(v.begin(), v.end());
    v.erase(std::unique(v.begin(), v.end()), v.end());
    while (!v.empty() && v.size() % 16 != 0) v.push_back(v.back());
    const int64_t rows = (int64_t)v.size();
    if (graph_exec) {   // a captured draft run holds the old head
        (void)hipGraphExecDestroy(graph_exec);
        graph_exec = nullptr;
    }
    if (rows > 0) {
        try {
            if (rows > draft_cap) {   // arrays of the largest head so far (kept until the engine goes)
                draft_ids = alloc<uint32_t>((size_t)rows);
                if (m.output_r.type != 8) {
                    draft_r = m.output_r;
                    draft_r.w = alloc<uint8_t>((size_t)(rows * raw_row_bytes(m.output_r)));
                } else {
                    draft_w.q = alloc<int8_t>((size_t)rows * E);
                    draft_w.d = alloc<uint16_t>((size_t)rows * (E / 32));
                }
                draft_cap = rows;
            }
        } catch (...) {
            return -3;
        }
        if (hipMemcpyAsync(draft_ids, v.data(), (size_t)rows * 4, hipMemcpyHostToDevice, st) != hipSuccess) return -2;
        auto gather = [&](const void *src, int64_t rb, void *dst) {
            const int64_t nw = rows * rb / 4;
            hipLaunchKernelGGL(gather_rows_kernel, dim3((unsigned)std::min<int64_t>((nw + 255) / 256, 65535)), dim3(256), 0, st,
                               (const uint8_t *)src, rb, draft_ids, rows, (uint8_t *)dst);
        };
        if (m.output_r.type != 8) {
            draft_r.rows = rows;
            gather(m.output_r.w, raw_row_bytes(m.output_r), draft_r.w);
        } else {
            draft_w.rows = rows;
            draft_w.k = E;
            gather(m.output.q, E, draft_w.q);
            gather(m.output.d, (E / 32) * 2, draft_w.d);
        }
    }
    draft_rows = rows;
    if (fused_ok) {
        fz_host[FM_DRAFT].head_w = rows > 0 ? draft_w : m.output;
        fz_host[FM_DRAFT].head_ids = rows > 0 ? draft_ids : nullptr;
        if (hipMemcpyAsync(fz_args, fz_host, sizeof(fz_host), hipMemcpyHostToDevice, st) != hipSuccess) return -2;
    }
    if (hipStreamSynchronize(st) != hipSuccess || hipGetLastError() != hipSuccess) return -2;
    return (int)rows;
}

int create_engine(const oxe_model_desc *desc, uint64_t seed, int n_ctx, bool caller, void *stream, const ModelTypes *mt,
                  oxe_engine **out) {
    // the attention kernel keeps a kv group's f16 probabilities in LDS: contexts up to 6144
    if (!desc || !out || n_ctx < 1 || n_ctx > 6144) {
        oxe::set_err("n_ctx must be in [1, 6144]");
        return -1;
    }
    if (!Engine::shape_ok(*desc)) {
        oxe::set_err("model shape differs from the kernels' qwen35moe 35B-A3B per-layer shape");
        return -1;
    }
    Engine *e = new Engine();
    try {
        e->create(*desc, seed, n_ctx, caller, (hipStream_t)stream, mt);
    } catch (const std::exception &ex) {
        oxe::set_err(ex.what());
        delete e;
        return -3;
    }
    *out = (oxe_engine *)e;
    return 0;
}
}  // namespace oxe

extern "C" {

int oxe_engine_create(const oxe_model_desc *desc, uint64_t seed, int n_ctx, oxe_engine **out) {
    return oxe::create_engine(desc, seed, n_ctx, false, nullptr, nullptr, out);
}

int oxe_engine_create_on(const oxe_model_desc *desc, uint64_t seed, int n_ctx, void *stream, oxe_engine **out) {
    return oxe::create_engine(desc, seed, n_ctx, true, stream, nullptr, out);
}

// An engine whose matrices take the types of a model file without the file: types[layer * 64 +
// kind] (layer 63: the global tensors, kinds of include/oxe_model.h) is a ggml type id, 8 (Q8_0)
// where a matrix is Q8_0. The combinations the file loader takes (k_load.hip model_types); any
// other -> -1 naming it. oxe_engine_synth_weights then fills every matrix in its type.
int oxe_engine_create_typed(const oxe_model_desc *desc, uint64_t seed, int n_ctx, const int32_t *types, oxe_engine **out) {
    if (!desc || !types || !out) return -1;
    auto kq = [](int t) { return t >= 11 && t <= 14; };
    const int nl = desc->n_layer;
    if (nl < 1 || nl > 62) {
        oxe::set_err("typed engine: layer count out of range");
        return -1;
    }
    oxe::ModelTypes mt;
    mt.layer.assign(nl + 1, oxe::LayerTypes{});
    std::string bad;
    auto ty = [&](int l, int k) { return (int)types[l * 64 + k]; };
    for (int l = 0; l <= nl && bad.empty(); l++) {
        const bool att = l == nl || ((l + 1) % desc->full_attention_interval == 0);
        oxe::LayerTypes &t = mt.layer[l];
        const std::string where = "layer " + std::to_string(l) + ": ";
        for (int k = 0; k < 64; k++) {
            const int v = ty(l, k);
            const bool q8 = v == 8;
            switch (k) {
                case OXE_T_GATE_EXPS: case OXE_T_UP_EXPS: case OXE_T_DOWN_EXPS: case OXE_T_GATE_SHEXP:
                case OXE_T_UP_SHEXP: case OXE_T_DOWN_SHEXP: case OXE_T_DN_QKV: case OXE_T_DN_Z: case OXE_T_DN_OUT:
                case OXE_T_ATT_Q: case OXE_T_ATT_K: case OXE_T_ATT_V: case OXE_T_ATT_OUT:
                    if (!q8 && !kq(v)) bad = where + "matrix kind " + std::to_string(k) + " must be Q8_0 or a K-quant";
                    break;
                case OXE_T_DN_BETA: case OXE_T_DN_ALPHA:
                    if (!q8 && !kq(v) && v != 0) bad = where + "ssm_beta / ssm_alpha must be Q8_0, F32 or a K-quant";
                    break;
                default:
                    if (!q8) bad = where + "kind " + std::to_string(k) + " takes no other type";
            }
        }
        if (!bad.empty()) break;
        t.gate = ty(l, OXE_T_GATE_EXPS); t.up = ty(l, OXE_T_UP_EXPS); t.down = ty(l, OXE_T_DOWN_EXPS);
        t.sh_gate = ty(l, OXE_T_GATE_SHEXP); t.sh_up = ty(l, OXE_T_UP_SHEXP); t.sh_down = ty(l, OXE_T_DOWN_SHEXP);
        if ((t.gate == 8) != (t.up == 8) || (t.sh_gate == 8) != (t.sh_up == 8))
            bad = where + "gate and up are both Q8_0 or both K-quants";
        if (!att) {
            t.qkv = ty(l, OXE_T_DN_QKV); t.z = ty(l, OXE_T_DN_Z); t.beta = ty(l, OXE_T_DN_BETA); t.alpha = ty(l, OXE_T_DN_ALPHA);
            t.out = ty(l, OXE_T_DN_OUT);
            const bool f32ba = t.beta == 0 && t.alpha == 0, q8ba = t.beta == 8 && t.alpha == 8;
            const bool kba = kq(t.beta) && kq(t.alpha);
            if (t.qkv == 8 ? !(t.z == 8 && (q8ba || f32ba)) : !(kq(t.z) && (f32ba || kba)))
                bad = where + "the delta-net projection parts mix Q8_0 with other types";
        } else {
            t.q = ty(l, OXE_T_ATT_Q); t.k = ty(l, OXE_T_ATT_K); t.v = ty(l, OXE_T_ATT_V); t.out = ty(l, OXE_T_ATT_OUT);
            if (!((t.q == 8 && t.k == 8 && t.v == 8) || (kq(t.q) && kq(t.k) && kq(t.v))))
                bad = where + "the attention projection parts mix Q8_0 with K-quants";
        }
    }
    for (int k = 0; k < 64 && bad.empty(); k++) {
        const int v = ty(OXE_GLOBAL_LAYER, k);
        if (v != 8 && !((k == OXE_T_OUTPUT || k == OXE_T_TOK_EMBD) && kq(v))) bad = "global kind " + std::to_string(k) + " takes no other type";
    }
    if (!bad.empty()) {
        oxe::set_err("typed engine: " + bad);
        return -1;
    }
    mt.output = ty(OXE_GLOBAL_LAYER, OXE_T_OUTPUT);
    mt.tok_embd = ty(OXE_GLOBAL_LAYER, OXE_T_TOK_EMBD);
    return oxe::create_engine(desc, seed, n_ctx, false, nullptr, &mt, out);
}

void oxe_engine_destroy(oxe_engine *e) { delete (Engine *)e; }

int oxe_engine_synth_weights(oxe_engine *e) { return ((Engine *)e)->synth_weights(); }

int oxe_engine_verify(oxe_engine *e, const uint32_t *toks, int n, uint32_t *argmax_out) {
    return ((Engine *)e)->verify(toks, n, argmax_out);
}

// oxe_engine_verify with HIP events around every launch of kernel kind `kind` (the kinds of
// oxe_mtp_device_probe); *avg_us = their mean duration, *count = launches timed
int oxe_engine_verify_probe(oxe_engine *e, const uint32_t *toks, int n, int kind, uint32_t *argmax_out, float *avg_us,
                            int *count) {
    Engine *g = (Engine *)e;
    if (kind < 0 || !avg_us || !count) return -1;
    g->probe_kind = kind;
    g->probe_used = 0;
    const int rc = g->verify(toks, n, argmax_out);
    g->probe_kind = -1;
    if (rc) return rc;
    double tot = 0.0;
    int cnt = 0;
    for (size_t i = 0; i + 1 < g->probe_used; i += 2) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, g->probe_ev[i], g->probe_ev[i + 1]) != hipSuccess) return -2;
        tot += ms;
        cnt++;
    }
    *avg_us = cnt ? (float)(tot * 1000.0 / cnt) : 0.0f;
    *count = cnt;
    return 0;
}

int oxe_engine_commit(oxe_engine *e, int m) { return ((Engine *)e)->commit(m); }

int oxe_engine_step(oxe_engine *e, uint32_t tok, uint32_t *argmax_out) {
    Engine *g = (Engine *)e;
    const int rc = g->verify(&tok, 1, argmax_out);
    return rc ? rc : g->commit(1);
}

int oxe_engine_mtp_run(oxe_engine *e, const uint32_t *toks, int n, int pos0, const float *hs, int head_last,
                       uint32_t *argmax_out) {
    return ((Engine *)e)->mtp_run(toks, n, pos0, hs, head_last, argmax_out);
}

int oxe_engine_mtp_seed(oxe_engine *e, const uint32_t *toks, int n, int pos0, const float *hs) {
    return ((Engine *)e)->mtp_seed(toks, n, pos0, hs);
}

int oxe_engine_pos(const oxe_engine *e) { return ((const Engine *)e)->pos; }
int oxe_engine_n_ctx(const oxe_engine *e) { return ((const Engine *)e)->m.n_ctx; }

int oxe_engine_hidden(oxe_engine *e, int lane, float *out) {
    Engine *g = (Engine *)e;
    if (lane < 0 || lane >= oxe::HID_N) return -1;
    if (hipMemcpyAsync(out, g->b.hid + (size_t)lane * oxe::shp::E, oxe::shp::E * 4, hipMemcpyDeviceToHost, g->st) != hipSuccess) return -2;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

int oxe_engine_logits(oxe_engine *e, int lane, float *out) {
    Engine *g = (Engine *)e;
    if (lane < 0 || lane >= oxe::OXE_NL) return -1;
    if (hipMemcpyAsync(out, g->b.logits + (size_t)lane * g->d.n_vocab, (size_t)g->d.n_vocab * 4, hipMemcpyDeviceToHost, g->st) != hipSuccess) return -2;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

int oxe_engine_counter(oxe_engine *e, int which, uint32_t *out) {
    Engine *g = (Engine *)e;
    if (which < 0 || which >= oxe::CNT_N) return -1;
    if (hipMemcpyAsync(out, g->b.counters + which, 4, hipMemcpyDeviceToHost, g->st) != hipSuccess) return -2;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

// Copy engine state between host and device for parity checks and state hand-off.
// which: 0 K cache [n_att][NKV][n_ctx][HD] f16, 1 V^T cache [n_att][NKV*HD][n_ctx] f16,
//        2 conv state of the current slot [n_rec][NCH][KC-1] f32, 3 delta-net S of the current slot
//        [n_rec][NVH][HV][HV] f32 (row j of head h holds S[i][j] at [h][j][i]).
// dir 0: device -> host, 1: host -> device. offset/nbytes in bytes within the region.
int oxe_engine_state_copy(oxe_engine *e, int which, int dir, int64_t offset, void *host, int64_t nbytes) {
    Engine *g = (Engine *)e;
    using namespace oxe::shp;
    char *base = nullptr;
    int64_t size = 0;
    switch (which) {
    case 0: base = (char *)g->m.kcache; size = (int64_t)g->m.n_att * NKV * g->m.n_ctx * HD * 2; break;
    case 1: base = (char *)g->m.vcache; size = (int64_t)g->m.n_att * NKV * HD * g->m.n_ctx * 2; break;
    case 2: size = (int64_t)g->m.n_rec * NCH * (KC - 1) * 4; base = (char *)g->m.conv_state + (int64_t)g->cur * size; break;
    case 3: size = (int64_t)g->m.n_rec * NVH * HV * HV * 4; base = (char *)g->m.ssm_state + (int64_t)g->cur * size; break;
    default: return -1;
    }
    if (offset < 0 || nbytes < 0 || offset + nbytes > size) return -1;
    const hipError_t r = dir == 0 ? hipMemcpyAsync(host, base + offset, nbytes, hipMemcpyDeviceToHost, g->st)
                                  : hipMemcpyAsync(base + offset, host, nbytes, hipMemcpyHostToDevice, g->st);
    if (r != hipSuccess) return -2;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

int oxe_engine_set_pos(oxe_engine *e, int pos) {
    Engine *g = (Engine *)e;
    if (pos < 0 || pos > g->m.n_ctx) return -1;
    g->pos = pos;
    g->pend_n = 0;
    return 0;
}

int oxe_engine_set_router(oxe_engine *e, int layer, int row0, int nrows, const float *host) {
    Engine *g = (Engine *)e;
    if (layer < 0 || layer > g->d.n_layer || row0 < 0 || nrows < 1 || row0 + nrows > oxe::NEXP || !host) return -1;
    float *dst = g->L[layer].router + (int64_t)row0 * oxe::E;
    if (hipMemcpyAsync(dst, host, (size_t)nrows * oxe::E * sizeof(float), hipMemcpyHostToDevice, g->st) != hipSuccess) return -2;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

int64_t oxe_engine_device_bytes(const oxe_engine *e) { return (int64_t)((const Engine *)e)->bytes; }

// Engine::state_bytes (engine.rs:1570-1576): K and V^T of the positions < pos of every attention
// layer (the MTP layer's included), f16, then the current slot's conv and delta-net state, f32.
int64_t oxe_engine_state_bytes(const oxe_engine *e) {
    const Engine *g = (const Engine *)e;
    using namespace oxe::shp;
    const int64_t rec = (int64_t)g->m.n_rec * (NCH * (KC - 1) + NVH * HV * HV) * 4;
    return (int64_t)g->m.n_att * NKV * (2 * HD + 2 * HD) * g->pos + rec;
}

// K and V^T rows of positions [a, b) of every attention layer (the MTP layer's included), in the
// order of Engine::write_kv_rows / read_kv_rows (engine.rs:1727-1810): per layer the K rows of
// each KV head, then the V^T rows (kv head * head_dim + dim), f16 bits. to_host: device -> host.
static int kv_rows_copy(Engine *g, int a, int b, char *host, bool to_host) {
    using namespace oxe::shp;
    const int n = b - a, n_ctx = g->m.n_ctx;
    if (n == 0) return 0;
    const hipMemcpyKind kind = to_host ? hipMemcpyDeviceToHost : hipMemcpyHostToDevice;
    for (int ai = 0; ai < g->m.n_att; ai++) {
        for (int h = 0; h < NKV; h++) {
            uint16_t *k = g->m.kcache + ((int64_t)ai * NKV + h) * n_ctx * HD + (int64_t)a * HD;
            if (hipMemcpyAsync(to_host ? (void *)host : (void *)k, to_host ? (const void *)k : (const void *)host,
                               (size_t)n * HD * 2, kind, g->st) != hipSuccess)
                return -2;
            host += (size_t)n * HD * 2;
        }
        uint16_t *vt = g->m.vcache + (int64_t)ai * NKV * HD * n_ctx + a;
        const hipError_t r = to_host ? hipMemcpy2DAsync(host, (size_t)n * 2, vt, (size_t)n_ctx * 2, (size_t)n * 2,
                                                        NKV * HD, kind, g->st)
                                     : hipMemcpy2DAsync(vt, (size_t)n_ctx * 2, host, (size_t)n * 2, (size_t)n * 2,
                                                        NKV * HD, kind, g->st);
        if (r != hipSuccess) return -2;
        host += (size_t)NKV * HD * n * 2;
    }
    return 0;
}

// Engine::kv_row_bytes (engine.rs:1812-1814): K + V bytes per position over every attention layer
int64_t oxe_engine_kv_row_bytes(const oxe_engine *e) {
    using namespace oxe::shp;
    return (int64_t)((const Engine *)e)->m.n_att * NKV * 4 * HD;
}

// Engine::write_kv_rows (engine.rs:1727-1767): rows of positions [a, b), b <= pos
int oxe_engine_write_kv_rows(oxe_engine *e, int a, int b, void *host, int64_t cap) {
    Engine *g = (Engine *)e;
    if (a < 0 || a > b || b > g->pos) {
        oxe::set_err("kv rows beyond the current position");
        return -1;
    }
    if (!host || cap < oxe_engine_kv_row_bytes(e) * (b - a)) return -1;
    int rc = kv_rows_copy(g, a, b, (char *)host, true);
    if (rc) return rc;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

// Engine::read_kv_rows (engine.rs:1769-1810): rows of positions [a, b), b <= n_ctx; the position
// does not change (a recurrent snapshot sets it after the rows)
int oxe_engine_read_kv_rows(oxe_engine *e, int a, int b, const void *host, int64_t nbytes) {
    Engine *g = (Engine *)e;
    if (a < 0 || a > b || b > g->m.n_ctx) {
        oxe::set_err("kv rows beyond the context");
        return -1;
    }
    if (!host || nbytes != oxe_engine_kv_row_bytes(e) * (b - a)) return -1;
    int rc = kv_rows_copy(g, a, b, (char *)host, false);
    if (rc) return rc;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

// Engine::write_state (engine.rs:1682-1722): the KV rows of positions < pos, then conv and S of
// the current slot. Little-endian raw bits into host memory of cap bytes.
int oxe_engine_write_state(oxe_engine *e, void *host, int64_t cap) {
    Engine *g = (Engine *)e;
    using namespace oxe::shp;
    const int64_t need = oxe_engine_state_bytes(e);
    if (!host || cap < need) return -1;
    char *o = (char *)host;
    int rc = kv_rows_copy(g, 0, g->pos, o, true);
    if (rc) return rc;
    o += oxe_engine_kv_row_bytes(e) * g->pos;
    const size_t conv = (size_t)g->m.n_rec * NCH * (KC - 1) * 4, ssm = (size_t)g->m.n_rec * NVH * HV * HV * 4;
    if (hipMemcpyAsync(o, (const char *)g->m.conv_state + g->cur * conv, conv, hipMemcpyDeviceToHost, g->st) != hipSuccess)
        return -2;
    o += conv;
    if (hipMemcpyAsync(o, (const char *)g->m.ssm_state + g->cur * ssm, ssm, hipMemcpyDeviceToHost, g->st) != hipSuccess)
        return -2;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

// Engine::read_state (engine.rs:1819-1871): the inverse of write_state for n_pos positions; V^T
// columns [n_pos, pos) of a longer current sequence are zeroed (zero_v), the position becomes n_pos
// and any uncommitted verify is dropped.
int oxe_engine_read_state(oxe_engine *e, const void *host, int64_t nbytes, int n_pos) {
    Engine *g = (Engine *)e;
    using namespace oxe::shp;
    if (!host || n_pos < 0 || n_pos > g->m.n_ctx) return -1;
    const size_t conv = (size_t)g->m.n_rec * NCH * (KC - 1) * 4, ssm = (size_t)g->m.n_rec * NVH * HV * HV * 4;
    const int64_t need = oxe_engine_kv_row_bytes(e) * n_pos + (int64_t)(conv + ssm);
    if (nbytes != need) return -1;
    const char *in = (const char *)host;
    int rc = kv_rows_copy(g, 0, n_pos, (char *)in, false);
    if (rc) return rc;
    in += oxe_engine_kv_row_bytes(e) * n_pos;
    if (hipMemcpyAsync((char *)g->m.conv_state + g->cur * conv, in, conv, hipMemcpyHostToDevice, g->st) != hipSuccess)
        return -2;
    in += conv;
    if (hipMemcpyAsync((char *)g->m.ssm_state + g->cur * ssm, in, ssm, hipMemcpyHostToDevice, g->st) != hipSuccess)
        return -2;
    // every attention layer's V^T of the positions the old sequence held beyond n_pos back to +0
    if (g->pos > n_pos) oxe::launch_zero_v(g->m, g->m.n_att, n_pos, g->pos, g->st);
    g->pos = n_pos;
    g->pend_n = 0;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

}  // extern "C"

extern "C" int oxe_engine_set_fused(oxe_engine *e, int on) {
    Engine *g = (Engine *)e;
    if (g->set_fused(on != 0)) {
        oxe::set_err(g->kq ? "the fused run kernel reads Q8_0 matrices only: this engine's K-quant / F32 matrices run per phase"
                           : "the fused run kernel is not available on this device");
        return -1;
    }
    return 0;
}

extern "C" int oxe_engine_fused(const oxe_engine *e) { return ((const Engine *)e)->fused ? 1 : 0; }

extern "C" int oxe_engine_set_trace(oxe_engine *e, int on) { return ((Engine *)e)->set_trace(on != 0); }

extern "C" int64_t oxe_engine_read_trace(oxe_engine *e, unsigned long long *host, int64_t cap) {
    Engine *g = (Engine *)e;
    if (!g->fz_trace) return -1;
    const int64_t n = (int64_t)g->fz_grid * oxe::FZ_TRACE_EV * 4;
    if (cap < n) return -1;
    if (hipMemcpyAsync(host, g->fz_trace, (size_t)n * 8, hipMemcpyDeviceToHost, g->st) != hipSuccess) return -2;
    if (hipStreamSynchronize(g->st) != hipSuccess) return -2;
    return n;
}
