// TEST INFRASTRUCTURE ONLY (see oxo.h). The reference's qwen35moe decode engine restated on the CPU:
// lanes, recurrent slots, KV cache, the per-layer phases, the LM head and the MTP head
// (crates/model/src/engine.rs, crates/model/src/mtp.rs), on the synthetic model of
// include/oxe_model.h. Phase bodies follow the reference's per-lane arithmetic exactly; the
// per-thread row splits of the reference become OpenMP row loops (rows are independent, so the
// split never changes a value: the reference's own thread-count-invariance property,
// crates/model/src/tests.rs:288).
#include "oxo.h"
#include "oxo_model.h"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cmath>
#include <cstring>
#include <functional>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include <omp.h>
#include <sched.h>

namespace {

// A weight matrix [rows][k]: Q8_0 (codes q and fp16 block scales d), a K-quant (the file's ggml
// blocks in raw, rows contiguous) or F32 (rows in raw as floats); type is the ggml type id.
struct Mat {
    int64_t rows = 0, k = 0;
    int type = 8;   // 0 F32, 8 Q8_0, 11 Q3_K, 12 Q4_K, 13 Q5_K, 14 Q6_K
    std::vector<int8_t> q;
    std::vector<uint16_t> d;
    std::vector<uint8_t> raw;
};

int kq_block_bytes(int type) {
    switch (type) {
        case 11: return 110;
        case 12: return 144;
        case 13: return 176;
        case 14: return 210;
        default: return 0;
    }
}

// set on the threads of a plan run: their work is their share, so nothing inside spawns a team
thread_local bool tl_in_plan = false;

// Generate rows [r0, r0+n) of expert e of a Q8_0 tensor [experts][rows][k] into m.
void gen_q8(uint64_t seed, int layer, int kind, int64_t rows, int64_t k, int64_t e, Mat &m) {
    m.rows = rows;
    m.k = k;
    m.q.resize(rows * k);
    m.d.resize(rows * k / 32);
    const uint64_t key = oxe_tensor_key(seed, layer, kind);
    const uint64_t skey = oxe_tensor_key(seed, layer, kind + OXE_T_SCALE_OFFSET);
    const oxe_synth_param p = oxe_synth_param_of(kind);
    const uint64_t base = (uint64_t)e * rows * k;
#pragma omp parallel for schedule(static) if (!tl_in_plan)
    for (int64_t r = 0; r < rows; r++) {
        for (int64_t i = 0; i < k; i++) m.q[r * k + i] = oxe_synth_code(key, base + r * k + i);
        for (int64_t b = 0; b < k / 32; b++)
            m.d[r * (k / 32) + b] = oxe_synth_scale(skey, (base + r * k) / 32 + b, p);
    }
}

// rows [r0, r1) of expert e's matrix m (already sized rows x k), on the calling thread
void gen_q8_rows(uint64_t seed, int layer, int kind, int64_t rows, int64_t k, int64_t e, int64_t r0, int64_t r1, Mat &m) {
    const uint64_t key = oxe_tensor_key(seed, layer, kind);
    const uint64_t skey = oxe_tensor_key(seed, layer, kind + OXE_T_SCALE_OFFSET);
    const oxe_synth_param p = oxe_synth_param_of(kind);
    const uint64_t base = (uint64_t)e * rows * k;
    for (int64_t r = r0; r < r1; r++) {
        for (int64_t i = 0; i < k; i++) m.q[r * k + i] = oxe_synth_code(key, base + r * k + i);
        for (int64_t b = 0; b < k / 32; b++)
            m.d[r * (k / 32) + b] = oxe_synth_scale(skey, (base + r * k) / 32 + b, p);
    }
}

std::vector<float> gen_f32(uint64_t seed, int layer, int kind, int64_t n) {
    std::vector<float> v(n);
    const uint64_t key = oxe_tensor_key(seed, layer, kind);
    for (int64_t i = 0; i < n; i++) v[i] = oxe_synth_f32(key, (uint64_t)i, kind);
    return v;
}

struct Layer {
    bool att = false;
    std::vector<float> attn_norm, post_norm;
    // delta-net
    Mat qkv, z, beta, alpha, out;
    std::vector<float> conv, a, dt, ssm_norm;
    // attention
    Mat wq, wk, wv;
    std::vector<float> q_norm, k_norm;
    // MoE
    std::vector<float> router, shexp_gate;
    Mat gate_sh, up_sh, down_sh;
    std::vector<std::unique_ptr<Mat[]>> experts;  // [expert] -> {gate, up, down}, lazily generated
    // MTP block
    Mat eh_proj;
    std::vector<float> enorm, hnorm, head_norm;
    int index = 0;  // recurrent or attention index
};

// ---- The reference's worker pool (crates/sched/src/lib.rs:1-11, 43-84, 320-345): a persistent
// team, thread i pinned to the i-th CPU of the creating thread's affinity set (the creator is
// thread 0 and gets its mask back when the pool goes), jobs published through an epoch, and a
// centralised sense-reversing spin barrier whose episodes are counted. Idle workers spin on the
// epoch for a while and then yield.
struct PlanPool {
    struct alignas(128) Line {
        std::atomic<uint32_t> v{0};
    };
    int n = 1;
    std::vector<std::thread> th;
    Line epoch, arrived, sense, stop;
    std::atomic<uint64_t> episodes{0};
    std::vector<Line> lsense;   // per-thread barrier sense (each slot touched by its owner only)
    const std::function<void(int)> *job = nullptr;
    cpu_set_t caller_mask;
    bool pinned = false;

    static void pin(int cpu) {
        cpu_set_t one;
        CPU_ZERO(&one);
        CPU_SET(cpu, &one);
        sched_setaffinity(0, sizeof(one), &one);
    }
    // team of n threads (n <= CPUs of the caller's mask); returns false if the mask is unreadable
    bool start(int nthreads) {
        CPU_ZERO(&caller_mask);
        if (sched_getaffinity(0, sizeof(caller_mask), &caller_mask) != 0) return false;
        std::vector<int> cpus;
        for (int c = 0; c < CPU_SETSIZE; c++)
            if (CPU_ISSET(c, &caller_mask)) cpus.push_back(c);
        if (cpus.empty()) return false;
        n = std::max(1, std::min<int>(nthreads, (int)cpus.size()));
        lsense = std::vector<Line>(n);
        pin(cpus[0]);
        pinned = true;
        for (int t = 1; t < n; t++) th.emplace_back([this, t, c = cpus[t]] { worker(t, c); });
        return true;
    }
    ~PlanPool() {
        stop.v.store(1, std::memory_order_release);
        epoch.v.fetch_add(1, std::memory_order_release);
        for (auto &t : th) t.join();
        if (pinned) sched_setaffinity(0, sizeof(caller_mask), &caller_mask);
    }
    // counted: false for the barriers of synthetic-weight generation (not part of the plan)
    void barrier(int tid, bool counted = true) {
        const uint32_t s = lsense[tid].v.load(std::memory_order_relaxed) ^ 1u;
        lsense[tid].v.store(s, std::memory_order_relaxed);
        if (n == 1) {
            if (counted) episodes.fetch_add(1, std::memory_order_relaxed);
            return;
        }
        if (arrived.v.fetch_add(1, std::memory_order_acq_rel) + 1 == (uint32_t)n) {
            arrived.v.store(0, std::memory_order_relaxed);
            if (counted) episodes.fetch_add(1, std::memory_order_relaxed);
            sense.v.store(s, std::memory_order_release);
        } else {
            while (sense.v.load(std::memory_order_acquire) != s) __builtin_ia32_pause();
        }
    }
    void worker(int tid, int cpu) {
        pin(cpu);
        tl_in_plan = true;
        uint32_t seen = 0;
        for (;;) {
            uint32_t e;
            int spins = 0;
            while ((e = epoch.v.load(std::memory_order_acquire)) == seen) {
                if (++spins < (1 << 16)) __builtin_ia32_pause();
                else std::this_thread::yield();
            }
            seen = e;
            if (stop.v.load(std::memory_order_acquire)) return;
            (*job)(tid);
            barrier(tid);   // the join
        }
    }
    // run f on every thread (the caller is thread 0); returns after the join barrier
    void run(const std::function<void(int)> &f) {
        job = &f;
        epoch.v.fetch_add(1, std::memory_order_release);
        tl_in_plan = true;
        f(0);
        barrier(0);
        tl_in_plan = false;
    }
};

// plan::split / split_rows (crates/model/src/plan.rs:156-164)
inline void split(int64_t n, int parts, int i, int64_t &a, int64_t &b) {
    a = n * i / parts;
    b = n * (i + 1) / parts;
}
inline void split_rows(int64_t rows, int parts, int i, int64_t &a, int64_t &b) {
    split(rows / 8, parts, i, a, b);
    a *= 8;
    b *= 8;
}

// rows [r0, r1) of a Q8_0 matrix for nl lanes, y[l][r - r0], on the calling thread: the same
// per-(row, lane) block chain as oxo_gemv_q8_0
void gemv_rows(const int8_t *wq, const uint16_t *wd, int64_t k, int64_t r0, int64_t r1, int nl, const int8_t *const *xq,
               const uint16_t *const *xd, float *const *y) {
    const int64_t nb = k / 32;
    for (int64_t r = r0; r < r1; r++) {
        const int8_t *w = wq + r * k;
        for (int l = 0; l < nl; l++) {
            const int8_t *x = xq[l];
            float acc = 0.0f;
            for (int64_t b = 0; b < nb; b++) {
                int32_t s = 0;
                for (int j = 0; j < 32; j++) s += (int32_t)w[b * 32 + j] * (int32_t)x[b * 32 + j];
                const float prod = oxo_f16_to_f32(xd[l][b]) * oxo_f16_to_f32(wd[r * nb + b]);
                acc = std::fma((float)s, prod, acc);
            }
            y[l][r - r0] = acc;
        }
    }
}

inline int64_t padded_n_kv(int64_t pos, int64_t n_ctx) {
    return std::min(n_ctx, std::max<int64_t>(256, (pos + 1 + 255) / 256 * 256));
}

}  // namespace

struct oxo_engine {
    oxe_model_desc d{};
    uint64_t seed = 0;
    int64_t n_ctx = 0;
    int n_slots = 2, max_lanes = 8;
    std::vector<Layer> layers;  // n_layer (+1 MTP)
    std::vector<float> out_norm;
    Mat output;
    std::mutex gen_mu;
    // ggml type of each matrix: [layer (OXE_GLOBAL_LAYER for the global tensors)][tensor kind];
    // 8 (Q8_0) unless set at creation
    std::vector<int32_t> types = std::vector<int32_t>(64 * 64, 8);
    bool typed = false;   // some matrix is not Q8_0 (the plan mode takes Q8_0 models only)
    int type_of(int layer, int kind) const { return types[(size_t)layer * 64 + kind]; }
    void gen_mat(int layer, int kind, int64_t rows, int64_t k, int64_t e, Mat &m) const {
        const int ty = type_of(layer, kind);
        if (ty == 8) {
            gen_q8(seed, layer, kind, rows, k, e, m);
            m.type = 8;
            return;
        }
        m.rows = rows;
        m.k = k;
        m.type = ty;
        if (ty == 0) {
            const std::vector<float> v = gen_f32(seed, layer, kind, rows * k);
            m.raw.resize(v.size() * 4);
            std::memcpy(m.raw.data(), v.data(), m.raw.size());
        } else {
            m.raw.resize((size_t)rows * (k / 256) * kq_block_bytes(ty));
            oxo_synth_kq(seed, layer, kind, ty, e, rows, k, m.raw.data());
        }
    }

    int n_rec = 0, n_att = 0;  // n_att includes the MTP layer
    int64_t conv_len = 0, ssm_len = 0, v_stride = 0;
    std::vector<float> conv_state, ssm_state;   // [slot][rec layer][...]
    std::vector<uint16_t> kcache, vcache;       // [att][kvh][n_ctx][hd], [att][kvh*hd][v_stride]
    std::vector<float> rope_tab;                // [n_ctx][n_rot]
    int64_t pos = 0;
    int cur_slot = 0;
    int64_t pend_pos0 = 0;
    int pend_cur = 0, pend_n = 0, pend_done = 0;
    int tie_count = 0;

    // per-lane buffers
    std::vector<std::vector<float>> xin, x1, x2, o, hout, hin, logits;
    std::vector<uint32_t> argmax;
    bool keep_logits = true;

    double gen_seconds = 0.0;
    const Mat &expert(int l, int e, int which) {
        Layer &L = layers[l];
        std::lock_guard<std::mutex> g(gen_mu);
        if (!L.experts[e]) {
            const auto t0 = std::chrono::steady_clock::now();
            std::unique_ptr<Mat[]> m(new Mat[3]);
            const int64_t E = d.n_embd, F = d.ff_exp;
            gen_mat(l, OXE_T_GATE_EXPS, F, E, e, m[0]);
            gen_mat(l, OXE_T_UP_EXPS, F, E, e, m[1]);
            gen_mat(l, OXE_T_DOWN_EXPS, E, F, e, m[2]);
            L.experts[e] = std::move(m);
            gen_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
        }
        return L.experts[e][which];
    }

    Mat tok_embd_k;   // a K-quant token embedding (its rows dequantised per token)
    std::vector<float> embed(uint32_t tok) {
        const int64_t E = d.n_embd;
        if (tok_embd_k.type != 8) {
            // dequantize_row of the token's row (engine.rs:2251-2256)
            std::vector<float> y(E);
            const size_t rb = (size_t)(E / 256) * kq_block_bytes(tok_embd_k.type);
            oxo_dequantize_row_kq(tok_embd_k.type, tok_embd_k.raw.data() + (size_t)tok * rb, y.data(), E);
            return y;
        }
        std::vector<int8_t> q(E);
        std::vector<uint16_t> dd(E / 32);
        const uint64_t key = oxe_tensor_key(seed, OXE_GLOBAL_LAYER, OXE_T_TOK_EMBD);
        const uint64_t skey = oxe_tensor_key(seed, OXE_GLOBAL_LAYER, OXE_T_TOK_EMBD + OXE_T_SCALE_OFFSET);
        const oxe_synth_param p = oxe_synth_param_of(OXE_T_TOK_EMBD);
        for (int64_t i = 0; i < E; i++) q[i] = oxe_synth_code(key, (uint64_t)tok * E + i);
        for (int64_t b = 0; b < E / 32; b++) dd[b] = oxe_synth_scale(skey, (uint64_t)tok * E / 32 + b, p);
        std::vector<float> y(E);
        oxo_dequantize_row_q8_0(q.data(), dd.data(), E, y.data());
        return y;
    }

    // y[nl][rows] = W . x[l] for each lane (the reference's mv / mv_lanes, engine.rs:2270-2343): F32
    // rows by oxe_vec_dot_f32 on x itself; K-quants by the lane GEMV on x quantised to q8_K; Q8_0 by
    // the block chain on x quantised to Q8_0
    static void mv(const Mat &w, const std::vector<const float *> &xs, std::vector<float *> ys) {
        const int nl = (int)xs.size();
        if (w.type == 0) {
            const float *rows = (const float *)w.raw.data();
            for (int l = 0; l < nl; l++)
                for (int64_t r = 0; r < w.rows; r++) ys[l][r] = oxo_vec_dot_f32((int)w.k, rows + r * w.k, xs[l]);
            return;
        }
        if (w.type != 8) {
            const int64_t nb = w.k / 256;
            std::vector<uint8_t> y((size_t)nl * nb * 292);
            for (int l = 0; l < nl; l++) oxo_quantize_row_q8_K(xs[l], y.data() + (size_t)l * nb * 292, w.k);
            std::vector<float> s((size_t)nl * w.rows);
            oxo_vl_gemv(w.type - 8, w.k, w.rows, nl, w.raw.data(), y.data(), s.data());
            for (int l = 0; l < nl; l++) std::memcpy(ys[l], s.data() + (size_t)l * w.rows, w.rows * sizeof(float));
            return;
        }
        std::vector<int8_t> xq(nl * w.k);
        std::vector<uint16_t> xd(nl * w.k / 32);
        for (int l = 0; l < nl; l++) oxo_quantize_row_q8_0(xs[l], w.k, xq.data() + l * w.k, xd.data() + l * w.k / 32);
        std::vector<float> y(nl * w.rows);
        oxo_gemv_q8_0(w.k, w.rows, nl, w.q.data(), w.d.data(), xq.data(), xd.data(), y.data(), nullptr);
        for (int l = 0; l < nl; l++) std::memcpy(ys[l], y.data() + l * w.rows, w.rows * sizeof(float));
    }

    void init(const oxe_model_desc &desc, uint64_t s, int64_t nctx) {
        d = desc;
        seed = s;
        n_ctx = (nctx + 255) / 256 * 256;
        const int64_t E = d.n_embd;
        const int nl_total = d.n_layer + (d.has_mtp ? 1 : 0);
        layers.resize(nl_total);
        const int64_t ds = d.ssm_d_state, nk = d.ssm_n_kheads, nv = d.ssm_n_vheads;
        const int64_t nch = d.ssm_d_inner + 2 * nk * ds, hv = d.ssm_d_inner / nv, hd = d.head_dim;
        for (int il = 0; il < nl_total; il++) {
            Layer &L = layers[il];
            const bool mtp = il == d.n_layer;
            L.att = mtp || ((il + 1) % d.full_attention_interval == 0);
            L.index = L.att ? n_att++ : n_rec++;
            L.attn_norm = gen_f32(seed, il, OXE_T_ATTN_NORM, E);
            L.post_norm = gen_f32(seed, il, OXE_T_POST_NORM, E);
            if (!L.att) {
                gen_mat(il, OXE_T_DN_QKV, nch, E, 0, L.qkv);
                gen_mat(il, OXE_T_DN_Z, d.ssm_d_inner, E, 0, L.z);
                gen_mat(il, OXE_T_DN_BETA, nv, E, 0, L.beta);
                gen_mat(il, OXE_T_DN_ALPHA, nv, E, 0, L.alpha);
                gen_mat(il, OXE_T_DN_OUT, E, d.ssm_d_inner, 0, L.out);
                L.conv = gen_f32(seed, il, OXE_T_DN_CONV, nch * d.ssm_conv_kernel);
                L.a = gen_f32(seed, il, OXE_T_DN_A, nv);
                L.dt = gen_f32(seed, il, OXE_T_DN_DT, nv);
                L.ssm_norm = gen_f32(seed, il, OXE_T_DN_NORM, hv);
            } else {
                gen_mat(il, OXE_T_ATT_Q, d.n_head * 2 * hd, E, 0, L.wq);
                gen_mat(il, OXE_T_ATT_K, d.n_head_kv * hd, E, 0, L.wk);
                gen_mat(il, OXE_T_ATT_V, d.n_head_kv * hd, E, 0, L.wv);
                gen_mat(il, OXE_T_ATT_OUT, E, d.n_head * hd, 0, L.out);
                L.q_norm = gen_f32(seed, il, OXE_T_ATT_QNORM, hd);
                L.k_norm = gen_f32(seed, il, OXE_T_ATT_KNORM, hd);
            }
            L.router = gen_f32(seed, il, OXE_T_ROUTER, (int64_t)d.n_expert * E);
            L.shexp_gate = gen_f32(seed, il, OXE_T_SHEXP_GATE, E);
            gen_mat(il, OXE_T_GATE_SHEXP, d.ff_shexp, E, 0, L.gate_sh);
            gen_mat(il, OXE_T_UP_SHEXP, d.ff_shexp, E, 0, L.up_sh);
            gen_mat(il, OXE_T_DOWN_SHEXP, E, d.ff_shexp, 0, L.down_sh);
            L.experts.resize(d.n_expert);
            if (mtp) {
                gen_mat(il, OXE_T_EH_PROJ, E, 2 * E, 0, L.eh_proj);
                L.enorm = gen_f32(seed, il, OXE_T_ENORM, E);
                L.hnorm = gen_f32(seed, il, OXE_T_HNORM, E);
                L.head_norm = gen_f32(seed, il, OXE_T_HEAD_NORM, E);
            }
        }
        out_norm = gen_f32(seed, OXE_GLOBAL_LAYER, OXE_T_OUT_NORM, E);
        gen_mat(OXE_GLOBAL_LAYER, OXE_T_OUTPUT, d.n_vocab, E, 0, output);
        if (type_of(OXE_GLOBAL_LAYER, OXE_T_TOK_EMBD) != 8) gen_mat(OXE_GLOBAL_LAYER, OXE_T_TOK_EMBD, d.n_vocab, E, 0, tok_embd_k);
        conv_len = (d.ssm_conv_kernel - 1) * nch;
        ssm_len = nv * hv * hv;
        conv_state.assign((size_t)n_slots * n_rec * conv_len, 0.0f);
        ssm_state.assign((size_t)n_slots * n_rec * ssm_len, 0.0f);
        v_stride = n_ctx;
        kcache.assign((size_t)n_att * d.n_head_kv * n_ctx * hd, 0);
        vcache.assign((size_t)n_att * d.n_head_kv * hd * v_stride, 0);
        rope_tab.resize((size_t)n_ctx * d.n_rot);
        for (int64_t p = 0; p < n_ctx; p++)
            oxo_mrope_cache_init(p, d.rope_sections, 1, d.n_rot, d.n_rot, d.rope_freq_base, 1.0f, 0.0f, 1.0f,
                                 32.0f, 1.0f, d.n_ctx_train, 0, rope_tab.data() + p * d.n_rot);
        auto lanes = [&](int64_t n) { return std::vector<std::vector<float>>(max_lanes, std::vector<float>(n, 0.0f)); };
        xin = lanes(E); x1 = lanes(E); x2 = lanes(E); hout = lanes(E); hin = lanes(E);
        o = lanes(std::max<int64_t>(d.ssm_d_inner, d.n_head * hd));
        logits = lanes(d.n_vocab);
        argmax.assign(max_lanes, 0);
    }

    void reset() {
        std::fill(conv_state.begin(), conv_state.end(), 0.0f);
        std::fill(ssm_state.begin(), ssm_state.end(), 0.0f);
        std::fill(vcache.begin(), vcache.end(), 0);
        pos = 0;
        cur_slot = 0;
        pend_n = 0;
    }

    // ---- phases (engine.rs); every phase loops over the run's lanes in order

    // rec_mix (engine.rs:2394-2570) for all lanes, then mixer_out (2573-2609)
    void recurrent(int l, int nl) {
        Layer &L = layers[l];
        const int64_t E = d.n_embd, ds = d.ssm_d_state, nk = d.ssm_n_kheads, nv = d.ssm_n_vheads;
        const int64_t hv = d.ssm_d_inner / nv, nch = d.ssm_d_inner + 2 * nk * ds, kc = d.ssm_conv_kernel;
        const float eps = d.rms_eps;
        std::vector<std::vector<float>> xn(nl, std::vector<float>(E)), qkv(nl, std::vector<float>(nch)),
            z(nl, std::vector<float>(d.ssm_d_inner)), beta(nl, std::vector<float>(nv)), alpha(nl, std::vector<float>(nv));
        std::vector<const float *> xs;
        for (int ln = 0; ln < nl; ln++) {
            oxo_rms_norm_mul_f32(xin[ln].data(), L.attn_norm.data(), xn[ln].data(), E, eps);
            xs.push_back(xn[ln].data());
        }
        auto outs = [&](std::vector<std::vector<float>> &v) {
            std::vector<float *> r;
            for (int ln = 0; ln < nl; ln++) r.push_back(v[ln].data());
            return r;
        };
        mv(L.qkv, xs, outs(qkv));
        mv(L.z, xs, outs(z));
        mv(L.beta, xs, outs(beta));
        mv(L.alpha, xs, outs(alpha));
        const int ri = L.index;
        std::vector<float> conv(nch), tmp(nch), gdn(hv), tmpn(hv), zs(hv);
        for (int ln = 0; ln < nl; ln++) {
            const int dst = (cur_slot + ln) % n_slots;
            const int src = ln == 0 ? dst : (cur_slot + ln - 1) % n_slots;
            float *cs = conv_state.data() + ((size_t)dst * n_rec + ri) * conv_len;
            if (src != dst) std::memcpy(cs, conv_state.data() + ((size_t)src * n_rec + ri) * conv_len, conv_len * 4);
            oxo_ssm_conv_step_f32(cs, qkv[ln].data(), L.conv.data(), (int)nch, (int)kc, conv.data());
            oxo_silu_f32((int)nch, tmp.data(), conv.data());
            conv = tmp;
            for (int64_t g = 0; g < nk; g++) {
                oxo_gdn_l2_norm_f32(conv.data() + g * ds, ds, eps);
                oxo_gdn_l2_norm_f32(conv.data() + nk * ds + g * ds, ds, eps);
            }
            std::vector<float> gate(nv), beta_s(nv);
            for (int64_t vh = 0; vh < nv; vh++) {
                const float ab = alpha[ln][vh] + L.dt[vh];
                float sp;
                oxo_softplus_f32(1, &sp, &ab);
                gate[vh] = sp * L.a[vh];
                oxo_sigmoid_f32(1, &beta_s[vh], &beta[ln][vh]);
            }
            for (int64_t vh = 0; vh < nv; vh++) {
                const int64_t kh = vh % nk;
                float *s = ssm_state.data() + ((size_t)dst * n_rec + ri) * ssm_len + vh * hv * hv;
                const float *s_in = ssm_state.data() + ((size_t)src * n_rec + ri) * ssm_len + vh * hv * hv;
                oxo_gated_delta_net_step_f32_from(s, s_in, conv.data() + kh * ds, conv.data() + nk * ds + kh * ds,
                                                  conv.data() + 2 * nk * ds + vh * hv, gate[vh], beta_s[vh], hv, gdn.data());
                oxo_rms_norm_mul_f32(gdn.data(), L.ssm_norm.data(), tmpn.data(), hv, eps);
                oxo_silu_f32((int)hv, zs.data(), z[ln].data() + vh * hv);
                for (int64_t j = 0; j < hv; j++) o[ln][vh * hv + j] = tmpn[j] * zs[j];
            }
        }
        mixer_out(l, nl, d.ssm_d_inner);
    }

    void mixer_out(int l, int nl, int64_t width) {
        Layer &L = layers[l];
        const int64_t E = d.n_embd;
        std::vector<const float *> xs;
        std::vector<std::vector<float>> t(nl, std::vector<float>(E));
        std::vector<float *> ys;
        for (int ln = 0; ln < nl; ln++) { xs.push_back(o[ln].data()); ys.push_back(t[ln].data()); }
        (void)width;
        mv(L.out, xs, ys);
        for (int ln = 0; ln < nl; ln++)
            for (int64_t i = 0; i < E; i++) x1[ln][i] = t[ln][i] + xin[ln][i];
    }

    // attn_qkv + attn_kv + write_k (engine.rs:2614-2739): projections for all lanes; K and V of
    // every lane written at pos0 + lane before any lane attends
    void attn_kv(int l, int nl, int64_t pos0, const std::vector<std::vector<float>> &xn) {
        Layer &L = layers[l];
        const int64_t hd = d.head_dim, nkv = d.n_head_kv;
        const int ai = L.index;
        std::vector<const float *> xs;
        std::vector<std::vector<float>> kraw(nl, std::vector<float>(nkv * hd)), vv(nl, std::vector<float>(nkv * hd));
        std::vector<float *> ko, vo;
        for (int ln = 0; ln < nl; ln++) { xs.push_back(xn[ln].data()); ko.push_back(kraw[ln].data()); vo.push_back(vv[ln].data()); }
        mv(L.wk, xs, ko);
        mv(L.wv, xs, vo);
        std::vector<float> kn(hd);
        for (int ln = 0; ln < nl; ln++) {
            const int64_t p = pos0 + ln;
            for (int64_t r = 0; r < nkv * hd; r++)
                vcache[((size_t)ai * nkv * hd + r) * v_stride + p] = oxo_f32_to_f16(vv[ln][r]);
            for (int64_t kvh = 0; kvh < nkv; kvh++) {
                oxo_rms_norm_mul_f32(kraw[ln].data() + kvh * hd, L.k_norm.data(), kn.data(), hd, d.rms_eps);
                oxo_rope_neox_inplace(kn.data(), d.n_rot, rope_tab.data() + p * d.n_rot);
                uint16_t *kr = kcache.data() + (((size_t)ai * nkv + kvh) * n_ctx + p) * hd;
                for (int64_t i = 0; i < hd; i++) kr[i] = oxo_f32_to_f16(kn[i]);
            }
        }
    }

    void attention(int l, int nl, int64_t pos0) {
        Layer &L = layers[l];
        const int64_t E = d.n_embd, hd = d.head_dim, nkv = d.n_head_kv, nh = d.n_head, group = nh / nkv;
        const int ai = L.index;
        std::vector<std::vector<float>> xn(nl, std::vector<float>(E)), qg(nl, std::vector<float>(nh * 2 * hd));
        std::vector<const float *> xs;
        std::vector<float *> qo;
        for (int ln = 0; ln < nl; ln++) {
            oxo_rms_norm_mul_f32(xin[ln].data(), L.attn_norm.data(), xn[ln].data(), E, d.rms_eps);
            xs.push_back(xn[ln].data());
            qo.push_back(qg[ln].data());
        }
        mv(L.wq, xs, qo);
        attn_kv(l, nl, pos0, xn);
        const float scale = 1.0f / sqrtf((float)hd);
        for (int ln = 0; ln < nl; ln++) {
            const int64_t p = pos0 + ln;
            const int n_kv = (int)padded_n_kv(p, n_ctx);
#pragma omp parallel for schedule(static)
            for (int64_t h = 0; h < nh; h++) {
                std::vector<float> q(hd), aout(hd), gs(hd);
                oxo_rms_norm_mul_f32(qg[ln].data() + h * 2 * hd, L.q_norm.data(), q.data(), hd, d.rms_eps);
                oxo_rope_neox_inplace(q.data(), d.n_rot, rope_tab.data() + p * d.n_rot);
                const int64_t kvh = h / group;
                const uint16_t *kb = kcache.data() + ((size_t)ai * nkv + kvh) * n_ctx * hd;
                const uint16_t *vb = vcache.data() + ((size_t)ai * nkv * hd + kvh * hd) * v_stride;
                oxo_attn_head_f16(q.data(), kb, hd, kb + p * hd, vb, v_stride, n_kv, (int)p, (int)hd, scale, aout.data());
                oxo_sigmoid_f32(hd, gs.data(), qg[ln].data() + h * 2 * hd + hd);
                for (int64_t j = 0; j < hd; j++) o[ln][h * hd + j] = aout[j] * gs[j];
            }
        }
        mixer_out(l, nl, nh * hd);
    }

    // moe_router + route + moe_gate_up + moe_down (engine.rs:3372-3624)
    void moe(int l, int nl) {
        Layer &L = layers[l];
        const int64_t E = d.n_embd, F = d.ff_exp, K = d.n_expert_used, NE = d.n_expert;
        for (int ln = 0; ln < nl; ln++) {
            std::vector<float> xn(E);
            oxo_rms_norm_mul_f32(x1[ln].data(), L.post_norm.data(), xn.data(), E, d.rms_eps);
            std::vector<float> lg(NE);
#pragma omp parallel for schedule(static)
            for (int64_t e = 0; e < NE; e++) lg[e] = oxo_vec_dot_f32((int)E, L.router.data() + e * E, xn.data());
            const float sgd = oxo_vec_dot_f32((int)E, L.shexp_gate.data(), xn.data());
            float sg;
            oxo_sigmoid_f32(1, &sg, &sgd);
            std::vector<float> gsh(d.ff_shexp), ush(d.ff_shexp), hsh(d.ff_shexp);
            mv(L.gate_sh, {xn.data()}, {gsh.data()});
            mv(L.up_sh, {xn.data()}, {ush.data()});
            oxo_swiglu_f32(d.ff_shexp, hsh.data(), gsh.data(), ush.data());
            // route (engine.rs:3414-3429)
            std::vector<float> probs(NE), wp(NE);
            oxo_soft_max_f32((int)NE, probs.data(), lg.data(), 1.0f, nullptr, wp.data());
            std::vector<int32_t> ids(K), scr(NE);
            int tie = 0;
            oxo_argsort_top_k_f32(probs.data(), (int)NE, (int)K, ids.data(), scr.data(), &tie);
            tie_count += tie;
            std::vector<float> w(K);
            for (int64_t j = 0; j < K; j++) w[j] = probs[ids[j]];
            float s = oxo_vec_sum_f32((int)K, w.data());
            s = std::max(std::min(s, INFINITY), 6.103515625e-5f);
            for (int64_t j = 0; j < K; j++) w[j] = w[j] / s;
            // experts
            std::vector<std::vector<float>> dn(K, std::vector<float>(E));
            for (int64_t j = 0; j < K; j++) {
                const Mat &wg = expert(l, ids[j], 0), &wu = expert(l, ids[j], 1), &wdn = expert(l, ids[j], 2);
                std::vector<float> g(F), u(F), h(F);
                mv(wg, {xn.data()}, {g.data()});
                mv(wu, {xn.data()}, {u.data()});
                oxo_swiglu_f32((int)F, h.data(), g.data(), u.data());
                mv(wdn, {h.data()}, {dn[j].data()});
            }
            std::vector<float> dsh(E);
            mv(L.down_sh, {hsh.data()}, {dsh.data()});
            for (int64_t i = 0; i < E; i++) {
                float m = dn[0][i] * w[0];
                for (int64_t j = 1; j < K; j++) {
                    const float p = dn[j][i] * w[j];
                    m = m + p;
                }
                const float sh = dsh[i] * sg;
                const float f = m + sh;
                x2[ln][i] = f + x1[ln][i];
            }
        }
    }

    // restricted-vocabulary draft head (MtpWeights::set_draft_vocab, mtp.rs:166-197): the draft
    // runs' argmax over these ids only (ascending, unique); empty: the whole head
    std::vector<uint32_t> draft_ids;
    std::vector<char> draft_mask;
    int set_draft_vocab(const uint32_t *ids, int n) {
        std::vector<uint32_t> v;
        for (int i = 0; i < n; i++)
            if (ids[i] < (uint32_t)d.n_vocab) v.push_back(ids[i]);
        if (n > 0 && v.empty()) return -1;
        std::sort(v.begin(), v.end());
        v.erase(std::unique(v.begin(), v.end()), v.end());
        draft_ids = v;
        draft_mask.assign(v.empty() ? 0 : d.n_vocab, 0);
        for (uint32_t i : v) draft_mask[i] = 1;
        return (int)v.size();
    }

    // head (engine.rs:3630-3715) + gather_argmax (1969-1987); draft: an MTP draft run's head (the
    // restricted one when set: its rows are the ids ascending, so the first maximum over them is
    // the first by id)
    void head(int nl, uint32_t mask, const std::vector<float> &norm, bool draft = false) {
        const int64_t E = d.n_embd, V = d.n_vocab;
        for (int ln = 0; ln < nl; ln++) {
            oxo_rms_norm_mul_f32(x2[ln].data(), norm.data(), hout[ln].data(), E, d.rms_eps);
            if (!(mask & (1u << ln))) continue;
            std::vector<float> lg(V);
            mv(output, {hout[ln].data()}, {lg.data()});
            float best = -INFINITY;
            uint32_t bi = UINT32_MAX;
            if (draft && !draft_ids.empty()) {
                for (uint32_t r : draft_ids)
                    if (lg[r] > best) { best = lg[r]; bi = r; }
            } else {
                for (int64_t r = 0; r < V; r++)
                    if (lg[r] > best) { best = lg[r]; bi = (uint32_t)r; }
            }
            argmax[ln] = bi == UINT32_MAX ? 0 : bi;
            if (keep_logits) logits[ln] = lg;
        }
    }

    void run_layer(int l, int nl, int64_t pos0, const uint32_t *toks) {
        if (l == 0)
            for (int ln = 0; ln < nl; ln++) xin[ln] = embed(toks[ln]);
        else
            for (int ln = 0; ln < nl; ln++) xin[ln] = x2[ln];
        if (layers[l].att) attention(l, nl, pos0);
        else recurrent(l, nl);
        moe(l, nl);
    }

    // ---- the static plan on the pinned team (crates/model/src/plan.rs:171-249, engine.rs:2137-2190):
    // every thread walks the run's phases and does its share of each; one barrier after each phase.
    // Each row, head, unit and logit is computed by one thread with the same arithmetic as the
    // methods above, so a plan run gives the same bits as they do.
    struct TS {
        std::vector<std::vector<float>> xin, xn, qkv, z, beta, alpha, conv, qg, cat, dtmp, probs, w;
        std::vector<std::vector<int8_t>> xq, oq;
        std::vector<std::vector<uint16_t>> xd, od;
        std::vector<std::vector<int32_t>> ids;
        std::vector<float> gate, beta_s, gdn, tmpn, zs, tmp, q, aout, gs, kn, g, u, wp, sh_gate;
        std::vector<int32_t> iscr;
        std::vector<std::pair<uint32_t, uint32_t>> uni_u;   // union units (expert, 256-row block)
        std::vector<uint32_t> uni_e;
    };
    std::unique_ptr<PlanPool> pool;
    std::vector<TS> pts;
    std::vector<std::vector<float>> p_router, p_hsh, p_h, p_kraw;
    std::vector<std::vector<int8_t>> p_hq, p_hshq;
    std::vector<std::vector<uint16_t>> p_hd, p_hshd;
    std::vector<std::vector<std::pair<float, uint32_t>>> p_best;   // [lane][thread]

    int set_plan(int nthreads) {
        pool.reset();
        pts.clear();
        if (nthreads <= 0) return 0;
        if (typed) return -1;
        pool.reset(new PlanPool());
        if (!pool->start(nthreads)) {
            pool.reset();
            return -1;
        }
        const int nt = pool->n, L = max_lanes;
        const int64_t E = d.n_embd, nk = d.ssm_n_kheads, ds = d.ssm_d_state, K = d.n_expert_used, F = d.ff_exp;
        const int64_t nch = d.ssm_d_inner + 2 * nk * ds, W = std::max<int64_t>(d.ssm_d_inner, d.n_head * d.head_dim);
        auto vv = [&](int64_t n) { return std::vector<std::vector<float>>(L, std::vector<float>(n, 0.0f)); };
        pts.resize(nt);
        for (TS &t : pts) {
            t.xin = vv(E); t.xn = vv(E); t.qkv = vv(nch); t.z = vv(d.ssm_d_inner); t.beta = vv(d.ssm_n_vheads);
            t.alpha = vv(d.ssm_n_vheads); t.conv = vv(nch); t.qg = vv(2 * d.n_head * d.head_dim); t.cat = vv(2 * E);
            t.dtmp = vv((K + 1) * E); t.probs = vv(d.n_expert); t.w = vv(K);
            t.xq.assign(L, std::vector<int8_t>(2 * E)); t.xd.assign(L, std::vector<uint16_t>(2 * E / 32));
            t.oq.assign(L, std::vector<int8_t>(W)); t.od.assign(L, std::vector<uint16_t>(W / 32));
            t.ids.assign(L, std::vector<int32_t>(K));
            t.gate.assign(d.ssm_n_vheads, 0.f); t.beta_s.assign(d.ssm_n_vheads, 0.f);
            const int64_t hv = d.ssm_d_inner / d.ssm_n_vheads;
            t.gdn.assign(hv, 0.f); t.tmpn.assign(hv, 0.f); t.zs.assign(hv, 0.f);
            t.tmp.assign(std::max<int64_t>(nch, 256), 0.f);
            t.q.assign(d.head_dim, 0.f); t.aout.assign(d.head_dim, 0.f); t.gs.assign(d.head_dim, 0.f);
            t.kn.assign(d.head_dim, 0.f); t.g.assign(256, 0.f); t.u.assign(256, 0.f);
            t.wp.assign(d.n_expert, 0.f); t.sh_gate.assign(L, 0.f); t.iscr.assign(d.n_expert, 0);
        }
        p_router = vv(d.n_expert); p_hsh = vv(d.ff_shexp); p_h = vv(K * F); p_kraw = vv(d.n_head_kv * d.head_dim);
        p_hq.assign(L, std::vector<int8_t>(K * F)); p_hd.assign(L, std::vector<uint16_t>(K * F / 32));
        p_hshq.assign(L, std::vector<int8_t>(d.ff_shexp)); p_hshd.assign(L, std::vector<uint16_t>(d.ff_shexp / 32));
        p_best.assign(L, std::vector<std::pair<float, uint32_t>>(nt));
        return nt;
    }

    // thread `tid`'s rows of w for its lanes: y[ln] + 0 .. (r1 - r0)
    static void rows_of(const Mat &w, int64_t r0, int64_t r1, int nl, std::vector<std::vector<int8_t>> &xq,
                        std::vector<std::vector<uint16_t>> &xd, const std::function<float *(int)> &y) {
        if (r1 <= r0) return;
        const int8_t *q[8];
        const uint16_t *dd[8];
        float *ys[8];
        for (int ln = 0; ln < nl; ln++) { q[ln] = xq[ln].data(); dd[ln] = xd[ln].data(); ys[ln] = y(ln); }
        gemv_rows(w.q.data(), w.d.data(), w.k, r0, r1, nl, q, dd, ys);
    }
    // the layer input and its norm on this thread (layer_entry + norm, engine.rs:2239-2266)
    void p_entry(TS &ts, int l, int nl, const uint32_t *toks, const std::vector<float> &normw) {
        for (int ln = 0; ln < nl; ln++) {
            if (l == 0) ts.xin[ln] = embed(toks[ln]);
            else std::memcpy(ts.xin[ln].data(), x2[ln].data(), d.n_embd * 4);
            oxo_rms_norm_mul_f32(ts.xin[ln].data(), normw.data(), ts.xn[ln].data(), d.n_embd, d.rms_eps);
            oxo_quantize_row_q8_0(ts.xn[ln].data(), d.n_embd, ts.xq[ln].data(), ts.xd[ln].data());
        }
    }

    // RecMix (engine.rs:2394-2570): key heads [kh0, kh1) of this thread, their value heads
    void p_rec_mix(TS &ts, int tid, int nt, int l, int nl, const uint32_t *toks) {
        Layer &L = layers[l];
        p_entry(ts, l, nl, toks, L.attn_norm);
        const int64_t ds = d.ssm_d_state, nk = d.ssm_n_kheads, nv = d.ssm_n_vheads, hv = d.ssm_d_inner / nv;
        const int64_t kc = d.ssm_conv_kernel, vpk = nv / nk;
        int64_t kh0, kh1;
        split(nk, nt, tid, kh0, kh1);
        if (kh1 <= kh0) return;
        std::vector<std::pair<int64_t, int64_t>> rg;
        rg.push_back({kh0 * ds, kh1 * ds});
        rg.push_back({nk * ds + kh0 * ds, nk * ds + kh1 * ds});
        for (int64_t m = 0; m < vpk; m++) rg.push_back({2 * nk * ds + (kh0 + m * nk) * hv, 2 * nk * ds + (kh1 + m * nk) * hv});
        for (auto &r : rg) rows_of(L.qkv, r.first, r.second, nl, ts.xq, ts.xd, [&](int ln) { return ts.qkv[ln].data() + r.first; });
        for (int64_t m = 0; m < vpk; m++) {
            const int64_t v0 = kh0 + m * nk, v1 = kh1 + m * nk;
            rows_of(L.z, v0 * hv, v1 * hv, nl, ts.xq, ts.xd, [&](int ln) { return ts.z[ln].data() + v0 * hv; });
            rows_of(L.beta, v0, v1, nl, ts.xq, ts.xd, [&](int ln) { return ts.beta[ln].data() + v0; });
            rows_of(L.alpha, v0, v1, nl, ts.xq, ts.xd, [&](int ln) { return ts.alpha[ln].data() + v0; });
        }
        const int ri = L.index;
        for (int ln = 0; ln < nl; ln++) {
            const int dst = (cur_slot + ln) % n_slots;
            const int src = ln == 0 ? dst : (cur_slot + ln - 1) % n_slots;
            float *cs = conv_state.data() + ((size_t)dst * n_rec + ri) * conv_len;
            const float *cs_src = conv_state.data() + ((size_t)src * n_rec + ri) * conv_len;
            float *cv = ts.conv[ln].data();
            for (auto &r : rg) {
                if (src != dst) std::memcpy(cs + r.first * (kc - 1), cs_src + r.first * (kc - 1), (r.second - r.first) * (kc - 1) * 4);
                oxo_ssm_conv_step_f32(cs + r.first * (kc - 1), ts.qkv[ln].data() + r.first, L.conv.data() + r.first * kc,
                                      (int)(r.second - r.first), (int)kc, cv + r.first);
                oxo_silu_f32((int)(r.second - r.first), ts.tmp.data(), cv + r.first);
                std::memcpy(cv + r.first, ts.tmp.data(), (r.second - r.first) * 4);
            }
            for (int64_t g = kh0; g < kh1; g++) {
                oxo_gdn_l2_norm_f32(cv + g * ds, ds, d.rms_eps);
                oxo_gdn_l2_norm_f32(cv + nk * ds + g * ds, ds, d.rms_eps);
            }
            for (int64_t m = 0; m < vpk; m++)
                for (int64_t vh = kh0 + m * nk; vh < kh1 + m * nk; vh++) {
                    const float ab = ts.alpha[ln][vh] + L.dt[vh];
                    float sp;
                    oxo_softplus_f32(1, &sp, &ab);
                    ts.gate[vh] = sp * L.a[vh];
                    oxo_sigmoid_f32(1, &ts.beta_s[vh], &ts.beta[ln][vh]);
                }
            for (int64_t m = 0; m < vpk; m++)
                for (int64_t vh = kh0 + m * nk; vh < kh1 + m * nk; vh++) {
                    const int64_t kh = vh % nk;
                    float *st = ssm_state.data() + ((size_t)dst * n_rec + ri) * ssm_len + vh * hv * hv;
                    const float *s_in = ssm_state.data() + ((size_t)src * n_rec + ri) * ssm_len + vh * hv * hv;
                    oxo_gated_delta_net_step_f32_from(st, s_in, cv + kh * ds, cv + nk * ds + kh * ds, cv + 2 * nk * ds + vh * hv,
                                                      ts.gate[vh], ts.beta_s[vh], hv, ts.gdn.data());
                    oxo_rms_norm_mul_f32(ts.gdn.data(), L.ssm_norm.data(), ts.tmpn.data(), hv, d.rms_eps);
                    oxo_silu_f32((int)hv, ts.zs.data(), ts.z[ln].data() + vh * hv);
                    for (int64_t j = 0; j < hv; j++) o[ln][vh * hv + j] = ts.tmpn[j] * ts.zs[j];
                }
        }
    }
    // RecOut / AttnOut (engine.rs:2573-2609): this thread's rows of the output projection + residual
    void p_mix_out_lanes(TS &ts, int tid, int nt, int l, int nl, int64_t width) {
        int64_t r0, r1;
        split_rows(d.n_embd, nt, tid, r0, r1);
        if (r1 <= r0) return;
        for (int ln = 0; ln < nl; ln++) oxo_quantize_row_q8_0(o[ln].data(), width, ts.oq[ln].data(), ts.od[ln].data());
        rows_of(layers[l].out, r0, r1, nl, ts.oq, ts.od, [&](int ln) { return ts.dtmp[ln].data(); });
        for (int ln = 0; ln < nl; ln++)
            for (int64_t r = r0; r < r1; r++) x1[ln][r] = ts.dtmp[ln][r - r0] + ts.xin[ln][r];
    }
    // AttnQkv (engine.rs:2614-2705): query heads [qh0, qh1) (q + gate rows, q norm, RoPE), raw K
    // rows k_rows, V rows v_rows (the reversed split) into V^T at pos0 + lane
    void p_attn_qkv(TS &ts, int tid, int nt, int l, int nl, int64_t pos0, const uint32_t *toks, bool with_q) {
        Layer &L = layers[l];
        if (with_q) p_entry(ts, l, nl, toks, L.attn_norm);
        const int64_t hd = d.head_dim, nkv = d.n_head_kv;
        const int ai = L.index;
        if (with_q) {
            int64_t qh0, qh1;
            split(d.n_head, nt, tid, qh0, qh1);
            rows_of(L.wq, qh0 * 2 * hd, qh1 * 2 * hd, nl, ts.xq, ts.xd, [&](int ln) { return ts.qg[ln].data() + qh0 * 2 * hd; });
        }
        int64_t k0, k1, v0, v1;
        split_rows(nkv * hd, nt, tid, k0, k1);
        split_rows(nkv * hd, nt, nt - 1 - tid, v0, v1);
        rows_of(L.wk, k0, k1, nl, ts.xq, ts.xd, [&](int ln) { return p_kraw[ln].data() + k0; });
        if (v1 > v0) {
            rows_of(L.wv, v0, v1, nl, ts.xq, ts.xd, [&](int ln) { return ts.dtmp[ln].data(); });
            for (int ln = 0; ln < nl; ln++)
                for (int64_t r = v0; r < v1; r++)
                    vcache[((size_t)ai * nkv * hd + r) * v_stride + pos0 + ln] = oxo_f32_to_f16(ts.dtmp[ln][r - v0]);
        }
    }
    // write_k (engine.rs:2709-2745): the owners of query head kvh * group write K rows of every lane
    void p_write_k(TS &ts, int tid, int nt, int l, int nl, int64_t pos0) {
        Layer &L = layers[l];
        const int64_t hd = d.head_dim, nkv = d.n_head_kv, group = d.n_head / nkv;
        int64_t qh0, qh1;
        split(d.n_head, nt, tid, qh0, qh1);
        for (int64_t kvh = 0; kvh < nkv; kvh++) {
            if (kvh * group < qh0 || kvh * group >= qh1) continue;
            for (int ln = 0; ln < nl; ln++) {
                const int64_t p = pos0 + ln;
                oxo_rms_norm_mul_f32(p_kraw[ln].data() + kvh * hd, L.k_norm.data(), ts.kn.data(), hd, d.rms_eps);
                oxo_rope_neox_inplace(ts.kn.data(), d.n_rot, rope_tab.data() + p * d.n_rot);
                uint16_t *kr = kcache.data() + (((size_t)L.index * nkv + kvh) * n_ctx + p) * hd;
                for (int64_t i = 0; i < hd; i++) kr[i] = oxo_f32_to_f16(ts.kn[i]);
            }
        }
    }
    // AttnCore (engine.rs:2748-2830) after the K rows are written: query heads [qh0, qh1), every lane
    void p_attn_core(TS &ts, int tid, int nt, int l, int nl, int64_t pos0) {
        Layer &L = layers[l];
        const int64_t hd = d.head_dim, nkv = d.n_head_kv, group = d.n_head / nkv;
        const int ai = L.index;
        const float scale = 1.0f / sqrtf((float)hd);
        int64_t qh0, qh1;
        split(d.n_head, nt, tid, qh0, qh1);
        for (int ln = 0; ln < nl; ln++) {
            const int64_t p = pos0 + ln;
            const int n_kv = (int)padded_n_kv(p, n_ctx);
            for (int64_t h = qh0; h < qh1; h++) {
                oxo_rms_norm_mul_f32(ts.qg[ln].data() + h * 2 * hd, L.q_norm.data(), ts.q.data(), hd, d.rms_eps);
                oxo_rope_neox_inplace(ts.q.data(), d.n_rot, rope_tab.data() + p * d.n_rot);
                const int64_t kvh = h / group;
                const uint16_t *kb = kcache.data() + ((size_t)ai * nkv + kvh) * n_ctx * hd;
                const uint16_t *vb = vcache.data() + ((size_t)ai * nkv * hd + kvh * hd) * v_stride;
                oxo_attn_head_f16(ts.q.data(), kb, hd, kb + p * hd, vb, v_stride, n_kv, (int)p, (int)hd, scale, ts.aout.data());
                oxo_sigmoid_f32(hd, ts.gs.data(), ts.qg[ln].data() + h * 2 * hd + hd);
                for (int64_t j = 0; j < hd; j++) o[ln][h * hd + j] = ts.aout[j] * ts.gs[j];
            }
        }
    }
    // MoeRouter (engine.rs:3372-3410): router rows, the shared gate (every thread), shared gate/up rows
    void p_moe_router(TS &ts, int tid, int nt, int l, int nl) {
        Layer &L = layers[l];
        const int64_t E = d.n_embd;
        int64_t e0, e1, s0, s1;
        split(d.n_expert, nt, tid, e0, e1);
        split_rows(d.ff_shexp, nt, tid, s0, s1);
        for (int ln = 0; ln < nl; ln++) {
            oxo_rms_norm_mul_f32(x1[ln].data(), L.post_norm.data(), ts.xn[ln].data(), E, d.rms_eps);
            oxo_quantize_row_q8_0(ts.xn[ln].data(), E, ts.xq[ln].data(), ts.xd[ln].data());
            for (int64_t e = e0; e < e1; e++) p_router[ln][e] = oxo_vec_dot_f32((int)E, L.router.data() + e * E, ts.xn[ln].data());
            const float sgd = oxo_vec_dot_f32((int)E, L.shexp_gate.data(), ts.xn[ln].data());
            oxo_sigmoid_f32(1, &ts.sh_gate[ln], &sgd);
        }
        if (s1 > s0) {
            for (int ln = 0; ln < nl; ln++) {
                const int8_t *q[1] = {ts.xq[ln].data()};
                const uint16_t *dd[1] = {ts.xd[ln].data()};
                float *yg[1] = {ts.tmp.data()}, *yu[1] = {ts.tmp.data() + (s1 - s0)};
                gemv_rows(L.gate_sh.q.data(), L.gate_sh.d.data(), E, s0, s1, 1, q, dd, yg);
                gemv_rows(L.up_sh.q.data(), L.up_sh.d.data(), E, s0, s1, 1, q, dd, yu);
                oxo_swiglu_f32((int)(s1 - s0), p_hsh[ln].data() + s0, ts.tmp.data(), ts.tmp.data() + (s1 - s0));
            }
        }
    }
    // route (engine.rs:3414-3429), on every thread for every lane
    void p_route(TS &ts, int nl) {
        const int64_t NE = d.n_expert, K = d.n_expert_used;
        for (int ln = 0; ln < nl; ln++) {
            oxo_soft_max_f32((int)NE, ts.probs[ln].data(), p_router[ln].data(), 1.0f, nullptr, ts.wp.data());
            int tie = 0;
            oxo_argsort_top_k_f32(ts.probs[ln].data(), (int)NE, (int)K, ts.ids[ln].data(), ts.iscr.data(), &tie);
            for (int64_t j = 0; j < K; j++) ts.w[ln][j] = ts.probs[ln][ts.ids[ln][j]];
            float s = oxo_vec_sum_f32((int)K, ts.w[ln].data());
            s = std::max(std::min(s, INFINITY), 6.103515625e-5f);
            for (int64_t j = 0; j < K; j++) ts.w[ln][j] = ts.w[ln][j] / s;
        }
    }
    // Synthetic expert weights this run routes to and nothing has generated yet, made by the whole
    // team (rows split) before the units run; its time counts as generation, its barriers do not
    // count. Every thread sees the same list: the units are the same on every thread and nothing
    // generates experts between the previous barrier and the first one here.
    void p_gen_experts(TS &ts, int tid, int nt, int l) {
        Layer &L = layers[l];
        std::vector<uint32_t> miss;
        for (auto &u : ts.uni_u)
            if (u.second == 0 && !L.experts[u.first]) miss.push_back(u.first);
        if (miss.empty()) return;
        const auto t0 = std::chrono::steady_clock::now();
        pool->barrier(tid, false);
        if (tid == 0)
            for (uint32_t e : miss) {
                std::unique_ptr<Mat[]> m(new Mat[3]);
                const int64_t E = d.n_embd, F = d.ff_exp;
                const int64_t rk[3][2] = {{F, E}, {F, E}, {E, F}};
                for (int w = 0; w < 3; w++) {
                    m[w].rows = rk[w][0];
                    m[w].k = rk[w][1];
                    m[w].q.resize(rk[w][0] * rk[w][1]);
                    m[w].d.resize(rk[w][0] * rk[w][1] / 32);
                }
                L.experts[e] = std::move(m);
            }
        pool->barrier(tid, false);
        const int kinds[3] = {OXE_T_GATE_EXPS, OXE_T_UP_EXPS, OXE_T_DOWN_EXPS};
        for (uint32_t e : miss)
            for (int w = 0; w < 3; w++) {
                Mat &m = L.experts[e][w];
                int64_t r0, r1;
                split(m.rows, nt, tid, r0, r1);
                gen_q8_rows(seed, l, kinds[w], m.rows, m.k, e, r0, r1, m);
            }
        pool->barrier(tid, false);
        if (tid == 0) gen_seconds += std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
    }
    // MoeGateUp (engine.rs:3437-3539): units (expert, 256-row block); several lanes: the union of
    // the lanes' experts in lane-major first use, split evenly, each unit for every lane that routed there
    void p_moe_gate_up(TS &ts, int tid, int nt, int l, int nl) {
        const int64_t E = d.n_embd, F = d.ff_exp, K = d.n_expert_used, bpe = F / 256;
        p_route(ts, nl);
        ts.uni_u.clear();
        ts.uni_e.clear();
        if (nl == 1) {
            for (int64_t j = 0; j < K; j++)
                for (int64_t b = 0; b < bpe; b++) ts.uni_u.push_back({(uint32_t)ts.ids[0][j], (uint32_t)b});
        } else {
            for (int ln = 0; ln < nl; ln++)
                for (int64_t j = 0; j < K; j++) {
                    const uint32_t e = (uint32_t)ts.ids[ln][j];
                    if (std::find(ts.uni_e.begin(), ts.uni_e.end(), e) == ts.uni_e.end()) {
                        ts.uni_e.push_back(e);
                        for (int64_t b = 0; b < bpe; b++) ts.uni_u.push_back({e, (uint32_t)b});
                    }
                }
        }
        p_gen_experts(ts, tid, nt, l);
        int64_t u0, u1;
        split((int64_t)ts.uni_u.size(), nt, tid, u0, u1);
        for (int64_t uu = u0; uu < u1; uu++) {
            const uint32_t e = ts.uni_u[uu].first;
            const int64_t b = ts.uni_u[uu].second;
            const Mat &wg = expert(l, (int)e, 0), &wu = expert(l, (int)e, 1);
            for (int ln = 0; ln < nl; ln++) {
                int64_t j = -1;
                for (int64_t i = 0; i < K; i++)
                    if ((uint32_t)ts.ids[ln][i] == e) { j = i; break; }
                if (j < 0) continue;
                const int8_t *q[1] = {ts.xq[ln].data()};
                const uint16_t *dd[1] = {ts.xd[ln].data()};
                float *yg[1] = {ts.g.data()}, *yu[1] = {ts.u.data()};
                gemv_rows(wg.q.data(), wg.d.data(), E, b * 256, (b + 1) * 256, 1, q, dd, yg);
                gemv_rows(wu.q.data(), wu.d.data(), E, b * 256, (b + 1) * 256, 1, q, dd, yu);
                const int64_t off = j * F + b * 256;
                oxo_swiglu_f32(256, p_h[ln].data() + off, ts.g.data(), ts.u.data());
                oxo_quantize_row_q8_0(p_h[ln].data() + off, 256, p_hq[ln].data() + off, p_hd[ln].data() + off / 32);
            }
        }
        for (int64_t b = 0; b < d.ff_shexp / 256; b++)
            if (nt - 1 - (int)(b % nt) == tid)
                for (int ln = 0; ln < nl; ln++)
                    oxo_quantize_row_q8_0(p_hsh[ln].data() + b * 256, 256, p_hshq[ln].data() + b * 256, p_hshd[ln].data() + b * 8);
    }
    // MoeDown (engine.rs:3542-3625): this thread's output rows of every routed expert and the shared
    // expert, combined in the reference's order, + residual
    void p_moe_down(TS &ts, int tid, int nt, int l, int nl) {
        Layer &L = layers[l];
        const int64_t E = d.n_embd, F = d.ff_exp, K = d.n_expert_used;
        int64_t r0, r1;
        split_rows(E, nt, tid, r0, r1);
        const int64_t nr = r1 - r0;
        if (nr <= 0) return;
        for (int ln = 0; ln < nl; ln++) {
            float *dt = ts.dtmp[ln].data();
            for (int64_t j = 0; j < K; j++) {
                const Mat &wdn = expert(l, ts.ids[ln][j], 2);
                const int8_t *q[1] = {p_hq[ln].data() + j * F};
                const uint16_t *dd[1] = {p_hd[ln].data() + j * F / 32};
                float *y[1] = {dt + j * nr};
                gemv_rows(wdn.q.data(), wdn.d.data(), F, r0, r1, 1, q, dd, y);
            }
            const int8_t *q[1] = {p_hshq[ln].data()};
            const uint16_t *dd[1] = {p_hshd[ln].data()};
            float *y[1] = {dt + K * nr};
            gemv_rows(L.down_sh.q.data(), L.down_sh.d.data(), d.ff_shexp, r0, r1, 1, q, dd, y);
            const float sg = ts.sh_gate[ln];
            for (int64_t i = 0; i < nr; i++) {
                float m = dt[i] * ts.w[ln][0];
                for (int64_t j = 1; j < K; j++) {
                    const float pp = dt[j * nr + i] * ts.w[ln][j];
                    m = m + pp;
                }
                const float sh = dt[K * nr + i] * sg;
                const float f = m + sh;
                x2[ln][r0 + i] = f + x1[ln][r0 + i];
            }
        }
    }
    // Head (engine.rs:3630-3715): this thread's vocabulary rows in chunks of 256, the first strict
    // maximum per lane; thread 0 keeps the normed hidden state
    void p_head(TS &ts, int tid, int nt, int nl, uint32_t mask, const std::vector<float> &norm, bool draft = false) {
        const bool restricted = draft && !draft_ids.empty();
        const int64_t E = d.n_embd, V = d.n_vocab;
        int64_t r0, r1;
        split_rows(V, nt, tid, r0, r1);
        for (int ln = 0; ln < nl; ln++) {
            oxo_rms_norm_mul_f32(x2[ln].data(), norm.data(), ts.xn[ln].data(), E, d.rms_eps);
            if (tid == 0) std::memcpy(hout[ln].data(), ts.xn[ln].data(), E * 4);
            std::pair<float, uint32_t> b{-INFINITY, UINT32_MAX};
            if (mask & (1u << ln)) {
                oxo_quantize_row_q8_0(ts.xn[ln].data(), E, ts.xq[ln].data(), ts.xd[ln].data());
                for (int64_t r = r0; r < r1; r += 256) {
                    const int64_t c = std::min<int64_t>(256, r1 - r);
                    const int8_t *q[1] = {ts.xq[ln].data()};
                    const uint16_t *dd[1] = {ts.xd[ln].data()};
                    float *y[1] = {ts.tmp.data()};
                    gemv_rows(output.q.data(), output.d.data(), E, r, r + c, 1, q, dd, y);
                    for (int64_t i = 0; i < c; i++)
                        if (ts.tmp[i] > b.first && (!restricted || draft_mask[r + i])) b = {ts.tmp[i], (uint32_t)(r + i)};
                    if (keep_logits) std::memcpy(logits[ln].data() + r, ts.tmp.data(), c * 4);
                }
            }
            p_best[ln][tid] = b;
        }
    }
    void p_gather_argmax(int nl) {
        for (int ln = 0; ln < nl; ln++) {
            std::pair<float, uint32_t> b{-INFINITY, UINT32_MAX};
            for (auto &t : p_best[ln])
                if (t.first > b.first) b = t;
            argmax[ln] = b.second == UINT32_MAX ? 0 : b.second;
        }
    }
    // the MoE phases of layer l (three barriers)
    void p_moe(TS &ts, int tid, int nt, int l, int nl) {
        p_moe_router(ts, tid, nt, l, nl);
        pool->barrier(tid);
        p_moe_gate_up(ts, tid, nt, l, nl);
        pool->barrier(tid);
        p_moe_down(ts, tid, nt, l, nl);
        pool->barrier(tid);
    }
    // the attention layer's mixer phases (AttnQkv, AttnCore with write_k + its inner barrier, AttnOut)
    void p_attention(TS &ts, int tid, int nt, int l, int nl, int64_t pos0, const uint32_t *toks) {
        p_attn_qkv(ts, tid, nt, l, nl, pos0, toks, true);
        pool->barrier(tid);
        p_write_k(ts, tid, nt, l, nl, pos0);
        pool->barrier(tid);
        p_attn_core(ts, tid, nt, l, nl, pos0);
        pool->barrier(tid);
        p_mix_out_lanes(ts, tid, nt, l, nl, d.n_head * d.head_dim);
        pool->barrier(tid);
    }
    int verify_plan(const uint32_t *toks, int n, uint32_t *out) {
        pend_pos0 = pos;
        pend_cur = cur_slot;
        pend_n = n;
        pend_done = 0;
        const int nt = pool->n;
        const int64_t p0 = pos;
        std::function<void(int)> job = [&](int tid) {
            TS &ts = pts[tid];
            for (int l = 0; l < d.n_layer; l++) {
                if (layers[l].att) {
                    p_attention(ts, tid, nt, l, n, p0, toks);
                } else {
                    p_rec_mix(ts, tid, nt, l, n, toks);
                    pool->barrier(tid);
                    p_mix_out_lanes(ts, tid, nt, l, n, d.ssm_d_inner);
                    pool->barrier(tid);
                }
                p_moe(ts, tid, nt, l, n);
            }
            p_head(ts, tid, nt, n, (1u << n) - 1, out_norm);
        };
        pool->run(job);
        p_gather_argmax(n);
        for (int ln = 0; ln < n; ln++) out[ln] = argmax[ln];
        return 0;
    }
    // MtpEntry (engine.rs:2362-2390) as its own phase: eh_proj rows of this thread for every lane
    void p_mtp_entry(TS &ts, int tid, int nt, int nl, const uint32_t *toks) {
        Layer &L = layers[d.n_layer];
        const int64_t E = d.n_embd;
        int64_t r0, r1;
        split_rows(E, nt, tid, r0, r1);
        for (int ln = 0; ln < nl; ln++) {
            std::vector<float> e = embed(toks[ln]);
            oxo_rms_norm_mul_f32(e.data(), L.enorm.data(), ts.cat[ln].data(), E, d.rms_eps);
            oxo_rms_norm_mul_f32(hin[ln].data(), L.hnorm.data(), ts.cat[ln].data() + E, E, d.rms_eps);
            oxo_quantize_row_q8_0(ts.cat[ln].data(), 2 * E, ts.xq[ln].data(), ts.xd[ln].data());
        }
        rows_of(L.eh_proj, r0, r1, nl, ts.xq, ts.xd, [&](int ln) { return x2[ln].data() + r0; });
    }
    uint32_t mtp_run_plan(const uint32_t *toks, int n, int64_t pos0, int head_last) {
        const int l = d.n_layer, nt = pool->n;
        std::function<void(int)> job = [&](int tid) {
            TS &ts = pts[tid];
            p_mtp_entry(ts, tid, nt, n, toks);
            pool->barrier(tid);
            p_attention(ts, tid, nt, l, n, pos0, toks);
            p_moe(ts, tid, nt, l, n);
            p_head(ts, tid, nt, n, head_last ? 1u << (n - 1) : 0u, layers[l].head_norm, true);
        };
        pool->run(job);
        p_gather_argmax(n);
        return head_last ? argmax[n - 1] : UINT32_MAX;
    }
    void mtp_seed_plan(const uint32_t *toks, int n, int64_t pos0) {
        const int l = d.n_layer, nt = pool->n;
        std::function<void(int)> job = [&](int tid) {
            TS &ts = pts[tid];
            p_mtp_entry(ts, tid, nt, n, toks);
            pool->barrier(tid);
            for (int ln = 0; ln < n; ln++) {
                oxo_rms_norm_mul_f32(x2[ln].data(), layers[l].attn_norm.data(), ts.xn[ln].data(), d.n_embd, d.rms_eps);
                oxo_quantize_row_q8_0(ts.xn[ln].data(), d.n_embd, ts.xq[ln].data(), ts.xd[ln].data());
            }
            p_attn_qkv(ts, tid, nt, l, n, pos0, toks, false);
            pool->barrier(tid);
            p_write_k(ts, tid, nt, l, n, pos0);
        };
        pool->run(job);
    }

    int verify(const uint32_t *toks, int n, uint32_t *out) {
        if (n < 1 || n > n_slots || pos + n > n_ctx) return -1;
        if (pool) return verify_plan(toks, n, out);
        pend_pos0 = pos;
        pend_cur = cur_slot;
        pend_n = n;
        pend_done = 0;
        for (int l = 0; l < d.n_layer; l++) run_layer(l, n, pos, toks);
        head(n, (1u << n) - 1, out_norm);
        for (int ln = 0; ln < n; ln++) out[ln] = argmax[ln];
        return 0;
    }

    void zero_v(int64_t a, int64_t b) {
        if (b <= a) return;
        const int64_t rows = (int64_t)(n_att - (d.has_mtp ? 1 : 0)) * d.n_head_kv * d.head_dim;
        for (int64_t r = 0; r < rows; r++)
            for (int64_t p = a; p < b; p++) vcache[(size_t)r * v_stride + p] = 0;
    }

    int commit(int m) {
        if (pend_n == 0) return -1;
        const int hi = pend_done == 0 ? pend_n : pend_done;
        if (m < 1 || m > hi) return -1;
        zero_v(pend_pos0 + m, pend_pos0 + hi);
        pos = pend_pos0 + m;
        cur_slot = (pend_cur + m - 1) % n_slots;
        pend_done = m;
        return 0;
    }

    // mtp_entry (engine.rs:2362-2390): x2 = eh_proj . [enorm(embd(tok)); hnorm(h)]
    void mtp_entry(int nl, const uint32_t *toks) {
        Layer &L = layers[d.n_layer];
        const int64_t E = d.n_embd;
        std::vector<std::vector<float>> cat(nl, std::vector<float>(2 * E));
        std::vector<const float *> xs;
        std::vector<float *> ys;
        for (int ln = 0; ln < nl; ln++) {
            std::vector<float> e = embed(toks[ln]);
            oxo_rms_norm_mul_f32(e.data(), L.enorm.data(), cat[ln].data(), E, d.rms_eps);
            oxo_rms_norm_mul_f32(hin[ln].data(), L.hnorm.data(), cat[ln].data() + E, E, d.rms_eps);
            xs.push_back(cat[ln].data());
            ys.push_back(x2[ln].data());
        }
        mv(L.eh_proj, xs, ys);
    }

    uint32_t mtp_run(const uint32_t *toks, int n, int64_t pos0, const float *hs, int head_last) {
        const int l = d.n_layer;
        for (int ln = 0; ln < n; ln++) std::memcpy(hin[ln].data(), hs + ln * d.n_embd, d.n_embd * 4);
        if (pool) return mtp_run_plan(toks, n, pos0, head_last);
        mtp_entry(n, toks);
        for (int ln = 0; ln < n; ln++) xin[ln] = x2[ln];
        attention(l, n, pos0);
        moe(l, n);
        head(n, head_last ? 1u << (n - 1) : 0u, layers[l].head_norm, true);
        return head_last ? argmax[n - 1] : UINT32_MAX;
    }

    // mtp_seed (engine.rs:2077-2091, 2121-2136): entry + attn_norm + K/V rows only
    void mtp_seed(const uint32_t *toks, int n, int64_t pos0, const float *hs) {
        const int l = d.n_layer;
        for (int ln = 0; ln < n; ln++) std::memcpy(hin[ln].data(), hs + ln * d.n_embd, d.n_embd * 4);
        if (pool) {
            mtp_seed_plan(toks, n, pos0);
            return;
        }
        mtp_entry(n, toks);
        std::vector<std::vector<float>> xn(n, std::vector<float>(d.n_embd));
        for (int ln = 0; ln < n; ln++)
            oxo_rms_norm_mul_f32(x2[ln].data(), layers[l].attn_norm.data(), xn[ln].data(), d.n_embd, d.rms_eps);
        attn_kv(l, n, pos0, xn);
    }
};

// ---- MtpDriver (crates/model/src/mtp.rs:314-608), depth 1..
struct oxo_driver {
    oxo_engine *eng = nullptr;
    int depth = 1;
    int64_t q = 0;
    std::vector<uint32_t> cu_tok;
    std::vector<float> cu_h;
    std::vector<float> hl;
    int64_t steps = 0, drafted = 0, accepted = 0, tokens_out = 0;
    int64_t last_p0 = 0;
    int last_n = 0;                // MtpDriver.last (mtp.rs:336)
    std::vector<float> last_h;     // MtpDriver.last_h

    int mtp_lanes() const { return eng->max_lanes; }

    void remember(int64_t p0, int n) {
        last_p0 = p0;
        last_n = n;
        last_h.clear();
        for (int i = 0; i < n; i++) last_h.insert(last_h.end(), eng->hout[i].begin(), eng->hout[i].end());
    }

    void note(int64_t p0, const uint32_t *toks, int n) {
        const int64_t E = eng->d.n_embd;
        for (int i = 0; i < n; i++) {
            const int64_t p = p0 + i;
            if (p >= q) {
                cu_tok.push_back(toks[i]);
                if (i == 0) cu_h.insert(cu_h.end(), hl.begin(), hl.end());
                else cu_h.insert(cu_h.end(), eng->hout[i - 1].begin(), eng->hout[i - 1].end());
            }
        }
        hl = eng->hout[n - 1];
        (void)E;
    }

    void flush(size_t keep) {
        const int64_t E = eng->d.n_embd;
        while (cu_tok.size() > keep) {
            const int n = (int)std::min<size_t>(mtp_lanes(), cu_tok.size());
            eng->mtp_seed(cu_tok.data(), n, q, cu_h.data());
            cu_tok.erase(cu_tok.begin(), cu_tok.begin() + n);
            cu_h.erase(cu_h.begin(), cu_h.begin() + n * E);
            q += n;
        }
    }

    uint32_t prefill(const uint32_t *toks, int n) {
        uint32_t next = UINT32_MAX;
        for (int c0 = 0; c0 < n; c0 += eng->n_slots) {
            const int c = std::min(eng->n_slots, n - c0);
            const int64_t p0 = eng->pos;
            uint32_t g[8];
            eng->verify(toks + c0, c, g);
            eng->commit(c);
            next = g[c - 1];
            note(p0, toks + c0, c);
            flush(mtp_lanes() - 1);
        }
        return next;
    }

    // MtpDriver::step (mtp.rs:522-592); force[i] >= 0 (i < nforce) replaces draft i after the draft
    // chain is formed, as the reference's draft_override hook does (mtp.rs:554-558)
    int step(uint32_t x, uint32_t *out, int64_t override_d1) { return step_force(x, out, &override_d1, 1); }
    int step_force(uint32_t x, uint32_t *out, const int64_t *force, int nforce) {
        const int64_t p = eng->pos;
        const int64_t k = std::min<int64_t>(depth, std::max<int64_t>(0, eng->n_ctx - (p + 1)));
        flush(mtp_lanes() - 1);
        if (k == 0) {
            uint32_t g[8];
            eng->verify(&x, 1, g);
            eng->commit(1);
            note(p, &x, 1);
            remember(p, 1);
            out[0] = g[0];
            return 1;
        }
        flush(0);
        uint32_t drafts[8];
        drafts[0] = eng->mtp_run(&x, 1, p, hl.data(), 1);
        q = p + 1;
        std::vector<float> h = eng->hout[0];
        for (int64_t i = 1; i < k; i++) {
            drafts[i] = eng->mtp_run(&drafts[i - 1], 1, p + i, h.data(), 1);
            h = eng->hout[0];
        }
        for (int64_t i = 0; i < k && i < nforce; i++)
            if (force[i] >= 0) drafts[i] = (uint32_t)force[i];
        uint32_t vt[8];
        vt[0] = x;
        for (int64_t i = 0; i < k; i++) vt[1 + i] = drafts[i];
        uint32_t g[8];
        eng->verify(vt, (int)k + 1, g);
        int a = 0;
        while (a < k && drafts[a] == g[a]) a++;
        eng->commit(a + 1);
        note(p, vt, a + 1);
        remember(p, a + 1);
        steps++;
        drafted += k;
        accepted += a;
        tokens_out += a + 1;
        for (int i = 0; i <= a; i++) out[i] = g[i];
        return a + 1;
    }

    // MtpDriver::step_plain (mtp.rs:504-515)
    uint32_t step_plain(uint32_t x) {
        const int64_t p = eng->pos;
        uint32_t g[8];
        eng->verify(&x, 1, g);
        eng->commit(1);
        note(p, &x, 1);
        remember(p, 1);
        flush(mtp_lanes() - 1);
        return g[0];
    }

    // MtpDriver::rewind (mtp.rs:596-608)
    int rewind(int m) {
        if (last_n == 0 || m < 1 || m > last_n) return -1;
        if (m == last_n) return 0;
        eng->commit(m);
        const int64_t E = eng->d.n_embd;
        const size_t keep = std::min<size_t>((size_t)std::max<int64_t>(0, last_p0 + m - q), cu_tok.size());
        cu_tok.resize(keep);
        cu_h.resize(keep * E);
        hl.assign(last_h.begin() + (m - 1) * E, last_h.begin() + m * E);
        last_n = m;
        return 0;
    }
};

extern "C" {

oxo_engine *oxo_engine_new(const oxe_model_desc *d, uint64_t seed, int64_t n_ctx) {
    oxo_engine *e = new oxo_engine();
    e->init(*d, seed, n_ctx);
    return e;
}
// n_slots recurrent slots = verify lanes (the reference's verify width for MTP depth n_slots - 1)
oxo_engine *oxo_engine_new_lanes(const oxe_model_desc *d, uint64_t seed, int64_t n_ctx, int n_slots) {
    if (n_slots < 1 || n_slots > 8) return nullptr;
    oxo_engine *e = new oxo_engine();
    e->n_slots = n_slots;
    e->init(*d, seed, n_ctx);
    return e;
}
// with each matrix's ggml type from types[layer * 64 + kind] (layer OXE_GLOBAL_LAYER: the global
// tensors): Q8_0 (8) anywhere; K-quants (11..14) anywhere but the MTP entry's eh_proj; F32 (0) for
// ssm_beta / ssm_alpha. Null for another combination.
oxo_engine *oxo_engine_new_typed(const oxe_model_desc *d, uint64_t seed, int64_t n_ctx, int n_slots, const int32_t *types) {
    if (n_slots < 1 || n_slots > 8 || !types) return nullptr;
    oxo_engine *e = new oxo_engine();
    e->n_slots = n_slots;
    for (int l = 0; l < 64; l++)
        for (int k = 0; k < 64; k++) {
            const int32_t t = types[l * 64 + k];
            if (!oxe_kind_is_q8(k)) continue;
            const bool kq = t >= 11 && t <= 14, ok = t == 8 || (kq && k != OXE_T_EH_PROJ) ||
                (t == 0 && (k == OXE_T_DN_BETA || k == OXE_T_DN_ALPHA));
            if (!ok) {
                delete e;
                return nullptr;
            }
            e->types[(size_t)l * 64 + k] = t;
            e->typed |= t != 8;
        }
    e->init(*d, seed, n_ctx);
    return e;
}
void oxo_engine_free(oxo_engine *e) { delete e; }
void oxo_engine_reset(oxo_engine *e) { e->reset(); }
int oxo_verify(oxo_engine *e, const uint32_t *toks, int n, uint32_t *out) { return e->verify(toks, n, out); }
int oxo_commit(oxo_engine *e, int m) { return e->commit(m); }
uint32_t oxo_step(oxo_engine *e, uint32_t tok) {
    uint32_t g[8];
    if (e->verify(&tok, 1, g) != 0) return UINT32_MAX;
    e->commit(1);
    return g[0];
}
uint32_t oxo_mtp_run(oxo_engine *e, const uint32_t *toks, int n, int64_t pos0, const float *hs, int head_last) {
    return e->mtp_run(toks, n, pos0, hs, head_last);
}
void oxo_mtp_seed(oxo_engine *e, const uint32_t *toks, int n, int64_t pos0, const float *hs) { e->mtp_seed(toks, n, pos0, hs); }
int64_t oxo_pos(const oxo_engine *e) { return e->pos; }
int oxo_cur_slot(const oxo_engine *e) { return e->cur_slot; }
int oxo_tie_count(const oxo_engine *e) { return e->tie_count; }
const float *oxo_hidden(const oxo_engine *e, int lane) { return e->hout[lane].data(); }
const float *oxo_logits(const oxo_engine *e, int lane) { return e->logits[lane].data(); }
int64_t oxo_n_ctx(const oxo_engine *e) { return e->n_ctx; }
void oxo_set_keep_logits(oxo_engine *e, int on) { e->keep_logits = on != 0; }
double oxo_gen_seconds(const oxo_engine *e) { return e->gen_seconds; }
// Runs from now on go through the reference's static plan on a pinned team of `nthreads` threads
// (at most the CPUs of the caller's mask; the caller is thread 0 and is pinned to the first of
// them until the plan is dropped); 0 drops the plan and its team. Returns the team size, 0, or -1.
int oxo_set_plan(oxo_engine *e, int nthreads) { return e->set_plan(nthreads); }
// the restricted draft head's ids (below n_vocab, sorted, unique); n = 0 restores the whole head.
// Returns the ids kept, or -1 when none is below n_vocab
int oxo_set_draft_vocab(oxo_engine *e, const uint32_t *ids, int n) { return e->set_draft_vocab(ids, n); }
// barrier episodes of the plan's team so far (the reference's barriers/token counter)
int64_t oxo_plan_barriers(const oxo_engine *e) { return e->pool ? (int64_t)e->pool->episodes.load() : -1; }

// Pin the OpenMP team the way the reference's worker pool is pinned (crates/sched/src/lib.rs:1-11,
// 137-147, 233-249): team thread i on the i-th CPU of the calling thread's affinity set, the caller
// (thread 0) included, its previous mask kept and restored by oxo_pin_team(0). libgomp keeps the
// team's threads alive between parallel regions, so the pinned threads serve every later region of
// the same size. Returns the team size pinned (0 after unpinning), or -1 if a mask call failed.
namespace {
cpu_set_t g_caller_mask;
bool g_pinned = false;
}  // namespace

int oxo_pin_team(int on) {
    if (!on) {
        if (!g_pinned) return 0;
        int bad = 0;
#pragma omp parallel reduction(+ : bad)
        bad += sched_setaffinity(0, sizeof(cpu_set_t), &g_caller_mask) != 0;
        g_pinned = false;
        return bad ? -1 : 0;
    }
    cpu_set_t mask;
    CPU_ZERO(&mask);
    if (sched_getaffinity(0, sizeof(cpu_set_t), &mask) != 0) return -1;
    std::vector<int> cpus;
    for (int c = 0; c < CPU_SETSIZE; c++)
        if (CPU_ISSET(c, &mask)) cpus.push_back(c);
    if (cpus.empty()) return -1;
    if (!g_pinned) g_caller_mask = mask;
    int bad = 0, team = 0;
#pragma omp parallel reduction(+ : bad)
    {
        const int t = omp_get_thread_num();
        if (t == 0) team = omp_get_num_threads();
        cpu_set_t one;
        CPU_ZERO(&one);
        CPU_SET(cpus[t % cpus.size()], &one);
        bad += sched_setaffinity(0, sizeof(cpu_set_t), &one) != 0;
    }
    g_pinned = true;
    return bad ? -1 : team;
}

// raw state views for parity checks: K cache [att][kvh][n_ctx][hd] f16, V^T [att][kvh*hd][n_ctx] f16,
// conv [slot][rec][(kc-1)*channels], S [slot][rec][nv][hv][hv]
const uint16_t *oxo_kcache(const oxo_engine *e) { return e->kcache.data(); }
const uint16_t *oxo_vcache(const oxo_engine *e) { return e->vcache.data(); }
float *oxo_conv_state(oxo_engine *e) { return e->conv_state.data(); }
float *oxo_ssm_state(oxo_engine *e) { return e->ssm_state.data(); }
uint16_t *oxo_kcache_mut(oxo_engine *e) { return e->kcache.data(); }
uint16_t *oxo_vcache_mut(oxo_engine *e) { return e->vcache.data(); }
void oxo_set_pos(oxo_engine *e, int64_t pos) { e->pos = pos; }

// one mixer + MoE layer for parity of configs 2/3: x[nl][E] is the layer input, x2 out
void oxo_mixer(oxo_engine *e, int l, int nl, int64_t pos0, const float *x, float *out) {
    for (int ln = 0; ln < nl; ln++) std::memcpy(e->xin[ln].data(), x + ln * e->d.n_embd, e->d.n_embd * 4);
    if (e->layers[l].att) e->attention(l, nl, pos0);
    else e->recurrent(l, nl);
    for (int ln = 0; ln < nl; ln++) std::memcpy(out + ln * e->d.n_embd, e->x1[ln].data(), e->d.n_embd * 4);
}
// router rows [row0, row0 + nrows) of layer l replaced (test hook for exact routing ties)
void oxo_engine_set_router(oxo_engine *e, int l, int row0, int nrows, const float *src) {
    std::memcpy(e->layers[l].router.data() + (size_t)row0 * e->d.n_embd, src, (size_t)nrows * e->d.n_embd * 4);
}
// the MTP entry alone (engine.rs:2362-2390): x[nl][E] = eh_proj . [enorm(embd(tok)); hnorm(h)]
void oxo_mtp_entry(oxo_engine *e, const uint32_t *toks, int nl, const float *hs, float *x) {
    for (int ln = 0; ln < nl; ln++) std::memcpy(e->hin[ln].data(), hs + ln * e->d.n_embd, e->d.n_embd * 4);
    e->mtp_entry(nl, toks);
    for (int ln = 0; ln < nl; ln++) std::memcpy(x + ln * e->d.n_embd, e->x2[ln].data(), e->d.n_embd * 4);
}
void oxo_moe(oxo_engine *e, int l, int nl, const float *x1, float *x2) {
    for (int ln = 0; ln < nl; ln++) std::memcpy(e->x1[ln].data(), x1 + ln * e->d.n_embd, e->d.n_embd * 4);
    e->moe(l, nl);
    for (int ln = 0; ln < nl; ln++) std::memcpy(x2 + ln * e->d.n_embd, e->x2[ln].data(), e->d.n_embd * 4);
}

oxo_driver *oxo_driver_new(oxo_engine *e, int depth) {
    oxo_driver *d = new oxo_driver();
    d->eng = e;
    d->depth = depth;
    d->q = e->pos;
    d->hl.assign(e->d.n_embd, 0.0f);
    return d;
}
void oxo_driver_free(oxo_driver *d) { delete d; }
// a driver state imported from elsewhere (MtpDriver::import_state with no pending pairs): the MTP
// head's KV seeded below q, h_{P-1} = hl
void oxo_driver_import(oxo_driver *d, int64_t q, const float *hl) {
    d->q = q;
    d->cu_tok.clear();
    d->cu_h.clear();
    d->hl.assign(hl, hl + d->eng->d.n_embd);
}
// the engine's state in Engine::write_state's byte order (K rows, V^T rows per attention layer, then
// the current slot's conv state and S) for n_pos positions; the position becomes n_pos
int oxo_engine_read_state(oxo_engine *e, const uint8_t *buf, int64_t nbytes, int64_t n_pos) {
    const int64_t hd = e->d.head_dim, nkv = e->d.n_head_kv;
    const int64_t need = (int64_t)e->n_att * nkv * 2 * hd * 2 * n_pos + (e->conv_len + e->ssm_len) * e->n_rec * 4;
    if (n_pos < 0 || n_pos > e->n_ctx || nbytes != need) return -1;
    const uint8_t *p = buf;
    for (int a = 0; a < e->n_att; a++) {
        for (int64_t h = 0; h < nkv; h++) {
            std::memcpy(e->kcache.data() + ((size_t)(a * nkv + h) * e->n_ctx) * hd, p, (size_t)n_pos * hd * 2);
            p += n_pos * hd * 2;
        }
        for (int64_t r = 0; r < nkv * hd; r++) {
            std::memcpy(e->vcache.data() + ((size_t)a * nkv * hd + r) * e->v_stride, p, (size_t)n_pos * 2);
            p += n_pos * 2;
        }
    }
    std::memcpy(e->conv_state.data() + (size_t)e->cur_slot * e->n_rec * e->conv_len, p, (size_t)e->n_rec * e->conv_len * 4);
    p += e->n_rec * e->conv_len * 4;
    std::memcpy(e->ssm_state.data() + (size_t)e->cur_slot * e->n_rec * e->ssm_len, p, (size_t)e->n_rec * e->ssm_len * 4);
    e->pos = n_pos;
    e->pend_n = 0;
    return 0;
}
uint32_t oxo_driver_prefill(oxo_driver *d, const uint32_t *toks, int n) { return d->prefill(toks, n); }
int oxo_driver_step(oxo_driver *d, uint32_t x, uint32_t *out, int64_t override_d1) { return d->step(x, out, override_d1); }
int oxo_driver_step_force(oxo_driver *d, uint32_t x, uint32_t *out, const int64_t *force, int nforce) {
    return d->step_force(x, out, force, nforce);
}
void oxo_driver_stats(const oxo_driver *d, int64_t *st) {
    st[0] = d->steps; st[1] = d->drafted; st[2] = d->accepted; st[3] = d->tokens_out;
}
uint32_t oxo_driver_step_plain(oxo_driver *dr, uint32_t x) { return dr->step_plain(x); }
int oxo_driver_rewind(oxo_driver *dr, int m) { return dr->rewind(m); }

}  // extern "C"

extern "C" {
// Synthetic tensors of include/oxe_model.h on the host (inputs for parity tests).
void oxo_synth_q8(uint64_t seed, int layer, int kind, int64_t expert, int64_t rows, int64_t k, int8_t *q, uint16_t *d) {
    Mat m;
    gen_q8(seed, layer, kind, rows, k, expert, m);
    std::memcpy(q, m.q.data(), m.q.size());
    std::memcpy(d, m.d.data(), m.d.size() * 2);
}
void oxo_synth_f32(uint64_t seed, int layer, int kind, int64_t n, float *out) {
    std::vector<float> v = gen_f32(seed, layer, kind, n);
    std::memcpy(out, v.data(), n * 4);
}
// mu + sigma * z with the Irwin-Hall z of the generator, under the key of (seed, uid)
void oxo_synth_normal(uint64_t seed, uint64_t uid, int64_t n, float mu, float sigma, float *out) {
    const uint64_t key = oxe_rng(seed, uid);
    for (int64_t i = 0; i < n; i++) {
        const float t = sigma * oxe_synth_z(key, (uint64_t)i);
        out[i] = mu + t;
    }
}
}
