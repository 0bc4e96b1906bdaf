// Host-side engine object shared by engine.hip (run sequences, C ABI) and mtp.hip (MTP driver and
// the device-driven step).
#pragma once
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <stdexcept>
#include <string>
#include <vector>

#include "../../include/oxe_amd.h"
#include "oxe_engine.h"
#include "oxe_kernels.h"
#include "oxe_fused.h"
#include "oxe_model_kernels.h"
#include "oxe_shape.h"

#define OXE_HOST_DEV_INLINE __host__ __device__ inline

namespace oxe {

using namespace shp;

struct Engine;
struct Gguf;

// MtpDriver (crates/model/src/mtp.rs:314-608), host-driven, depth 1..MTP_MAX_DEPTH; dev_begin /
// dev_end hand its state to and from the device-driven step (depth 1 or 2).
constexpr int MTP_MAX_DEPTH = 3;
struct MtpDriverHost {
    int depth = 1;               // drafts per step (MtpDriver.depth)
    int q = 0;                   // MTP KV holds correct pairs for positions < q
    std::vector<uint32_t> cu_tok;  // pending catch-up pairs for positions q, q+1, ...
    std::vector<float> cu_h;
    std::vector<float> hl = std::vector<float>(shp::E, 0.0f);  // target h_nextn of position pos-1
    int64_t steps = 0, accepted = 0, drafted = 0;
    int last_p0 = 0, last_n = 0;   // the last host-driven step's committed span (MtpDriver.last)
    int last_cur0 = 0;             // the recurrent slot before that span
    std::vector<float> last_h;     // h_nextn of each committed lane of that step (MtpDriver.last_h)
    void note(Engine &e, int p0, const uint32_t *toks, int n);
    void note_h(int p0, const uint32_t *toks, int n, const float *h);
    void remember(Engine &e, int p0, int n);
    int flush(Engine &e, size_t keep);
    int prefill(Engine &e, const uint32_t *toks, int n, uint32_t *next);
    int prefill_batched(Engine &e, const uint32_t *toks, int n, uint32_t *next);
    int step(Engine &e, uint32_t x, uint32_t *out, int *n_out, int64_t override_d1);
    int step_k(Engine &e, uint32_t x, uint32_t *out, int *n_out, const int64_t *force, int nforce, float *rows);
    int step_plain(Engine &e, uint32_t x, uint32_t *out);
    int rewind(Engine &e, int m);
    int dev_begin(Engine &e, uint32_t x);
    int dev_end(Engine &e, uint32_t *out_tok, int cap, int *n_out, uint32_t *next_x);
};

// Buffers of the batched prefill, [T][...] for up to cap tokens (allocated on first use)
struct PfBufs {
    int cap = 0, max_tiles = 0, attn_lds = 0, attn_lds_gqa = 0;
    float *x, *x1, *xn, *hin, *proj, *cy, *gg, *gb, *o, *lg, *sg, *wts, *gu, *dout, *sh;
    int8_t *xq, *oq, *hq;
    uint16_t *xd, *od, *qh, *hd;
    int32_t *ids, *mo, *ptok, *pair_of;
    int4 *tiles;
    uint32_t *tok;
};
constexpr int PF_CHUNK = 2048;   // tokens per batched pass

// engine creation behind oxe_engine_create / _create_on / _create_from_gguf (engine.hip); mt: the
// matrices' types, Q8_0 everywhere when null
int create_engine(const oxe_model_desc *desc, uint64_t seed, int n_ctx, bool caller, void *stream, const ModelTypes *mt,
                  oxe_engine **out);

inline thread_local std::string g_last_error;
inline void set_err(const std::string &s) { g_last_error = s; }

struct Engine {
    oxe_model_desc d{};
    uint64_t seed = 0;
    int dev = 0;            // the device current at creation (every buffer and the stream live there)
    hipStream_t st = nullptr;
    bool own_stream = true; // st created by the engine (destroyed with it), else the caller's
    ModelRt m{};
    std::vector<LayerW> L;  // n_layer (+1 MTP block)
    ModelTypes types;       // the matrices' types
    bool kq = false;        // some matrix is not Q8_0: per-phase runs, token-by-token prefill
    ActBufs b{};
    RunCtl *ctl = nullptr;  // device
    // the device-driven step's draft control block (fused runs), filled by the previous step's
    // commit kernel or by dev_begin
    RunCtl *ctl_draft = nullptr;
    std::vector<void *> allocs;
    size_t bytes = 0;
    // host mirror of the engine position (host-driven API)
    int pos = 0, cur = 0;
    int pend_pos0 = 0, pend_cur = 0, pend_n = 0, pend_done = 0;
    int n_att_main = 0;
    bool keep_logits = true;
    // device-driven MTP step
    MtpDriverHost drv;
    MtpState *mtp_state = nullptr;
    uint32_t *out_tok = nullptr;
    int out_cap = 0;
    int32_t *force_d1 = nullptr;
    int force_n = 0;
    hipGraphExec_t graph_exec = nullptr;
    // fused run kernel (one persistent launch per run) when the device supports it
    bool fused = false, fused_ok = false;
    int fz_grid = 0;
    size_t fz_lds = 0;
    uint32_t *fz_sync = nullptr;
    uint64_t *fz_xch = nullptr;     // the tagged exchange buffers (FzXch), one allocation
    size_t fz_xch_words = 0;
    uint64_t fz_launches = 0;       // fused launches (an upper bound) since the tag base was last zeroed
    bool fz_capturing = false;      // launches being captured into a graph are counted per replay
    unsigned long long *fz_keys = nullptr;
    MtpHooks *fz_hooks = nullptr;   // the device-driven MTP step's stages in the fused runs
    LayerDev *fz_layers = nullptr;
    FusedArgs *fz_args = nullptr;   // [3]: verify, draft, seed
    unsigned long long *fz_trace = nullptr;
    FusedArgs fz_host[3];
    const unsigned long long *keys() const { return fused ? fz_keys : b.amax_key; }
    int nkeys() const { return fused ? fz_grid : 1; }
    // batched prefill (k_prefill.hip)
    PfBufs pfb{};
    int pf_alloc(int T);
    int pf_attn_lds(int kv_cap);
    int pf_chunk(const uint32_t *toks, int T, float *h_out);
    int prefill(const uint32_t *toks, int n, uint32_t *next, float *h_all);
    int seed_batched(const uint32_t *toks, int n, int pos0, const float *hs);
    // weights from a GGUF file (k_load.hip): through a staging buffer allocated for the call, or
    // through `stage` (chunk bytes) when given
    int load_gguf(const Gguf &g, uint8_t *stage = nullptr, int64_t chunk = 0);
    // kernel probe: HIP events around every launch of one kernel kind while enqueuing eagerly
    int probe_kind = -1;
    std::vector<hipEvent_t> probe_ev;
    size_t probe_used = 0;
    void probe(int kind) {
        if (kind != probe_kind) return;
        if (probe_used == probe_ev.size()) {
            hipEvent_t ev;
            if (hipEventCreate(&ev) != hipSuccess) return;
            probe_ev.push_back(ev);
        }
        (void)hipEventRecord(probe_ev[probe_used++], st);
    }

    int dev_depth = 1;   // drafts per device-driven step (1 or 2), set by dev_begin
    void enqueue_mtp_device_step();
    void enqueue_mtp_device_step2();
    int mtp_steps_async(int k, bool use_graph);
    int ensure_out(int cap) {
        if (cap <= out_cap) return 0;
        try {
            out_tok = alloc<uint32_t>((size_t)cap);
        } catch (...) {
            return -3;
        }
        out_cap = cap;
        if (graph_exec) {  // the captured commit kernel holds the old buffer
            (void)hipGraphExecDestroy(graph_exec);
            graph_exec = nullptr;
        }
        return hooks_upload();
    }
    // the fused runs' view of the device-driven step (MtpHooks), after any of its buffers changes
    int hooks_upload() {
        if (!fz_hooks) return 0;
        MtpHooks h{};
        h.ms = mtp_state;
        h.ctl_verify = ctl;
        h.ctl_draft = ctl_draft;
        h.out_tok = out_tok;
        h.out_cap = out_cap;
        h.force = force_d1;
        h.force_n = force_n;
        h.n_ctx = m.n_ctx;
        if (hipMemcpyAsync(fz_hooks, &h, sizeof(h), hipMemcpyHostToDevice, st) != hipSuccess) return -2;
        return hipStreamSynchronize(st) == hipSuccess ? 0 : -2;
    }
    int set_force(const int32_t *f, int n) {
        for (int i = 0; i < n; i++)
            if (f[i] >= d.n_vocab) return -1;
        if (n <= 0) {
            force_n = 0;
            force_d1 = nullptr;
        } else {
            try {
                force_d1 = alloc<int32_t>((size_t)n);
            } catch (...) {
                return -3;
            }
            if (hipMemcpy(force_d1, f, (size_t)n * 4, hipMemcpyHostToDevice) != hipSuccess) return -2;
            force_n = n;
        }
        if (graph_exec) {
            (void)hipGraphExecDestroy(graph_exec);
            graph_exec = nullptr;
        }
        return hooks_upload();
    }
    int hidden_host(int lane, float *out) {
        if (hipMemcpyAsync(out, b.hid + (size_t)lane * E, E * 4, hipMemcpyDeviceToHost, st) != hipSuccess) return -2;
        return hipStreamSynchronize(st) == hipSuccess ? 0 : -2;
    }

    template <class T>
    T *alloc(size_t n) {
        void *p = nullptr;
        if (hipMalloc(&p, n * sizeof(T) + 64) != hipSuccess) throw std::runtime_error("hipMalloc failed");
        allocs.push_back(p);
        bytes += n * sizeof(T);
        return (T *)p;
    }
    Q8W q8(int64_t rows, int64_t k) {
        Q8W w;
        w.q = alloc<int8_t>(rows * k);
        w.d = alloc<uint16_t>(rows * k / 32);
        w.rows = rows;
        w.k = k;
        return w;
    }
    ~Engine() {
        for (hipEvent_t ev : probe_ev) (void)hipEventDestroy(ev);
        if (graph_exec) (void)hipGraphExecDestroy(graph_exec);
        (void)hipStreamSynchronize(st);
        for (void *p : allocs) (void)hipFree(p);
        if (st && own_stream) (void)hipStreamDestroy(st);
    }

    static bool shape_ok(const oxe_model_desc &d) {
        return d.n_embd == E && d.n_head == NH && d.n_head_kv == NKV && d.head_dim == HD && d.n_expert == NEXP &&
               d.n_expert_used == KUSED && d.ff_exp == FF && d.ff_shexp == FFSH && d.ssm_conv_kernel == KC &&
               d.ssm_d_state == DS && d.ssm_n_kheads == NKH && d.ssm_n_vheads == NVH && d.ssm_d_inner == DIN &&
               d.n_rot == NROT && d.n_layer >= 1 && d.n_layer <= 62 && d.n_vocab >= 16 && d.n_vocab % 16 == 0 &&
               d.full_attention_interval >= 1 && d.has_mtp == 1;
    }

    // caller: every launch and copy of this engine goes to the caller's `stream` (the null stream
    // included); otherwise to a stream of its own. mt: the matrices' types (a model file's), Q8_0
    // everywhere when null
    void create(const oxe_model_desc &desc, uint64_t sd, int n_ctx, bool caller = false, hipStream_t stream = nullptr,
                const ModelTypes *mt = nullptr) {
        d = desc;
        seed = sd;
        types.layer.assign(d.n_layer + 1, LayerTypes{});
        types.output = 8;
        types.tok_embd = 8;
        if (mt && (int)mt->layer.size() == d.n_layer + 1) types = *mt;
        kq = types.any();
        if (hipGetDevice(&dev) != hipSuccess) throw std::runtime_error("hipGetDevice failed");
        if (caller) {
            st = stream;
            own_stream = false;
        } else if (hipStreamCreate(&st) != hipSuccess) {
            throw std::runtime_error("hipStreamCreate failed");
        }
        m.n_layer = d.n_layer;
        m.n_vocab = d.n_vocab;
        m.n_ctx = (n_ctx + 255) / 256 * 256;
        m.eps = d.rms_eps;
        const int nl_total = d.n_layer + 1;
        L.resize(nl_total);
        int n_rec = 0, n_att = 0;
        for (int il = 0; il < nl_total; il++) {
            LayerW &w = L[il];
            w.att = il == d.n_layer || ((il + 1) % d.full_attention_interval == 0);
            w.index = w.att ? n_att++ : n_rec++;
        }
        m.n_rec = n_rec;
        m.n_att = n_att;
        n_att_main = n_att - 1;
        // weights
        for (int il = 0; il < nl_total; il++) {
            LayerW &w = L[il];
            const LayerTypes &ty = types.layer[il];
            // a projection in the file's blocks (all its parts) or an output projection of another
            // type has no Q8_0 matrix; the Q8W keeps the row count the runs read
            const bool kq_proj = w.att ? ty.q != 8 : ty.qkv != 8;
            auto q8_or_rows = [&](bool q, int64_t rows, int64_t k) {
                if (q) return q8(rows, k);
                Q8W r{};
                r.rows = rows;
                r.k = k;
                return r;
            };
            w.attn_norm = alloc<float>(E);
            w.post_norm = alloc<float>(E);
            if (!w.att) {
                w.proj = q8_or_rows(!kq_proj, DN_ROWS, E);
                w.out = q8_or_rows(ty.out == 8, E, DIN);
                w.conv = alloc<float>((size_t)NCH * KC);
                w.ssm_a = alloc<float>(NVH);
                w.dt_bias = alloc<float>(NVH);
                w.ssm_norm = alloc<float>(HV);
            } else {
                w.proj = q8_or_rows(!kq_proj, AT_ROWS, E);
                w.out = q8_or_rows(ty.out == 8, E, NH * HD);
                w.q_norm = alloc<float>(HD);
                w.k_norm = alloc<float>(HD);
            }
            w.router = alloc<float>((size_t)NEXP * E);
            w.shexp_gate = alloc<float>(E);
            // a matrix of another type lives in its file blocks; its Q8_0 array is not allocated
            auto raw = [&](RawW &r, int type, int64_t n_grp, int64_t rows, int64_t k) {
                r.type = type;
                r.rows = rows;
                r.k = k;
                if (type != 8) r.w = alloc<uint8_t>((size_t)(n_grp * rows * raw_row_bytes(r)));
            };
            raw(w.sh_gate_r, ty.sh_gate, 1, FFSH, E);
            raw(w.sh_up_r, ty.sh_up, 1, FFSH, E);
            raw(w.sh_down_r, ty.sh_down, 1, E, FFSH);
            raw(w.exp_gate_r, ty.gate, NEXP, FF, E);
            raw(w.exp_up_r, ty.up, NEXP, FF, E);
            raw(w.exp_down_r, ty.down, NEXP, E, FF);
            if (!w.att) {
                raw(w.beta_r, ty.beta, 1, NVH, E);
                raw(w.alpha_r, ty.alpha, 1, NVH, E);
                raw(w.qkv_r, ty.qkv, 1, NCH, E);
                raw(w.z_r, ty.z, 1, DIN, E);
                raw(w.out_r, ty.out, 1, E, DIN);
            } else {
                raw(w.q_r, ty.q, 1, NH * 2 * HD, E);
                raw(w.k_r, ty.k, 1, NKV * HD, E);
                raw(w.v_r, ty.v, 1, NKV * HD, E);
                raw(w.out_r, ty.out, 1, E, NH * HD);
            }
            if (ty.sh_gate == 8) w.shexp_gu = q8(2 * FFSH, E);
            if (ty.sh_down == 8) w.shexp_down = q8(E, FFSH);
            if (ty.gate == 8) w.exp_gu = q8((int64_t)NEXP * 2 * FF, E);
            if (ty.down == 8) w.exp_down = q8((int64_t)NEXP * E, FF);
            if (il == d.n_layer) {
                w.eh_proj = q8(E, 2 * E);
                w.enorm = alloc<float>(E);
                w.hnorm = alloc<float>(E);
                w.head_norm = alloc<float>(E);
            }
        }
        m.tok_embd_r = RawW{};
        if (types.tok_embd != 8) {
            // a K-quant embedding: its rows are dequantised per run (launch_kq_embed)
            m.tok_embd_r.type = types.tok_embd;
            m.tok_embd_r.rows = d.n_vocab;
            m.tok_embd_r.k = E;
            m.tok_embd_r.w = alloc<uint8_t>((size_t)(d.n_vocab * raw_row_bytes(m.tok_embd_r)));
            m.tok_embd.rows = d.n_vocab;
            m.tok_embd.k = E;
        } else {
            m.tok_embd = q8(d.n_vocab, E);
        }
        m.output_r = RawW{};
        if (types.output != 8) {
            m.output_r.type = types.output;
            m.output_r.rows = d.n_vocab;
            m.output_r.k = E;
            m.output_r.w = alloc<uint8_t>((size_t)(d.n_vocab * raw_row_bytes(m.output_r)));
            m.output.rows = d.n_vocab;   // the vocabulary size every head reads; no Q8_0 array
            m.output.k = E;
        } else {
            m.output = q8(d.n_vocab, E);
        }
        m.out_norm = alloc<float>(E);
        // state
        m.conv_state = alloc<float>((size_t)OXE_NSLOTS * n_rec * NCH * (KC - 1));
        m.ssm_state = alloc<float>((size_t)OXE_NSLOTS * n_rec * NVH * HV * HV);
        m.kcache = alloc<uint16_t>((size_t)n_att * NKV * m.n_ctx * HD);
        m.vcache = alloc<uint16_t>((size_t)n_att * NKV * HD * m.n_ctx);
        m.rope = alloc<float>((size_t)m.n_ctx * NROT);
        // activations
        b.x = alloc<float>(OXE_NL * E);
        b.x1 = alloc<float>(OXE_NL * E);
        b.x2 = alloc<float>(OXE_NL * E);
        b.xq = alloc<int8_t>(OXE_NL * 2 * E);
        b.xd = alloc<uint16_t>(OXE_NL * 2 * E / 32);
        b.xn = alloc<float>(OXE_NL * E);
        b.proj = alloc<float>((size_t)OXE_NL * DN_ROWS);
        b.gdn = alloc<float>(OXE_NL * DIN);
        b.oq = alloc<int8_t>(OXE_NL * MIX_W);
        b.od = alloc<uint16_t>(OXE_NL * MIX_W / 32);
        b.scores = alloc<float>((size_t)OXE_NL * NH * m.n_ctx);
        b.router_lg = alloc<float>(OXE_NL * NEXP);
        b.sh_gate = alloc<float>(OXE_NL);
        b.hsh = alloc<float>(OXE_NL * FFSH);
        b.hexp = alloc<float>(OXE_NL * KUSED * FF);
        b.route_ids = alloc<int32_t>(OXE_NL * KUSED);
        b.route_w = alloc<float>(OXE_NL * KUSED);
        b.uni = alloc<int32_t>(OXE_MAX_UNION + 1);
        b.hid = alloc<float>((size_t)HID_N * E);
        b.logits = alloc<float>((size_t)OXE_NL * d.n_vocab);
        b.amax_key = alloc<unsigned long long>(OXE_NL);
        b.xk = alloc<uint8_t>((size_t)OXE_NL * (E / 256) * 292);
        b.hk = alloc<uint8_t>((size_t)OXE_NL * KUSED * (FF / 256) * 292);
        b.hshk = alloc<uint8_t>((size_t)OXE_NL * (FFSH / 256) * 292);
        if (kq) {
            b.o32 = alloc<float>(OXE_NL * MIX_W);
            b.ok = alloc<uint8_t>((size_t)OXE_NL * (MIX_W / 256) * 292);
            b.emb = alloc<float>(OXE_NL * E);
        }
        b.counters = alloc<uint32_t>(CNT_N);
        ctl = alloc<RunCtl>(2);
        ctl_draft = ctl + 1;
        mtp_state = alloc<MtpState>(1);
        (void)hipMemsetAsync(mtp_state, 0, sizeof(MtpState), st);
        // zero what must start at zero (before any graph capture)
        (void)hipMemsetAsync(m.conv_state, 0, (size_t)OXE_NSLOTS * n_rec * NCH * (KC - 1) * 4, st);
        (void)hipMemsetAsync(m.ssm_state, 0, (size_t)OXE_NSLOTS * n_rec * NVH * HV * HV * 4, st);
        (void)hipMemsetAsync(m.kcache, 0, (size_t)n_att * NKV * m.n_ctx * HD * 2, st);
        (void)hipMemsetAsync(m.vcache, 0, (size_t)n_att * NKV * HD * m.n_ctx * 2, st);
        (void)hipMemsetAsync(b.counters, 0, CNT_N * 4, st);
        (void)hipMemsetAsync(b.hid, 0, (size_t)HID_N * E * 4, st);
        (void)hipMemsetAsync(b.amax_key, 0, OXE_NL * 8, st);
        // RoPE cache per position with the host C library (oxe_mrope_cache_init, oxe_ops.cpp:386-439)
        std::vector<float> rope((size_t)m.n_ctx * NROT);
        for (int p = 0; p < m.n_ctx; p++) mrope_cache(p, rope.data() + (size_t)p * NROT);
        (void)hipMemcpyAsync(m.rope, rope.data(), rope.size() * 4, hipMemcpyHostToDevice, st);
        (void)hipStreamSynchronize(st);
        if (hipGetLastError() != hipSuccess) throw std::runtime_error("HIP error during engine creation");
        fused_init();
    }

    // The fused run kernel needs one workgroup per CU on exactly 256 CUs (its row splits assume
    // 256 workgroups) with every workgroup resident.
    void fused_init() {
        if (kq) return;   // the fused run kernel reads Q8_0 matrices only: such models run per phase
        int dev = 0, ncu = 0;
        if (hipGetDevice(&dev) != hipSuccess) return;
        if (hipDeviceGetAttribute(&ncu, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return;
        fz_lds = fused_lds_bytes(m.n_ctx);
        if (ncu != 256 || fused_blocks_per_cu(fz_lds) < 1) return;
        fz_grid = ncu;
        fz_sync = alloc<uint32_t>(FZ_SYNC_WORDS);
        // tags of a launch are base + 1 + 8 k + phase for run layers k <= n_layer
        if (8 * (d.n_layer + 2) >= (int64_t)FZ_TAG_STRIDE) return;
        const size_t NLs = OXE_NL;
        const size_t xw[13] = {2 * NLs * E, 2 * NLs * E, 2 * NLs * DN_ROWS, 2 * NLs * MIX_W, 2 * NLs * (MIX_W / 4),
                               2 * NLs * (MIX_W / 32), 2 * NLs * NEXP, 2 * NLs, 2 * NLs * FFSH,
                               2 * NLs * OXE_MAX_UNION * (FF / 4), 2 * NLs * OXE_MAX_UNION * (FF / 32),
                               2 * NLs * NH * (size_t)m.n_ctx, NLs * (size_t)fz_grid * 2};
        size_t off[13], tot = 0;
        for (int i = 0; i < 13; i++) {
            off[i] = tot;
            tot += (xw[i] + 31) / 32 * 32;   // 256-byte aligned parts
        }
        if (tot * 8 > 0x7fffffffull) return;   // buffer offsets are 31-bit
        fz_xch = alloc<uint64_t>(tot);
        fz_xch_words = tot;
        FzXch xc;
        uint64_t **parts[13] = {&xc.x, &xc.x1, &xc.p, &xc.g, &xc.o, &xc.od, &xc.lg, &xc.sg, &xc.hsh, &xc.hq, &xc.hd,
                                &xc.sc, &xc.kx};
        for (int i = 0; i < 13; i++) *parts[i] = fz_xch + off[i];
        fz_hooks = alloc<MtpHooks>(1);
        fz_keys = alloc<unsigned long long>((size_t)OXE_NL * fz_grid);
        const int nl_total = d.n_layer + 1;
        std::vector<LayerDev> ld(nl_total);
        for (int il = 0; il < nl_total; il++) {
            const LayerW &w = L[il];
            LayerDev &x = ld[il];
            x.att = w.att;
            x.index = w.index;
            x.attn_norm = w.attn_norm; x.post_norm = w.post_norm;
            x.proj = w.proj; x.out = w.out;
            x.conv = w.conv; x.ssm_a = w.ssm_a; x.dt_bias = w.dt_bias; x.ssm_norm = w.ssm_norm;
            x.q_norm = w.q_norm; x.k_norm = w.k_norm;
            x.router = w.router; x.shexp_gate = w.shexp_gate;
            x.shexp_gu = w.shexp_gu; x.shexp_down = w.shexp_down; x.exp_gu = w.exp_gu; x.exp_down = w.exp_down;
            x.eh_proj = w.eh_proj;
            x.enorm = w.enorm; x.hnorm = w.hnorm; x.head_norm = w.head_norm;
        }
        fz_layers = alloc<LayerDev>(nl_total);
        fz_args = alloc<FusedArgs>(3);
        FusedArgs fa[3];
        for (int mode = 0; mode < 3; mode++) {
            FusedArgs &f = fa[mode];
            f = FusedArgs{};
            f.mode = mode;
            f.n_layer = d.n_layer;
            f.keep_logits = (mode == FM_VERIFY && keep_logits) ? 1 : 0;   // the MTP head keeps no logits
            f.grid = fz_grid;
            f.layers = fz_layers;
            f.m = m;
            f.b = b;
            f.sync = fz_sync;
            f.xc = xc;
            f.xbase = fz_xch;
            f.xbytes = (uint32_t)(fz_xch_words * 8);
            f.keys = fz_keys;
            f.mh = fz_hooks;
            f.head_w = m.output;
            f.head_ids = nullptr;
        }
        if (hooks_upload()) return;
        (void)hipMemsetAsync(fz_sync, 0, FZ_SYNC_WORDS * 4, st);
        (void)hipMemsetAsync(fz_xch, 0, fz_xch_words * 8, st);
        (void)hipMemsetAsync(fz_keys, 0, (size_t)OXE_NL * fz_grid * 8, st);
        (void)hipMemcpyAsync(fz_layers, ld.data(), sizeof(LayerDev) * nl_total, hipMemcpyHostToDevice, st);
        for (int mode = 0; mode < 3; mode++) fz_host[mode] = fa[mode];
        (void)hipMemcpyAsync(fz_args, fa, sizeof(fa), hipMemcpyHostToDevice, st);
        if (hipStreamSynchronize(st) != hipSuccess || hipGetLastError() != hipSuccess) return;
        fused_ok = true;
        fused = true;
    }
    int set_fused(bool on) {
        if (on && !fused_ok) return -1;
        if (on != fused) {
            fused = on;
            if (graph_exec) {
                (void)hipGraphExecDestroy(graph_exec);
                graph_exec = nullptr;
            }
        }
        return 0;
    }
    // phase trace of the fused kernel: [grid][FZ_TRACE_EV][4] (phase id, start, barrier passed, end)
    int set_trace(bool on) {
        if (!fused_ok) return -1;
        if (on && !fz_trace) {
            try {
                fz_trace = alloc<unsigned long long>((size_t)fz_grid * FZ_TRACE_EV * 4);
            } catch (...) {
                return -3;
            }
        }
        for (int mode = 0; mode < 3; mode++) fz_host[mode].trace = on ? fz_trace : nullptr;
        if (on) (void)hipMemsetAsync(fz_trace, 0, (size_t)fz_grid * FZ_TRACE_EV * 32, st);
        if (hipMemcpyAsync(fz_args, fz_host, sizeof(fz_host), hipMemcpyHostToDevice, st) != hipSuccess) return -2;
        return hipStreamSynchronize(st) == hipSuccess ? 0 : -2;
    }
    // n more fused launches about to be enqueued (outside graph capture). The tag base grows by
    // FZ_TAG_STRIDE per launch; long before it wraps, every exchange word and the base go back to
    // zero (a fill kernel on the engine stream, ordered before the launches).
    static constexpr uint64_t FZ_CLEAR_EVERY = 1ull << 20;
    void fz_account(int n) {
        if (fz_launches + (uint64_t)n > FZ_CLEAR_EVERY) {
            launch_fused_xch_clear(fz_xch, fz_xch_words, fz_sync, st);
            fz_launches = 0;
        }
        fz_launches += (uint64_t)n;
    }
    // after a run of the fused kernel was aborted (a poll that timed out): clear the error word,
    // move the tag base on, and report -5 (OXE_E_ABORT). An aborted run commits nothing: its lanes
    // write only the recurrent slots after the current one and the K / V^T rows of their own
    // positions, which the next run that reaches those positions writes again.
    int fused_check() {
        if (!fused) return 0;
        uint32_t err[5] = {0, 0, 0, 0, 0};
        if (hipMemcpyAsync(err, fz_sync + FZ_W_ERR, sizeof(err), hipMemcpyDeviceToHost, st) != hipSuccess) return -2;
        if (hipStreamSynchronize(st) != hipSuccess) return -2;
        if (err[0]) {
            launch_fused_sync_reset(fz_sync, st);
            (void)hipStreamSynchronize(st);
            fz_account(1);
            // the word that timed out: its byte offset in the exchange allocation, the tags
            const int64_t off = (int64_t)(uint32_t)(err[3] - (uint32_t)(uintptr_t)fz_xch);
            char msg[256];
            snprintf(msg, sizeof msg,
                     "fused run aborted: an exchange poll timed out (workgroup %u, byte offset %lld, tag %u expected, "
                     "%u seen; sync words reset, nothing committed)",
                     err[4], (long long)off, err[1], err[2]);
            set_err(msg);
            return -5;
        }
        return 0;
    }

    // ggml_mrope_cache_init for a text position (IMRoPE sections, ext_factor 0, freq_scale 1)
    void mrope_cache(int64_t p, float *cache) const {
        const int n_dims = NROT;
        const float theta_scale = powf(d.rope_freq_base, -2.0f / n_dims);
        const int *sec = d.rope_sections;
        const int sect_dims = sec[0] + sec[1] + sec[2] + sec[3];
        float theta_t = (float)p, theta_h = (float)p, theta_w = (float)p, theta_e = 0.0f;
        for (int i0 = 0; i0 < n_dims; i0 += 2) {
            const int sector = (i0 / 2) % sect_dims;
            float theta;
            if (sector % 3 == 1 && sector < 3 * sec[1]) theta = theta_h;
            else if (sector % 3 == 2 && sector < 3 * sec[2]) theta = theta_w;
            else if (sector % 3 == 0 && sector < 3 * sec[0]) theta = theta_t;
            else theta = theta_e;
            const float th = 1.0f * theta;
            cache[i0] = cosf(th) * 1.0f;
            cache[i0 + 1] = sinf(th) * 1.0f;
            theta_t *= theta_scale;
            theta_w *= theta_scale;
            theta_h *= theta_scale;
            theta_e *= theta_scale;
        }
    }

    int synth_weights() {
        int rc = 0;
        auto chk = [&](int r) { if (r) rc = r; };
        // a matrix kept in another type (an engine created with types): the oracle's synthetic
        // K-quant blocks or F32 values of the same tensor; groups: the experts of an expert tensor
        auto raw = [&](const RawW &r, int il, int kind, int64_t groups) {
            if (r.type != 8) chk(synth_raw(seed, il, kind, r.type, groups * r.rows, r.k, r.w, st));
        };
        const int nl_total = d.n_layer + 1;
        for (int il = 0; il < nl_total; il++) {
            LayerW &w = L[il];
            chk(synth_f32(seed, il, OXE_T_ATTN_NORM, E, w.attn_norm, st));
            chk(synth_f32(seed, il, OXE_T_POST_NORM, E, w.post_norm, st));
            if (!w.att) {
                if (!w.kq_proj()) {
                    chk(synth_q8(seed, il, OXE_T_DN_QKV, -1, NCH, E, NCH, 0, w.proj.q, w.proj.d, st));
                    chk(synth_q8(seed, il, OXE_T_DN_Z, -1, DIN, E, DIN, 0, w.proj.q + (int64_t)DN_Z * E, w.proj.d + (int64_t)DN_Z * E / 32, st));
                } else {
                    raw(w.qkv_r, il, OXE_T_DN_QKV, 1);
                    raw(w.z_r, il, OXE_T_DN_Z, 1);
                }
                if (w.beta_r.type == 8) {
                    chk(synth_q8(seed, il, OXE_T_DN_BETA, -1, NVH, E, NVH, 0, w.proj.q + (int64_t)DN_BETA * E, w.proj.d + (int64_t)DN_BETA * E / 32, st));
                    chk(synth_q8(seed, il, OXE_T_DN_ALPHA, -1, NVH, E, NVH, 0, w.proj.q + (int64_t)DN_ALPHA * E, w.proj.d + (int64_t)DN_ALPHA * E / 32, st));
                } else {
                    raw(w.beta_r, il, OXE_T_DN_BETA, 1);
                    raw(w.alpha_r, il, OXE_T_DN_ALPHA, 1);
                }
                if (w.out_r.type == 8) chk(synth_q8(seed, il, OXE_T_DN_OUT, -1, E, DIN, E, 0, w.out.q, w.out.d, st));
                else raw(w.out_r, il, OXE_T_DN_OUT, 1);
                chk(synth_f32(seed, il, OXE_T_DN_CONV, (int64_t)NCH * KC, w.conv, st));
                chk(synth_f32(seed, il, OXE_T_DN_A, NVH, w.ssm_a, st));
                chk(synth_f32(seed, il, OXE_T_DN_DT, NVH, w.dt_bias, st));
                chk(synth_f32(seed, il, OXE_T_DN_NORM, HV, w.ssm_norm, st));
            } else {
                if (!w.kq_proj()) {
                    chk(synth_q8(seed, il, OXE_T_ATT_Q, -1, NH * 2 * HD, E, NH * 2 * HD, 0, w.proj.q, w.proj.d, st));
                    chk(synth_q8(seed, il, OXE_T_ATT_K, -1, NKV * HD, E, NKV * HD, 0, w.proj.q + (int64_t)AT_K * E, w.proj.d + (int64_t)AT_K * E / 32, st));
                    chk(synth_q8(seed, il, OXE_T_ATT_V, -1, NKV * HD, E, NKV * HD, 0, w.proj.q + (int64_t)AT_V * E, w.proj.d + (int64_t)AT_V * E / 32, st));
                } else {
                    raw(w.q_r, il, OXE_T_ATT_Q, 1);
                    raw(w.k_r, il, OXE_T_ATT_K, 1);
                    raw(w.v_r, il, OXE_T_ATT_V, 1);
                }
                if (w.out_r.type == 8) chk(synth_q8(seed, il, OXE_T_ATT_OUT, -1, E, NH * HD, E, 0, w.out.q, w.out.d, st));
                else raw(w.out_r, il, OXE_T_ATT_OUT, 1);
                chk(synth_f32(seed, il, OXE_T_ATT_QNORM, HD, w.q_norm, st));
                chk(synth_f32(seed, il, OXE_T_ATT_KNORM, HD, w.k_norm, st));
            }
            chk(synth_f32(seed, il, OXE_T_ROUTER, (int64_t)NEXP * E, w.router, st));
            chk(synth_f32(seed, il, OXE_T_SHEXP_GATE, E, w.shexp_gate, st));
            if (w.sh_gate_r.type == 8) {
                chk(synth_q8(seed, il, OXE_T_GATE_SHEXP, OXE_T_UP_SHEXP, 2 * FFSH, E, FFSH, 0, w.shexp_gu.q, w.shexp_gu.d, st));
            } else {
                raw(w.sh_gate_r, il, OXE_T_GATE_SHEXP, 1);
                raw(w.sh_up_r, il, OXE_T_UP_SHEXP, 1);
            }
            if (w.sh_down_r.type == 8) chk(synth_q8(seed, il, OXE_T_DOWN_SHEXP, -1, E, FFSH, E, 0, w.shexp_down.q, w.shexp_down.d, st));
            else raw(w.sh_down_r, il, OXE_T_DOWN_SHEXP, 1);
            if (w.exp_gate_r.type == 8) {
                for (int e = 0; e < NEXP; e++)
                    chk(synth_q8(seed, il, OXE_T_GATE_EXPS, OXE_T_UP_EXPS, 2 * FF, E, FF, e, w.exp_gu.q + (int64_t)e * 2 * FF * E,
                                 w.exp_gu.d + (int64_t)e * 2 * FF * E / 32, st));
            } else {
                raw(w.exp_gate_r, il, OXE_T_GATE_EXPS, NEXP);
                raw(w.exp_up_r, il, OXE_T_UP_EXPS, NEXP);
            }
            if (w.exp_down_r.type == 8) {
                for (int e = 0; e < NEXP; e++)
                    chk(synth_q8(seed, il, OXE_T_DOWN_EXPS, -1, E, FF, E, e, w.exp_down.q + (int64_t)e * E * FF,
                                 w.exp_down.d + (int64_t)e * E * FF / 32, st));
            } else {
                raw(w.exp_down_r, il, OXE_T_DOWN_EXPS, NEXP);
            }
            if (il == d.n_layer) {
                chk(synth_q8(seed, il, OXE_T_EH_PROJ, -1, E, 2 * E, E, 0, w.eh_proj.q, w.eh_proj.d, st));
                chk(synth_f32(seed, il, OXE_T_ENORM, E, w.enorm, st));
                chk(synth_f32(seed, il, OXE_T_HNORM, E, w.hnorm, st));
                chk(synth_f32(seed, il, OXE_T_HEAD_NORM, E, w.head_norm, st));
            }
        }
        if (m.tok_embd_r.type == 8)
            chk(synth_q8(seed, OXE_GLOBAL_LAYER, OXE_T_TOK_EMBD, -1, d.n_vocab, E, d.n_vocab, 0, m.tok_embd.q, m.tok_embd.d, st));
        else raw(m.tok_embd_r, OXE_GLOBAL_LAYER, OXE_T_TOK_EMBD, 1);
        if (m.output_r.type == 8)
            chk(synth_q8(seed, OXE_GLOBAL_LAYER, OXE_T_OUTPUT, -1, d.n_vocab, E, d.n_vocab, 0, m.output.q, m.output.d, st));
        else raw(m.output_r, OXE_GLOBAL_LAYER, OXE_T_OUTPUT, 1);
        chk(synth_f32(seed, OXE_GLOBAL_LAYER, OXE_T_OUT_NORM, E, m.out_norm, st));
        if (hipStreamSynchronize(st) != hipSuccess) return -2;
        return rc;
    }

    // ---- run sequences (device-side lanes/positions from RunCtl) ----
    enum { K_HEAD = 0, K_EXPERTS = 1, K_DOWN = 2, K_PROJ = 3, K_OUT = 4, K_DN = 5, K_ROUTER = 6, K_SCORES = 7, K_PV = 8, K_ENTRY = 9,
           K_FUSED = 10, K_FUSED_DRAFT = 11,
           // batched prefill: every matrix-core GEMM, the grouped expert GEMMs, attention, delta rule
           K_PF_GEMM = 12, K_PF_EXPERT = 13, K_PF_ATTN = 14, K_PF_DELTA = 15 };
    // a layer's projection (K-quant parts or the Q8_0 matrix), then F32 ssm_beta / ssm_alpha rows
    void enqueue_proj(const LayerW &w, const float *x, bool embed, float *x_store, int64_t row_begin = 0) {
        probe(K_PROJ);
        if (w.kq_proj()) (void)launch_kq_proj(ctl, m, w, x, embed, x_store, b, st, row_begin);
        else launch_proj(ctl, m, w, x, embed, x_store, b, st, row_begin);
        probe(K_PROJ);
        if (!w.att && w.beta_r.type == 0) (void)launch_ba_f32(ctl, m, w, embed ? x_store : x, b, st);
    }
    // the mixer's output projection + residual into x1 (K-quant: from the f32 gated outputs)
    void enqueue_out(const LayerW &w, const float *x) {
        probe(K_OUT);
        if (w.out_r.type != 8) (void)launch_kq_out(ctl, m, w, x, b, st);
        else launch_out(ctl, w, x, b, st);
        probe(K_OUT);
    }
    void enqueue_layer(int l, bool first) {
        const LayerW &w = L[l];
        const float *x = first ? b.x : b.x2;
        float *o32 = w.out_r.type != 8 ? b.o32 : nullptr;
        if (first && m.tok_embd_r.type != 8) (void)launch_kq_embed(ctl, m, b.emb, st);
        enqueue_proj(w, first ? nullptr : b.x2, first, first ? b.x : nullptr);
        if (!w.att) {
            probe(K_DN); launch_dn(ctl, m, w, b, st, o32); probe(K_DN);
        } else {
            launch_kwrite(ctl, m, w, b, st);
            probe(K_SCORES); launch_scores(ctl, m, w, b, st); probe(K_SCORES);
            probe(K_PV); launch_pv(ctl, m, w, b, st, o32); probe(K_PV);
        }
        enqueue_out(w, x);
        enqueue_moe(w);
    }
    // the MTP entry over the lanes' tokens (a K-quant embedding's rows dequantised first)
    void enqueue_entry(const LayerW &w) {
        const bool kemb = m.tok_embd_r.type != 8;
        if (kemb) (void)launch_kq_embed(ctl, m, b.emb, st);
        probe(K_ENTRY); launch_entry(ctl, m, w, b, st, kemb ? b.emb : nullptr); probe(K_ENTRY);
    }
    void enqueue_moe(const LayerW &w) {
        probe(K_ROUTER); launch_router(ctl, m, w, b, st); probe(K_ROUTER);
        launch_route(ctl, b, st);
        if (w.kq_moe()) {
            probe(K_EXPERTS); (void)launch_kq_moe(ctl, m, w, b, st); probe(K_EXPERTS);
            return;
        }
        probe(K_EXPERTS); launch_experts(ctl, w, b, st); probe(K_EXPERTS);
        probe(K_DOWN); launch_down(ctl, w, b, st); probe(K_DOWN);
    }
    // draft: an MTP draft run's head (the restricted draft head when one is set)
    void enqueue_head(const float *norm_w, bool store_logits, bool draft = false) {
        const uint32_t *ids = draft ? draft_ids : nullptr;
        if (m.output_r.type != 8) (void)launch_kq_head(ctl, m, norm_w, b, st, draft ? &draft_r : nullptr, ids);
        else launch_head(ctl, m, norm_w, b, store_logits, st, draft ? &draft_w : nullptr, ids);
    }
    // ---- restricted-vocabulary draft head (MtpWeights::set_draft_vocab, mtp.rs:166-197): the
    // output matrix's rows of `ids` (below n_vocab, sorted, duplicates dropped, padded to a multiple
    // of 16 rows by repeating the last id), gathered on the device; every MTP draft run's argmax
    // runs over them and maps local row r back to token ids[r]. Drafts only: verify runs keep the
    // whole head, so the output is unchanged. n = 0: drafts use the whole head again. Returns the
    // draft head's rows (0 when cleared) or -1 (no id in range), -2, -3.
    Q8W draft_w{};
    RawW draft_r{};
    uint32_t *draft_ids = nullptr;
    int64_t draft_rows = 0, draft_cap = 0;
    int set_draft_vocab(const uint32_t *ids, int n);
    void enqueue_verify() {
        if (fused) {
            if (!fz_capturing) fz_account(1);
            probe(K_FUSED);
            launch_fused(ctl, fz_args + FM_VERIFY, fz_grid, fz_lds, st);
            probe(K_FUSED);
            return;
        }
        for (int l = 0; l < d.n_layer; l++) enqueue_layer(l, l == 0);
        probe(K_HEAD); enqueue_head(m.out_norm, keep_logits); probe(K_HEAD);
    }
    // rc: the fused run's control block (default: ctl)
    void enqueue_mtp_run(const RunCtl *rc = nullptr) {
        if (fused) {
            if (!fz_capturing) fz_account(1);
            probe(K_FUSED_DRAFT);
            launch_fused(rc ? rc : ctl, fz_args + FM_DRAFT, fz_grid, fz_lds, st);
            probe(K_FUSED_DRAFT);
            return;
        }
        const LayerW &w = L[d.n_layer];
        enqueue_entry(w);
        // the MTP layer: input x2 (the entry output), as any layer > 0
        enqueue_proj(w, b.x2, false, nullptr);
        launch_kwrite(ctl, m, w, b, st);
        probe(K_SCORES); launch_scores(ctl, m, w, b, st); probe(K_SCORES);
        probe(K_PV); launch_pv(ctl, m, w, b, st, w.out_r.type != 8 ? b.o32 : nullptr); probe(K_PV);
        enqueue_out(w, b.x2);
        enqueue_moe(w);
        probe(K_HEAD); enqueue_head(w.head_norm, false, draft_rows > 0); probe(K_HEAD);
    }
    void enqueue_mtp_seed(const RunCtl *rc = nullptr) {
        if (fused) {
            if (!fz_capturing) fz_account(1);
            launch_fused(rc ? rc : ctl, fz_args + FM_SEED, fz_grid, fz_lds, st);
            return;
        }
        const LayerW &w = L[d.n_layer];
        enqueue_entry(w);
        enqueue_proj(w, b.x2, false, nullptr, AT_K);  // K and V rows only
        launch_kwrite(ctl, m, w, b, st);
    }

    // ---- host-driven API (mirrors Engine::{verify, commit, mtp_run, mtp_seed}) ----
    int read_argmax(uint32_t *out, int n) {
        const int nk = nkeys();
        std::vector<unsigned long long> k((size_t)OXE_NL * nk);
        if (hipMemcpyAsync(k.data(), keys(), k.size() * 8, hipMemcpyDeviceToHost, st) != hipSuccess) return -2;
        if (hipStreamSynchronize(st) != hipSuccess) return -2;
        if (int rc = fused_check()) return rc;
        for (int i = 0; i < n; i++) {
            unsigned long long best = 0ull;
            for (int j = 0; j < nk; j++) best = k[(size_t)i * nk + j] > best ? k[(size_t)i * nk + j] : best;
            out[i] = best == 0 ? 0u : 0xffffffffu - (uint32_t)(best & 0xffffffffu);
        }
        return 0;
    }
    RunCtl run(int nl, int pos0, const uint32_t *toks, int head_mask) const {
        RunCtl r{};
        r.nl = nl;
        r.pos0 = pos0;
        r.cur = cur;
        r.head_mask = head_mask;
        for (int i = 0; i < nl; i++) r.tok[i] = toks[i];
        r.hin_sel[0] = HID_HL;
        r.hin_sel[1] = HID_PEND;
        r.active = 1;
        return r;
    }
    // token ids index the embedding rows: every id from the host is checked before any launch
    bool toks_ok(const uint32_t *toks, int n) const {
        if (!toks) return false;
        for (int i = 0; i < n; i++)
            if (toks[i] >= (uint32_t)d.n_vocab) return false;
        return true;
    }
    int verify(const uint32_t *toks, int n, uint32_t *out) {
        if (n < 1 || n > OXE_NL || pos + n > m.n_ctx || !toks_ok(toks, n)) return -1;
        launch_set_run(ctl, run(n, pos, toks, (1 << n) - 1), st);
        enqueue_verify();
        pend_pos0 = pos;
        pend_cur = cur;
        pend_n = n;
        pend_done = 0;
        return read_argmax(out, n);
    }
    // back to position p_new < pos of the current host-driven step, whose state after position
    // p_new - 1 is in slot cur_new (an earlier verify piece of the step): V^T of the positions
    // after it back to +0, no pending verify
    int rollback(int p_new, int cur_new) {
        if (p_new < 0 || p_new > pos || cur_new < 0 || cur_new >= OXE_NSLOTS) return -1;
        launch_zero_v(m, n_att_main, p_new, pos, st);
        pos = p_new;
        cur = cur_new;
        pend_n = 0;
        return hipStreamSynchronize(st) == hipSuccess ? 0 : -2;
    }
    int commit(int mm) {
        if (pend_n == 0) return -1;
        const int hi = pend_done == 0 ? pend_n : pend_done;
        if (mm < 1 || mm > hi) return -1;
        launch_zero_v(m, n_att_main, pend_pos0 + mm, pend_pos0 + hi, st);
        pos = pend_pos0 + mm;
        cur = (pend_cur + mm) % OXE_NSLOTS;
        pend_done = mm;
        return hipStreamSynchronize(st) == hipSuccess ? 0 : -2;
    }
    int set_hidden(const float *hs, int n) {
        // lane i of an MTP run reads hid[HID_HL + i]
        return hipMemcpyAsync(b.hid + (size_t)HID_HL * E, hs, (size_t)n * E * 4, hipMemcpyHostToDevice, st) == hipSuccess ? 0 : -2;
    }
    int mtp_run(const uint32_t *toks, int n, int pos0, const float *hs, int head_last, uint32_t *out) {
        if (n < 1 || n > OXE_NL || pos0 < 0 || pos0 + n > m.n_ctx || !toks_ok(toks, n) || !hs) return -1;
        if (set_hidden(hs, n)) return -2;
        launch_set_run(ctl, run(n, pos0, toks, head_last ? 1 << (n - 1) : 0), st);
        enqueue_mtp_run();
        uint32_t a[OXE_NL];
        if (read_argmax(a, n)) return -2;
        *out = head_last ? a[n - 1] : 0xffffffffu;
        return 0;
    }
    int mtp_seed(const uint32_t *toks, int n, int pos0, const float *hs) {
        if (n < 1 || n > OXE_NL || pos0 < 0 || pos0 + n > m.n_ctx || !toks_ok(toks, n) || !hs) return -1;
        if (set_hidden(hs, n)) return -2;
        launch_set_run(ctl, run(n, pos0, toks, 0), st);
        enqueue_mtp_seed();
        if (hipStreamSynchronize(st) != hipSuccess) return -2;
        return fused_check();
    }
};

}  // namespace oxe
