// Weight loader (WeightStore::load, crates/model/src/weights.rs:556-700, for the device): every
// tensor the engine reads is taken from a GGUF file (gguf.cpp) into the engine's device arrays in
// the kernels' layout. Q8_0 matmul weights are split on the device from ggml's 34-byte blocks
// (fp16 d, 32 int8 codes) into codes [rows][k] + fp16 scales [rows][k/32] (the form every GEMV /
// GEMM kernel here reads, in place of the reference's 4-row interleave, oxe_shim.cpp:9-29),
// concatenated per projection ([qkv | z | beta | alpha], [q+gate | k | v]) and, for gate / up
// pairs, interleaved per 16-row tile (8 gate rows, then 8 up rows). F32 vectors and matrices are
// copied. The expert, shared-expert and output matrices may also be K-quants (Q3_K..Q6_K) and
// ssm_beta / ssm_alpha F32 (the types a Qwen3.6 file holds there): those are copied in the file's
// own blocks, for an engine created with those types (model_types reads them from the file). Any
// other tensor type is refused with the tensor's name.
#include <algorithm>
#include <mutex>
#include <string>

#include "oxe_engine_host.h"
#include "oxe_gguf.h"

namespace oxe {

namespace ld {

// rows of raw Q8_0 blocks -> codes + scales; source row R (of `rows`, `grp_rows` per group, e.g.
// per expert) goes to destination row dst0 + (R / grp_rows) * dst_grp + map(R % grp_rows), map =
// identity, or the gate / up tile interleave 16 (r / 8) + il + r % 8 (il 0 gate, 8 up)
__global__ void q8_split_kernel(const uint8_t *src, int64_t rows, int64_t k, int64_t grp_rows, int64_t dst_grp,
                                int64_t dst0, int il, int8_t *q, uint16_t *d) {
    const int64_t nbr = k / 32, nb = rows * nbr;
    for (int64_t b = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; b < nb; b += (int64_t)gridDim.x * blockDim.x) {
        const int64_t R = b / nbr, kb = b % nbr, g = R / grp_rows, r = R % grp_rows;
        const int64_t dr = dst0 + g * dst_grp + (il < 0 ? r : 16 * (r / 8) + il + r % 8);
        const uint16_t *blk = (const uint16_t *)(src + b * 34);   // 34-byte blocks: 2-byte aligned
        uint32_t w[8];
#pragma unroll
        for (int i = 0; i < 8; i++) w[i] = (uint32_t)blk[1 + 2 * i] | ((uint32_t)blk[2 + 2 * i] << 16);
        uint4 *dst = (uint4 *)(q + dr * k + kb * 32);
        dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
        dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
        d[dr * nbr + kb] = blk[0];
    }
}

}  // namespace ld

// host-visible status of a load: "" or the first problem
static std::string tensor_check(const GgufTensor *t, const std::string &name, uint32_t type,
                                std::initializer_list<uint64_t> shape) {
    if (!t) return "missing tensor " + name;
    GgmlTypeInfo ti{};
    ggml_type_info(t->type, &ti);
    if (t->type != type) {
        GgmlTypeInfo want{};
        ggml_type_info(type, &want);
        const bool kq = t->type >= 11 && t->type <= 14;
        if ((kq || t->type == GGML_F32) && type == GGML_Q8_0)
            return name + ": type " + (ti.name ? ti.name : "unknown") + " has no kernel for this tensor here (Q8_0 " +
                   "expected; K-quants load for the expert, shared-expert and output matrices, F32 for ssm_beta / " +
                   "ssm_alpha, of an engine created from the file)";
        return name + ": type " + (ti.name ? ti.name : "unknown") + " has no kernel in this build (expected " +
               want.name + ": Q8_0 or K-quant matmul weights, F32 or BF16 vectors and routers)";
    }
    if (t->shape != std::vector<uint64_t>(shape)) return name + ": unexpected shape";
    return "";
}

// The types of the matrices that may be other than Q8_0, as the file holds them: gate / up of the
// experts (or of the shared expert) both Q8_0 or both K-quants, down Q8_0 or a K-quant; a delta-net
// layer's attn_qkv and attn_gate both K-quants (its ssm_beta / ssm_alpha then both K-quants or both
// F32) or both Q8_0 (ssm_beta / ssm_alpha both Q8_0 or both F32); an attention layer's attn_q /
// attn_k / attn_v all K-quants or all Q8_0; ssm_out / attn_output, the token embedding and the LM
// head Q8_0 or a K-quant. A tensor of any other type or combination keeps Q8_0 here, and the load
// refuses it by name.
ModelTypes model_types(const Gguf &g, const oxe_model_desc &d) {
    ModelTypes mt;
    mt.layer.assign(d.n_layer + 1, LayerTypes{});
    auto ty = [&](const std::string &name) { const GgufTensor *t = g.tensor(name); return t ? (int)t->type : -1; };
    auto kq = [](int t) { return t >= 11 && t <= 14; };
    for (int il = 0; il <= d.n_layer; il++) {
        LayerTypes &lt = mt.layer[il];
        const std::string p = "blk." + std::to_string(il) + ".";
        const int g0 = ty(p + "ffn_gate_exps.weight"), u0 = ty(p + "ffn_up_exps.weight"), d0 = ty(p + "ffn_down_exps.weight");
        if (kq(g0) && kq(u0)) { lt.gate = g0; lt.up = u0; }
        if (kq(d0)) lt.down = d0;
        const int g1 = ty(p + "ffn_gate_shexp.weight"), u1 = ty(p + "ffn_up_shexp.weight"), d1 = ty(p + "ffn_down_shexp.weight");
        if (kq(g1) && kq(u1)) { lt.sh_gate = g1; lt.sh_up = u1; }
        if (kq(d1)) lt.sh_down = d1;
        const int b0 = ty(p + "ssm_beta.weight"), a0 = ty(p + "ssm_alpha.weight");
        const bool f32ba = b0 == (int)GGML_F32 && a0 == (int)GGML_F32;
        if (f32ba) lt.beta = lt.alpha = 0;
        const int qkv = ty(p + "attn_qkv.weight"), z = ty(p + "attn_gate.weight");
        if (kq(qkv) && kq(z) && (f32ba || (kq(b0) && kq(a0)))) {
            lt.qkv = qkv;
            lt.z = z;
            if (!f32ba) { lt.beta = b0; lt.alpha = a0; }
        }
        const int q = ty(p + "attn_q.weight"), k = ty(p + "attn_k.weight"), v = ty(p + "attn_v.weight");
        if (kq(q) && kq(k) && kq(v)) { lt.q = q; lt.k = k; lt.v = v; }
        const int out = ty(p + (g.tensor(p + "ssm_out.weight") ? "ssm_out.weight" : "attn_output.weight"));
        if (kq(out)) lt.out = out;
    }
    const int o = ty("output.weight");
    if (kq(o)) mt.output = o;
    const int e = ty("token_embd.weight");
    if (kq(e)) mt.tok_embd = e;
    return mt;
}

int Engine::load_gguf(const Gguf &g, uint8_t *given_stage, int64_t given_chunk) {
    const int64_t CHUNK = given_stage ? given_chunk : 256ll << 20;   // staging bytes per upload
    // the reference's MTP loader refuses a draft head with its own embedding or LM head (mtp.rs:97-99)
    const std::string mp = "blk." + std::to_string(d.n_layer) + ".";
    if (g.tensor(mp + "nextn.embed_tokens.weight") || g.tensor(mp + "nextn.shared_head_head.weight")) {
        set_err("MTP head with its own embedding/head is not supported (both GGUFs share the target's)");
        return -1;
    }
    uint8_t *stage = given_stage;
    if (!stage && hipMalloc(&stage, CHUNK) != hipSuccess) {
        set_err("out of device memory for the load staging buffer");
        return -3;
    }
    std::string err;
    int rc = 0;
    // Q8_0 tensor of rows x k (x n_grp groups) into (q, d) with the row mapping of q8_split_kernel
    auto q8 = [&](const std::string &name, int64_t k, int64_t rows, int64_t n_grp, int8_t *q, uint16_t *d,
                  int64_t dst0, int64_t dst_grp, int il) {
        if (!err.empty()) return;
        const GgufTensor *t = g.tensor(name);
        err = n_grp > 1 ? tensor_check(t, name, GGML_Q8_0, {(uint64_t)k, (uint64_t)rows, (uint64_t)n_grp})
                        : tensor_check(t, name, GGML_Q8_0, {(uint64_t)k, (uint64_t)rows});
        if (!err.empty()) return;
        const int64_t row_bytes = k / 32 * 34, grp_bytes = rows * row_bytes;
        const uint8_t *src = g.data(*t);
        auto launch = [&](int64_t off, int64_t n_rows, int64_t grp_rows, int64_t d0) {
            if (hipMemcpyAsync(stage, src + off, (size_t)(n_rows * row_bytes), hipMemcpyHostToDevice, st) != hipSuccess) {
                rc = -2;
                return;
            }
            const int64_t nb = n_rows * (k / 32);
            hipLaunchKernelGGL(ld::q8_split_kernel, dim3((unsigned)std::min<int64_t>((nb + 255) / 256, 65535)), dim3(256),
                               0, st, stage, n_rows, k, grp_rows, dst_grp, d0, il, q, d);
            if (hipGetLastError() != hipSuccess) rc = -2;
        };
        if (n_grp == 1) {
            // one matrix, in row chunks (an interleaved gate / up matrix is one chunk: the tile
            // mapping needs the matrix-local row)
            if (il >= 0 && grp_bytes > CHUNK) {
                err = name + ": interleaved matrix larger than the staging buffer";
                return;
            }
            const int64_t per = std::max<int64_t>(1, CHUNK / row_bytes);
            for (int64_t r0 = 0; r0 < rows && !rc; r0 += per) {
                const int64_t n = std::min(per, rows - r0);
                launch(r0 * row_bytes, n, il >= 0 ? rows : ((int64_t)1 << 62), dst0 + (il >= 0 ? 0 : r0));
            }
        } else {
            // per-expert groups, whole groups per chunk
            const int64_t per = std::max<int64_t>(1, CHUNK / grp_bytes);
            if (grp_bytes > CHUNK) {
                err = name + ": expert matrix larger than the staging buffer";
                return;
            }
            for (int64_t g0 = 0; g0 < n_grp && !rc; g0 += per) {
                const int64_t n = std::min(per, n_grp - g0);
                launch(g0 * grp_bytes, n * rows, rows, dst0 + g0 * dst_grp);
            }
        }
    };
    // a matrix kept in the file's blocks (K-quant or F32): copied as it is, in chunks
    auto raw = [&](const std::string &name, const RawW &r, std::initializer_list<uint64_t> shape) {
        if (!err.empty()) return;
        const GgufTensor *t = g.tensor(name);
        err = tensor_check(t, name, (uint32_t)r.type, shape);
        if (!err.empty()) return;
        const uint8_t *src = g.data(*t);
        const int64_t n = (int64_t)t->bytes();
        for (int64_t off = 0; off < n && !rc; off += CHUNK)
            if (hipMemcpyAsync(r.w + off, src + off, (size_t)std::min(CHUNK, n - off), hipMemcpyHostToDevice, st) != hipSuccess)
                rc = -2;
    };
    // F32 vectors and routers; BF16 ones widened to f32 (exact: the bf16 bits are the high half of
    // the f32), as the reference converts BF16 small tensors at load (crates/model/src/mtp.rs:109-128)
    auto f32 = [&](const std::string &name, std::initializer_list<uint64_t> shape, float *dst) {
        if (!err.empty()) return;
        const GgufTensor *t = g.tensor(name);
        if (t && t->type == GGML_BF16) {
            err = tensor_check(t, name, GGML_BF16, shape);
            if (!err.empty()) return;
            const uint16_t *src = (const uint16_t *)g.data(*t);
            const size_t n = (size_t)t->bytes() / 2;
            std::vector<uint32_t> wide(n);
            for (size_t i = 0; i < n; i++) wide[i] = (uint32_t)src[i] << 16;
            if (hipMemcpy(dst, wide.data(), n * 4, hipMemcpyHostToDevice) != hipSuccess) rc = -2;
            return;
        }
        err = tensor_check(t, name, GGML_F32, shape);
        if (!err.empty()) return;
        if (hipMemcpyAsync(dst, g.data(*t), (size_t)t->bytes(), hipMemcpyHostToDevice, st) != hipSuccess) rc = -2;
    };
    const int nl_total = d.n_layer + 1;
    for (int il = 0; il < nl_total && err.empty() && !rc; il++) {
        LayerW &w = L[il];
        const std::string p = "blk." + std::to_string(il) + ".";
        f32(p + "attn_norm.weight", {E}, w.attn_norm);
        f32(p + "post_attention_norm.weight", {E}, w.post_norm);
        if (!w.att) {
            if (w.qkv_r.type == 8) {
                q8(p + "attn_qkv.weight", E, NCH, 1, w.proj.q, w.proj.d, 0, 0, -1);
                q8(p + "attn_gate.weight", E, DIN, 1, w.proj.q, w.proj.d, DN_Z, 0, -1);
            } else {
                raw(p + "attn_qkv.weight", w.qkv_r, {E, NCH});
                raw(p + "attn_gate.weight", w.z_r, {E, DIN});
            }
            if (w.beta_r.type == 8) {
                q8(p + "ssm_beta.weight", E, NVH, 1, w.proj.q, w.proj.d, DN_BETA, 0, -1);
                q8(p + "ssm_alpha.weight", E, NVH, 1, w.proj.q, w.proj.d, DN_ALPHA, 0, -1);
            } else {
                raw(p + "ssm_beta.weight", w.beta_r, {E, NVH});
                raw(p + "ssm_alpha.weight", w.alpha_r, {E, NVH});
            }
            if (w.out_r.type == 8) q8(p + "ssm_out.weight", DIN, E, 1, w.out.q, w.out.d, 0, 0, -1);
            else raw(p + "ssm_out.weight", w.out_r, {DIN, E});
            f32(p + "ssm_conv1d.weight", {KC, NCH}, w.conv);
            f32(p + "ssm_a", {NVH}, w.ssm_a);
            f32(p + "ssm_dt.bias", {NVH}, w.dt_bias);
            f32(p + "ssm_norm.weight", {HV}, w.ssm_norm);
        } else {
            if (w.q_r.type == 8) {
                q8(p + "attn_q.weight", E, NH * 2 * HD, 1, w.proj.q, w.proj.d, 0, 0, -1);
                q8(p + "attn_k.weight", E, NKV * HD, 1, w.proj.q, w.proj.d, AT_K, 0, -1);
                q8(p + "attn_v.weight", E, NKV * HD, 1, w.proj.q, w.proj.d, AT_V, 0, -1);
            } else {
                raw(p + "attn_q.weight", w.q_r, {E, NH * 2 * HD});
                raw(p + "attn_k.weight", w.k_r, {E, NKV * HD});
                raw(p + "attn_v.weight", w.v_r, {E, NKV * HD});
            }
            if (w.out_r.type == 8) q8(p + "attn_output.weight", NH * HD, E, 1, w.out.q, w.out.d, 0, 0, -1);
            else raw(p + "attn_output.weight", w.out_r, {NH * HD, E});
            f32(p + "attn_q_norm.weight", {HD}, w.q_norm);
            f32(p + "attn_k_norm.weight", {HD}, w.k_norm);
        }
        f32(p + "ffn_gate_inp.weight", {E, NEXP}, w.router);
        f32(p + "ffn_gate_inp_shexp.weight", {E}, w.shexp_gate);
        if (w.sh_gate_r.type == 8) {
            q8(p + "ffn_gate_shexp.weight", E, FFSH, 1, w.shexp_gu.q, w.shexp_gu.d, 0, 0, 0);
            q8(p + "ffn_up_shexp.weight", E, FFSH, 1, w.shexp_gu.q, w.shexp_gu.d, 0, 0, 8);
        } else {
            raw(p + "ffn_gate_shexp.weight", w.sh_gate_r, {E, FFSH});
            raw(p + "ffn_up_shexp.weight", w.sh_up_r, {E, FFSH});
        }
        if (w.sh_down_r.type == 8) q8(p + "ffn_down_shexp.weight", FFSH, E, 1, w.shexp_down.q, w.shexp_down.d, 0, 0, -1);
        else raw(p + "ffn_down_shexp.weight", w.sh_down_r, {FFSH, E});
        if (w.exp_gate_r.type == 8) {
            q8(p + "ffn_gate_exps.weight", E, FF, NEXP, w.exp_gu.q, w.exp_gu.d, 0, 2 * FF, 0);
            q8(p + "ffn_up_exps.weight", E, FF, NEXP, w.exp_gu.q, w.exp_gu.d, 0, 2 * FF, 8);
        } else {
            raw(p + "ffn_gate_exps.weight", w.exp_gate_r, {E, FF, NEXP});
            raw(p + "ffn_up_exps.weight", w.exp_up_r, {E, FF, NEXP});
        }
        if (w.exp_down_r.type == 8) q8(p + "ffn_down_exps.weight", FF, E, NEXP, w.exp_down.q, w.exp_down.d, 0, E, -1);
        else raw(p + "ffn_down_exps.weight", w.exp_down_r, {FF, E, NEXP});
        if (il == d.n_layer) {
            q8(p + "nextn.eh_proj.weight", 2 * E, E, 1, w.eh_proj.q, w.eh_proj.d, 0, 0, -1);
            f32(p + "nextn.enorm.weight", {E}, w.enorm);
            f32(p + "nextn.hnorm.weight", {E}, w.hnorm);
            f32(p + "nextn.shared_head_norm.weight", {E}, w.head_norm);
        }
    }
    if (m.tok_embd_r.type == 8) q8("token_embd.weight", E, d.n_vocab, 1, m.tok_embd.q, m.tok_embd.d, 0, 0, -1);
    else raw("token_embd.weight", m.tok_embd_r, {E, (uint64_t)d.n_vocab});
    if (m.output_r.type == 8) q8("output.weight", E, d.n_vocab, 1, m.output.q, m.output.d, 0, 0, -1);
    else raw("output.weight", m.output_r, {E, (uint64_t)d.n_vocab});
    f32("output_norm.weight", {E}, m.out_norm);
    const hipError_t se = hipStreamSynchronize(st);
    if (!given_stage) (void)hipFree(stage);
    if (!err.empty()) {
        set_err(err);
        return -1;
    }
    if (rc || se != hipSuccess) return -2;
    return 0;
}

// ---- staging of the allocation-free loader -----------------------------------------------------
// A file-scope device array (each GPU the library runs on holds its own copy until the process
// ends). Host code never passes `load_scratch` itself to a kernel or copy (on the host it names a
// stand-in, not device memory): its device address is looked up once per device with that device
// current and kept in load_scratch_ptr.
constexpr int64_t LOAD_SCRATCH_BYTES = 16ll << 20;
constexpr int LOAD_SCRATCH_MAX_DEV = 64;
static __device__ __align__(256) uint8_t load_scratch[LOAD_SCRATCH_BYTES];
static std::mutex load_scratch_mu;
static uint8_t *load_scratch_ptr[LOAD_SCRATCH_MAX_DEV];
// held by an allocation-free load from its first upload until its final stream synchronisation, so
// overlapping calls on one GPU (other threads, other streams) take turns with the array
static std::mutex load_stage_mu[LOAD_SCRATCH_MAX_DEV];

// the device address of device dev's load_scratch (dev must be current); null on failure
static uint8_t *load_scratch_of(int dev) {
    if (dev < 0 || dev >= LOAD_SCRATCH_MAX_DEV) return nullptr;
    std::lock_guard<std::mutex> lk(load_scratch_mu);
    if (!load_scratch_ptr[dev]) {
        void *p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(load_scratch)) != hipSuccess || !p) return nullptr;
        load_scratch_ptr[dev] = (uint8_t *)p;
    }
    return load_scratch_ptr[dev];
}

}  // namespace oxe

extern "C" {

// the file's descriptor against the engine's (0: equal)
static int load_gguf_check(oxe_engine *e, const oxe_gguf *gg) {
    oxe::Engine *g = (oxe::Engine *)e;
    oxe_model_desc d;
    if (oxe_gguf_model_desc(gg, &d)) return -1;
    // every descriptor field the kernels and the RoPE table depend on must equal the engine's
    const oxe_model_desc &c = g->d;
    bool same = d.n_layer == c.n_layer && d.n_embd == c.n_embd && d.n_vocab == c.n_vocab && d.n_head == c.n_head &&
                d.n_head_kv == c.n_head_kv && d.head_dim == c.head_dim && d.n_expert == c.n_expert &&
                d.n_expert_used == c.n_expert_used && d.ff_exp == c.ff_exp && d.ff_shexp == c.ff_shexp &&
                d.ssm_conv_kernel == c.ssm_conv_kernel && d.ssm_d_state == c.ssm_d_state &&
                d.ssm_n_kheads == c.ssm_n_kheads && d.ssm_n_vheads == c.ssm_n_vheads && d.ssm_d_inner == c.ssm_d_inner &&
                d.full_attention_interval == c.full_attention_interval && d.n_rot == c.n_rot &&
                d.rms_eps == c.rms_eps && d.rope_freq_base == c.rope_freq_base && d.has_mtp && c.has_mtp;
    for (int i = 0; i < 4; i++) same = same && d.rope_sections[i] == c.rope_sections[i];
    if (!same) {
        oxe::set_err("the file's model descriptor (shape, norms' eps, RoPE, layer pattern, MTP block) differs from the engine's");
        return -1;
    }
    return 0;
}

int oxe_engine_load_gguf_noalloc(oxe_engine *e, const oxe_gguf *gg) {
    oxe::Engine *g = (oxe::Engine *)e;
    if (!g || !gg) return -1;
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return -2;
    if (cur != g->dev) {
        oxe::set_err("load_gguf_noalloc: the engine's device must be current");
        return -1;
    }
    uint8_t *stage = oxe::load_scratch_of(cur);
    if (!stage) {
        oxe::set_err("load_gguf_noalloc: no device address for the staging array");
        return -2;
    }
    const int rc = load_gguf_check(e, gg);
    if (rc) return rc;
    // every upload goes through the 16 MiB array: a tensor group that must be staged whole (one
    // expert's matrix, an interleaved gate / up matrix) above that size is refused by name. The
    // device's staging lock is held until load_gguf has synchronised its stream (every copy out of
    // the array has completed).
    std::lock_guard<std::mutex> lk(oxe::load_stage_mu[cur]);
    return g->load_gguf(*(const oxe::Gguf *)gg, stage, oxe::LOAD_SCRATCH_BYTES);
}

int oxe_hip_repack_q8_0(const void *src, int64_t nrows, int64_t k, int8_t *q, uint16_t *d, void *stream) {
    if (!src || !q || !d || nrows <= 0 || k <= 0 || k % 32 != 0) return -1;
    const int64_t nb = nrows * (k / 32);
    hipLaunchKernelGGL(oxe::ld::q8_split_kernel, dim3((unsigned)std::min<int64_t>((nb + 255) / 256, 65535)), dim3(256), 0,
                       (hipStream_t)stream, (const uint8_t *)src, nrows, k, (int64_t)1 << 62, (int64_t)0, (int64_t)0, -1,
                       q, d);
    return hipGetLastError() == hipSuccess ? 0 : -2;
}

int oxe_engine_load_gguf(oxe_engine *e, const oxe_gguf *gg) {
    oxe::Engine *g = (oxe::Engine *)e;
    const oxe::Gguf *f = (const oxe::Gguf *)gg;
    if (!g || !f) return -1;
    const int rc = load_gguf_check(e, gg);
    if (rc) return rc;
    return g->load_gguf(*f);
}

int oxe_engine_create_from_gguf(const char *path, int n_ctx, oxe_engine **out) {
    if (!out) return -1;
    oxe_gguf *f = nullptr;
    int rc = oxe_gguf_open(path, &f);
    if (rc) return rc;
    oxe_model_desc d;
    if ((rc = oxe_gguf_model_desc(f, &d))) {
        oxe_gguf_close(f);
        return rc;
    }
    if (!d.has_mtp) {
        oxe::set_err("the file has no nextn (MTP) block: this engine runs MTP depth-1 decoding");
        oxe_gguf_close(f);
        return -1;
    }
    oxe_engine *e = nullptr;
    const oxe::ModelTypes mt = oxe::model_types(*(const oxe::Gguf *)f, d);
    if ((rc = oxe::create_engine(&d, 0, n_ctx, false, nullptr, &mt, &e))) {
        oxe_gguf_close(f);
        return rc;
    }
    rc = oxe_engine_load_gguf(e, f);
    oxe_gguf_close(f);
    if (rc) {
        oxe_engine_destroy(e);
        return rc;
    }
    *out = e;
    return 0;
}

}  // extern "C"
