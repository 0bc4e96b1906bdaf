// GGUF reader (host side of the weight loader). See oxe_gguf.h for the contract.
#include "oxe_gguf.h"

#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <cstring>

namespace oxe {

bool ggml_type_info(uint32_t ty, GgmlTypeInfo *out) {
    static const struct { uint32_t id; GgmlTypeInfo t; } table[] = {
        {0, {"F32", 1, 4}},        {1, {"F16", 1, 2}},        {2, {"Q4_0", 32, 18}},     {3, {"Q4_1", 32, 20}},
        {6, {"Q5_0", 32, 22}},     {7, {"Q5_1", 32, 24}},     {8, {"Q8_0", 32, 34}},     {9, {"Q8_1", 32, 36}},
        {10, {"Q2_K", 256, 84}},   {11, {"Q3_K", 256, 110}},  {12, {"Q4_K", 256, 144}},  {13, {"Q5_K", 256, 176}},
        {14, {"Q6_K", 256, 210}},  {15, {"Q8_K", 256, 292}},  {16, {"IQ2_XXS", 256, 66}}, {17, {"IQ2_XS", 256, 74}},
        {18, {"IQ3_XXS", 256, 98}}, {19, {"IQ1_S", 256, 50}}, {20, {"IQ4_NL", 32, 18}},  {21, {"IQ3_S", 256, 110}},
        {22, {"IQ2_S", 256, 82}},  {23, {"IQ4_XS", 256, 136}}, {24, {"I8", 1, 1}},       {25, {"I16", 1, 2}},
        {26, {"I32", 1, 4}},       {27, {"I64", 1, 8}},       {28, {"F64", 1, 8}},       {29, {"IQ1_M", 256, 56}},
        {30, {"BF16", 1, 2}},      {34, {"TQ1_0", 256, 54}},  {35, {"TQ2_0", 256, 66}},  {39, {"MXFP4", 32, 17}},
        {40, {"NVFP4", 64, 36}},   {41, {"Q1_0", 128, 18}},   {42, {"Q2_0", 64, 18}},    {43, {"F8_E4M3", 1, 1}},
    };
    for (const auto &e : table)
        if (e.id == ty) {
            if (out) *out = e.t;
            return true;
        }
    return false;
}

bool GgufValue::as_u64(uint64_t *out) const {
    switch (type) {
    case GV_U8: case GV_U16: case GV_U32: case GV_U64: *out = u; return true;
    case GV_I8: case GV_I16: case GV_I32: case GV_I64:
        if (i < 0) return false;
        *out = (uint64_t)i;
        return true;
    default: return false;
    }
}

bool GgufValue::as_f64(double *out) const {
    if (type == GV_F32 || type == GV_F64) {
        *out = f;
        return true;
    }
    uint64_t v;
    if (!as_u64(&v)) return false;
    *out = (double)v;
    return true;
}

static bool mul_ok(uint64_t a, uint64_t b, uint64_t *r) { return !__builtin_mul_overflow(a, b, r); }

uint64_t GgufTensor::elements() const {
    uint64_t n = 1;
    for (uint64_t d : shape)
        if (!mul_ok(n, d, &n)) return UINT64_MAX;
    return n;
}

uint64_t GgufTensor::bytes() const {
    GgmlTypeInfo ti;
    const uint64_t n = elements();
    if (!ggml_type_info(type, &ti) || n == UINT64_MAX) return UINT64_MAX;
    uint64_t b;
    return mul_ok(n / ti.blk, ti.size, &b) ? b : UINT64_MAX;
}

Gguf::~Gguf() {
    if (map) munmap((void *)map, map_len);
}

const GgufValue *Gguf::get(const std::string &key) const {
    for (const auto &kv : meta)
        if (kv.first == key) return &kv.second;
    return nullptr;
}

const GgufTensor *Gguf::tensor(const std::string &name) const {
    for (const auto &t : tensors)
        if (t.name == name) return &t;
    return nullptr;
}

namespace {

constexpr uint64_t LONG_ARRAY = 4096;   // longer metadata arrays keep only their length
constexpr uint32_t MAX_DIMS = 4;

struct Reader {
    const uint8_t *p;
    size_t len, pos = 0;
    bool take(size_t n, const uint8_t **out) {
        if (n > len - pos) return false;
        *out = p + pos;
        pos += n;
        return true;
    }
    template <class T>
    bool scalar(T *v) {
        const uint8_t *b;
        if (!take(sizeof(T), &b)) return false;
        std::memcpy(v, b, sizeof(T));   // little-endian host
        return true;
    }
    bool str(std::string *s) {
        uint64_t n;
        const uint8_t *b;
        if (!scalar(&n) || n > len - pos || !take((size_t)n, &b)) return false;
        s->assign((const char *)b, (size_t)n);
        return true;
    }
};

int scalar_size(uint32_t t) {
    switch (t) {
    case GV_U8: case GV_I8: case GV_BOOL: return 1;
    case GV_U16: case GV_I16: return 2;
    case GV_U32: case GV_I32: case GV_F32: return 4;
    case GV_U64: case GV_I64: case GV_F64: return 8;
    default: return 0;
    }
}

const char *TRUNC = "truncated GGUF header";

std::string read_value(Reader &r, uint32_t vt, GgufValue &v, int depth) {
    v.type = vt;
    switch (vt) {
    case GV_U8: { uint8_t x; if (!r.scalar(&x)) return TRUNC; v.u = x; v.i = x; break; }
    case GV_I8: { int8_t x; if (!r.scalar(&x)) return TRUNC; v.i = x; v.u = (uint64_t)(int64_t)x; break; }
    case GV_U16: { uint16_t x; if (!r.scalar(&x)) return TRUNC; v.u = x; v.i = x; break; }
    case GV_I16: { int16_t x; if (!r.scalar(&x)) return TRUNC; v.i = x; v.u = (uint64_t)(int64_t)x; break; }
    case GV_U32: { uint32_t x; if (!r.scalar(&x)) return TRUNC; v.u = x; v.i = x; break; }
    case GV_I32: { int32_t x; if (!r.scalar(&x)) return TRUNC; v.i = x; v.u = (uint64_t)(int64_t)x; break; }
    case GV_F32: { float x; if (!r.scalar(&x)) return TRUNC; v.f = x; break; }
    case GV_BOOL: { uint8_t x; if (!r.scalar(&x)) return TRUNC; v.u = x != 0; break; }
    case GV_STR: if (!r.str(&v.s)) return TRUNC; break;
    case GV_U64: { uint64_t x; if (!r.scalar(&x)) return TRUNC; v.u = x; v.i = (int64_t)x; break; }
    case GV_I64: { int64_t x; if (!r.scalar(&x)) return TRUNC; v.i = x; v.u = (uint64_t)x; break; }
    case GV_F64: { double x; if (!r.scalar(&x)) return TRUNC; v.f = x; break; }
    case GV_ARR: {
        if (depth > 8) return "metadata arrays nested too deep";
        uint32_t it;
        uint64_t n;
        if (!r.scalar(&it) || !r.scalar(&n)) return TRUNC;
        v.item_type = it;
        v.len = n;
        if (n > LONG_ARRAY) {
            v.long_array = true;
            const int sz = scalar_size(it);
            if (sz) {
                uint64_t bytes;
                const uint8_t *b;
                if (!mul_ok(n, (uint64_t)sz, &bytes) || bytes > r.len - r.pos) return "metadata array too long";
                r.take((size_t)bytes, &b);
            } else {
                for (uint64_t k = 0; k < n; k++) {
                    GgufValue tmp;
                    const std::string e = read_value(r, it, tmp, depth + 1);
                    if (!e.empty()) return e;
                }
            }
        } else {
            v.arr.resize((size_t)n);
            for (uint64_t k = 0; k < n; k++) {
                const std::string e = read_value(r, it, v.arr[(size_t)k], depth + 1);
                if (!e.empty()) return e;
            }
        }
        break;
    }
    default: return "unknown metadata value type " + std::to_string(vt);
    }
    return "";
}

}  // namespace

std::string gguf_parse(const uint8_t *buf, size_t len, Gguf &g) {
    Reader r{buf, len};
    const uint8_t *magic;
    if (!r.take(4, &magic) || std::memcmp(magic, "GGUF", 4) != 0) return "not a GGUF file";
    uint64_t n_tensors, n_kv;
    if (!r.scalar(&g.version)) return TRUNC;
    if (g.version != 2 && g.version != 3) return "unsupported GGUF version " + std::to_string(g.version);
    if (!r.scalar(&n_tensors) || !r.scalar(&n_kv)) return TRUNC;
    // a key/value takes at least 12 bytes and a tensor entry 24: counts the rest of the file cannot
    // hold are refused before anything is reserved
    const uint64_t left = len - r.pos;
    if (n_kv > left / 12 || n_tensors > left / 24)
        return "GGUF header claims " + std::to_string(n_kv) + " keys / " + std::to_string(n_tensors) +
               " tensors, more than its " + std::to_string(left) + " bytes hold";
    g.meta.reserve((size_t)n_kv);
    for (uint64_t k = 0; k < n_kv; k++) {
        std::string key;
        uint32_t vt;
        if (!r.str(&key) || !r.scalar(&vt)) return TRUNC;
        GgufValue v;
        const std::string e = read_value(r, vt, v, 0);
        if (!e.empty()) return e;
        g.meta.emplace_back(std::move(key), std::move(v));
    }
    g.tensors.reserve((size_t)n_tensors);
    for (uint64_t k = 0; k < n_tensors; k++) {
        GgufTensor t;
        uint32_t nd;
        if (!r.str(&t.name) || !r.scalar(&nd)) return TRUNC;
        if (nd > MAX_DIMS) return t.name + ": " + std::to_string(nd) + " dimensions (ggml has at most 4)";
        for (uint32_t i = 0; i < nd; i++) {
            uint64_t dim;
            if (!r.scalar(&dim)) return TRUNC;
            if (dim > (uint64_t)INT64_MAX) return t.name + ": dimension above 2^63";
            t.shape.push_back(dim);
        }
        if (!r.scalar(&t.type) || !r.scalar(&t.offset)) return TRUNC;
        GgmlTypeInfo ti;
        if (!ggml_type_info(t.type, &ti)) return t.name + ": unknown ggml type id " + std::to_string(t.type);
        const uint64_t n = t.elements();
        if (n == UINT64_MAX || n > (uint64_t)INT64_MAX) return t.name + ": element count overflows";
        if (n % ti.blk != 0)
            return t.name + ": " + std::to_string(n) + " elements not a multiple of " + ti.name + " block " +
                   std::to_string(ti.blk);
        if (t.bytes() == UINT64_MAX) return t.name + ": byte size overflows";
        g.tensors.push_back(std::move(t));
    }
    g.header_bytes = r.pos;
    uint64_t align = 32;
    if (const GgufValue *a = g.get("general.alignment")) {
        if (!a->as_u64(&align)) align = 32;
    }
    if (align == 0 || (align & (align - 1)) != 0)
        return "general.alignment " + std::to_string(align) + " is not a power of two";
    g.data_offset = (r.pos + align - 1) / align * align;
    return "";
}

std::string gguf_open(const char *path, Gguf &g) {
    g.path = path ? path : "";
    const int fd = path ? open(path, O_RDONLY | O_CLOEXEC) : -1;
    if (fd < 0) return g.path + ": cannot open";
    struct stat sb;
    if (fstat(fd, &sb) != 0 || sb.st_size <= 0) {
        close(fd);
        return g.path + ": cannot stat or empty";
    }
    void *m = mmap(nullptr, (size_t)sb.st_size, PROT_READ, MAP_PRIVATE, fd, 0);
    close(fd);
    if (m == MAP_FAILED) return "mmap " + g.path + " failed";
    g.map = (const uint8_t *)m;
    g.map_len = (size_t)sb.st_size;
    g.file_bytes = (uint64_t)sb.st_size;
    std::string e = gguf_parse(g.map, g.map_len, g);
    if (!e.empty()) return e;
    // every tensor's data inside the file, with checked arithmetic (lib.rs:320-330)
    for (const auto &t : g.tensors) {
        uint64_t end;
        const uint64_t b = t.bytes();
        if (b == UINT64_MAX || __builtin_add_overflow(g.data_offset, t.offset, &end) ||
            __builtin_add_overflow(end, b, &end) || end > g.file_bytes)
            return t.name + ": data beyond end of file";
    }
    return "";
}

std::string gguf_model_desc(const Gguf &g, oxe_model_desc *d) {
    const GgufValue *av = g.get("general.architecture");
    if (!av || av->type != GV_STR) return "no general.architecture";
    const std::string arch = av->s;
    if (arch != "qwen35moe") return "architecture " + arch + " is not supported (qwen35moe only)";
    std::string err;
    auto u = [&](const char *k, uint64_t *out) -> bool {
        const GgufValue *v = g.get(arch + "." + k);
        if (!v || !v->as_u64(out)) {
            if (err.empty()) err = "missing " + arch + "." + k;
            return false;
        }
        return true;
    };
    uint64_t block_count = 0, nextn = 0, interval = 0;
    if (!u("block_count", &block_count) || !u("full_attention_interval", &interval)) return err;
    if (const GgufValue *v = g.get(arch + ".nextn_predict_layers")) v->as_u64(&nextn);
    if (nextn > block_count || interval == 0) return "bad block_count / nextn_predict_layers / full_attention_interval";
    const uint64_t n_layer = block_count - nextn;
    double eps;
    const GgufValue *ev = g.get(arch + ".attention.layer_norm_rms_epsilon");
    if (!ev || !ev->as_f64(&eps)) return "missing rms eps";
    const GgufTensor *out = g.tensor("output.weight");
    if (!out) return "no output.weight";
    if (out->shape.size() < 2) return "output.weight: not a matrix";
    for (uint64_t il = 0; il < n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        const bool rec = g.tensor(p + "ssm_a") != nullptr, att = g.tensor(p + "attn_q.weight") != nullptr;
        if (rec == att)
            return "layer " + std::to_string(il) + ": cannot classify (ssm_a " + (rec ? "true" : "false") + ", attn_q " +
                   (att ? "true" : "false") + ")";
        // llama.cpp qwen35moe: recurrent iff (il + 1) % interval != 0
        const bool expect_rec = (il + 1) % interval != 0;
        if (rec != expect_rec)
            return "layer " + std::to_string(il) + ": tensors say " + (rec ? "Recurrent" : "Attention") +
                   ", full_attention_interval says " + (expect_rec ? "Recurrent" : "Attention");
    }
    uint64_t v[16];
    const char *keys[] = {"embedding_length", "attention.head_count", "attention.head_count_kv", "attention.key_length",
                          "expert_count", "expert_used_count", "expert_feed_forward_length",
                          "expert_shared_feed_forward_length", "ssm.conv_kernel", "ssm.state_size", "ssm.group_count",
                          "ssm.time_step_rank", "ssm.inner_size", "rope.dimension_count", "context_length"};
    for (int i = 0; i < 15; i++)
        if (!u(keys[i], &v[i])) return err;
    double base;
    const GgufValue *bv = g.get(arch + ".rope.freq_base");
    if (!bv || !bv->as_f64(&base)) return "missing rope.freq_base";
    const GgufValue *sv = g.get(arch + ".rope.dimension_sections");
    if (!sv || sv->type != GV_ARR || sv->long_array) return "missing rope.dimension_sections (qwen35moe uses IMRoPE)";
    int32_t sec[4] = {0, 0, 0, 0};
    for (size_t i = 0; i < sv->arr.size() && i < 4; i++) {
        double x;
        if (!sv->arr[i].as_f64(&x)) return "bad rope section";
        sec[i] = (int32_t)x;
    }
    for (int i = 0; i < 15; i++)
        if (v[i] > (uint64_t)INT32_MAX) return std::string("metadata ") + keys[i] + " out of range";
    if (out->shape[1] > (uint64_t)INT32_MAX || n_layer > (uint64_t)INT32_MAX) return "output.weight / layer count out of range";
    oxe_model_desc o{};
    o.n_layer = (int32_t)n_layer;
    o.n_embd = (int32_t)v[0];
    o.n_vocab = (int32_t)out->shape[1];
    o.n_head = (int32_t)v[1];
    o.n_head_kv = (int32_t)v[2];
    o.head_dim = (int32_t)v[3];
    o.n_expert = (int32_t)v[4];
    o.n_expert_used = (int32_t)v[5];
    o.ff_exp = (int32_t)v[6];
    o.ff_shexp = (int32_t)v[7];
    o.ssm_conv_kernel = (int32_t)v[8];
    o.ssm_d_state = (int32_t)v[9];
    o.ssm_n_kheads = (int32_t)v[10];
    o.ssm_n_vheads = (int32_t)v[11];
    o.ssm_d_inner = (int32_t)v[12];
    o.full_attention_interval = (int32_t)interval;
    o.n_rot = (int32_t)v[13];
    for (int i = 0; i < 4; i++) o.rope_sections[i] = sec[i];
    o.rms_eps = (float)eps;
    o.rope_freq_base = (float)base;
    o.n_ctx_train = (int32_t)v[14];
    o.has_mtp = nextn > 0 ? 1 : 0;
    // shape cross-checks (desc.rs:140-178)
    auto shape_is = [&](const std::string &n, std::vector<uint64_t> want, std::string *e) {
        const GgufTensor *t = g.tensor(n);
        if (!t) {
            *e = "missing tensor " + n;
            return false;
        }
        return t->shape == want;
    };
    if (o.ssm_n_vheads == 0 || o.ssm_n_kheads == 0 || o.n_head_kv == 0) return "head counts do not divide";
    const uint64_t e = (uint64_t)o.n_embd;
    const uint64_t conv_ch = (uint64_t)o.ssm_d_inner + 2ull * o.ssm_n_kheads * o.ssm_d_state;
    for (uint64_t il = 0; il < n_layer; il++) {
        const std::string p = "blk." + std::to_string(il) + ".";
        std::string se;
        if ((il + 1) % interval != 0) {
            if (!shape_is(p + "attn_qkv.weight", {e, conv_ch}, &se))
                return se.empty() ? "layer " + std::to_string(il) + ": attn_qkv shape" : se;
            if (!shape_is(p + "ssm_out.weight", {(uint64_t)o.ssm_d_inner, e}, &se))
                return se.empty() ? "layer " + std::to_string(il) + ": ssm_out shape" : se;
        } else if (!shape_is(p + "attn_q.weight", {e, 2ull * o.n_head * o.head_dim}, &se)) {
            return se.empty() ? "layer " + std::to_string(il) + ": attn_q shape (expected q + gate per head)" : se;
        }
        if (!shape_is(p + "ffn_gate_exps.weight", {e, (uint64_t)o.ff_exp, (uint64_t)o.n_expert}, &se))
            return se.empty() ? "layer " + std::to_string(il) + ": ffn_gate_exps shape" : se;
    }
    if (o.ssm_n_vheads % o.ssm_n_kheads != 0 || o.n_head % o.n_head_kv != 0) return "head counts do not divide";
    if (o.ff_exp % 256 != 0 || o.ff_shexp % 256 != 0)
        return "expert FFN width must be a multiple of 256 (one activation block per MoE unit)";
    if (o.ssm_d_state != o.ssm_d_inner / o.ssm_n_vheads)
        return "delta-net head_k_dim != head_v_dim (the fused GDN op requires S_k == S_v)";
    if (o.n_rot > o.head_dim || o.n_rot % 2 != 0) return "bad rope.dimension_count";
    *d = o;
    return "";
}

}  // namespace oxe

// ---- C ABI ---------------------------------------------------------------------------------------

#include "../../include/oxe_amd.h"
#include "oxe_engine_host.h"

using oxe::Gguf;

extern "C" {

int oxe_gguf_open(const char *path, oxe_gguf **out) {
    if (!out) return -1;
    Gguf *g = new Gguf();
    const std::string e = oxe::gguf_open(path, *g);
    if (!e.empty()) {
        oxe::set_err(e);
        delete g;
        return -1;
    }
    *out = (oxe_gguf *)g;
    return 0;
}

int oxe_gguf_parse(const void *buf, uint64_t len, oxe_gguf **out) {
    if (!buf || !out) return -1;
    Gguf *g = new Gguf();
    const std::string e = oxe::gguf_parse((const uint8_t *)buf, (size_t)len, *g);
    if (!e.empty()) {
        oxe::set_err(e);
        delete g;
        return -1;
    }
    g->file_bytes = len;
    *out = (oxe_gguf *)g;
    return 0;
}

int oxe_gguf_check_bounds(const oxe_gguf *gg, uint64_t file_bytes) {
    const Gguf *g = (const Gguf *)gg;
    for (const auto &t : g->tensors) {
        uint64_t end;
        const uint64_t b = t.bytes();
        if (b == UINT64_MAX || __builtin_add_overflow(g->data_offset, t.offset, &end) ||
            __builtin_add_overflow(end, b, &end) || end > file_bytes) {
            oxe::set_err(t.name + ": data beyond end of file");
            return -1;
        }
    }
    return 0;
}

void oxe_gguf_close(oxe_gguf *g) { delete (Gguf *)g; }

int oxe_gguf_info(const oxe_gguf *gg, uint32_t *version, uint64_t *n_tensors, uint64_t *n_meta, uint64_t *data_offset,
                  uint64_t *header_bytes, uint64_t *file_bytes) {
    const Gguf *g = (const Gguf *)gg;
    if (!g) return -1;
    if (version) *version = g->version;
    if (n_tensors) *n_tensors = g->tensors.size();
    if (n_meta) *n_meta = g->meta.size();
    if (data_offset) *data_offset = g->data_offset;
    if (header_bytes) *header_bytes = g->header_bytes;
    if (file_bytes) *file_bytes = g->file_bytes;
    return 0;
}

int oxe_gguf_tensor(const oxe_gguf *gg, uint64_t i, const char **name, uint32_t *type, uint32_t *n_dims,
                    uint64_t *shape4, uint64_t *offset, uint64_t *bytes) {
    const Gguf *g = (const Gguf *)gg;
    if (!g || i >= g->tensors.size()) return -1;
    const auto &t = g->tensors[i];
    if (name) *name = t.name.c_str();
    if (type) *type = t.type;
    if (n_dims) *n_dims = (uint32_t)t.shape.size();
    if (shape4)
        for (int k = 0; k < 4; k++) shape4[k] = k < (int)t.shape.size() ? t.shape[k] : 1;
    if (offset) *offset = t.offset;
    if (bytes) *bytes = t.bytes();
    return 0;
}

int oxe_gguf_meta(const oxe_gguf *gg, uint64_t i, const char **key, uint32_t *type) {
    const Gguf *g = (const Gguf *)gg;
    if (!g || i >= g->meta.size()) return -1;
    if (key) *key = g->meta[i].first.c_str();
    if (type) *type = g->meta[i].second.type;
    return 0;
}

int oxe_gguf_meta_u64(const oxe_gguf *gg, const char *key, uint64_t *out) {
    const Gguf *g = (const Gguf *)gg;
    const oxe::GgufValue *v = g && key ? g->get(key) : nullptr;
    return v && out && v->as_u64(out) ? 0 : -1;
}

int oxe_gguf_meta_f64(const oxe_gguf *gg, const char *key, double *out) {
    const Gguf *g = (const Gguf *)gg;
    const oxe::GgufValue *v = g && key ? g->get(key) : nullptr;
    return v && out && v->as_f64(out) ? 0 : -1;
}

int oxe_gguf_meta_str(const oxe_gguf *gg, const char *key, const char **out) {
    const Gguf *g = (const Gguf *)gg;
    const oxe::GgufValue *v = g && key ? g->get(key) : nullptr;
    if (!v || !out || v->type != oxe::GV_STR) return -1;
    *out = v->s.c_str();
    return 0;
}

int oxe_gguf_meta_array(const oxe_gguf *gg, const char *key, uint32_t *item_type, uint64_t *len, int *kept) {
    const Gguf *g = (const Gguf *)gg;
    const oxe::GgufValue *v = g && key ? g->get(key) : nullptr;
    if (!v || v->type != oxe::GV_ARR) return -1;
    if (item_type) *item_type = v->item_type;
    if (len) *len = v->len;
    if (kept) *kept = v->long_array ? 0 : 1;
    return 0;
}

int oxe_gguf_meta_array_f64(const oxe_gguf *gg, const char *key, uint64_t i, double *out) {
    const Gguf *g = (const Gguf *)gg;
    const oxe::GgufValue *v = g && key ? g->get(key) : nullptr;
    if (!v || v->type != oxe::GV_ARR || v->long_array || i >= v->arr.size() || !out) return -1;
    return v->arr[(size_t)i].as_f64(out) ? 0 : -1;
}

int oxe_gguf_model_desc(const oxe_gguf *gg, oxe_model_desc *out) {
    const Gguf *g = (const Gguf *)gg;
    if (!g || !out) return -1;
    const std::string e = oxe::gguf_model_desc(*g, out);
    if (!e.empty()) {
        oxe::set_err(e);
        return -1;
    }
    return 0;
}

}  // extern "C"
