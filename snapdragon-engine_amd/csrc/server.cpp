// The engine as the reference's server drives it: the `Engine` trait of crates/server/src/engine.rs
// (28-190) as implemented for oxe by the adapter crates/server/src/oxe_engine.rs (317-640). One
// object holds the device engine and, with MTP on, its depth-1 driver:
//   prefill      2+ tokens: batched prefill (+ MTP catch-up seeded in one pass); 1 token: a step
//   decode       one step; the last token's logits / argmax
//   decode_spec  one speculative MTP step: (accepted drafts, argmax of every committed row)
//   spec_rewind  keep a prefix of what the last speculative or lookup step committed
//   decode_verify  caller-supplied drafts (prompt lookup) on the plain engine
//   snapshot / restore  recurrent state + position (+ the MTP driver's catch-up state); KV in place
//   save_state / load_state  Engine::write_state / read_state bytes + the MTP driver's state
// Snapshots are kept in device memory (the state is 63 MB per slot; a device copy is ~20 us).
// With MTP on, OXE_MTP_DRAFT_VOCAB=<ranking> [OXE_MTP_DRAFT_K=<k>] restricts the draft head to the
// ranking file's ids (one per line, most frequent first, cut to k), as the reference's adapter does
// at load (oxe_engine.rs:215-222, MtpWeights::apply_draft_vocab, mtp.rs:199-222).
#include <cstdlib>
#include <fstream>
#include <sstream>

#include "../../include/oxe_amd.h"
#include "oxe_engine_host.h"

namespace oxe {

struct SrvSnapshot {
    int pos = -1;
    float *conv = nullptr, *ssm = nullptr;   // device copies of the current slot
    size_t conv_bytes = 0, ssm_bytes = 0;
    bool has_mtp = false;
    int q = 0;
    std::vector<uint32_t> cu_tok;
    std::vector<float> cu_h, hl;
    ~SrvSnapshot() {
        if (conv) (void)hipFree(conv);
        if (ssm) (void)hipFree(ssm);
    }
};

struct SrvEngine {
    Engine *e = nullptr;
    bool mtp = false;
    int lookup_last = 0;               // tokens committed by the last lookup verify (0: none)
    uint64_t lookup_drafted = 0, lookup_accepted = 0;
    // the engine is borrowed: the caller destroys this object before the engine

    int fail(int rc, const std::string &msg) {
        set_err(msg);
        return rc;
    }
    int check_tokens(const uint32_t *t, int n) {
        if (n < 1) return fail(-1, "empty prefill");
        if (e->pos + n > e->m.n_ctx) return fail(-1, "context full");
        for (int i = 0; i < n; i++)
            if (t[i] >= (uint32_t)e->d.n_vocab) return fail(-1, "token " + std::to_string(t[i]) + " out of vocab");
        return 0;
    }
    // one decode token: vocab, then room (decode_argmax / decode_spec, oxe_engine.rs:544-552)
    int check_one(uint32_t t) {
        if (t >= (uint32_t)e->d.n_vocab) return fail(-1, "token " + std::to_string(t) + " out of vocab");
        if (e->pos + 1 > e->m.n_ctx) return fail(-1, "context full");
        return 0;
    }
    int logits_row(float *out) {
        if (!out) return 0;
        if (hipMemcpy(out, e->b.logits, (size_t)e->d.n_vocab * 4, hipMemcpyDeviceToHost) != hipSuccess) return -2;
        return 0;
    }

    // MtpDriver::sync (mtp.rs:363-382): after the engine's position moved under the driver
    void mtp_sync(const float *h_prev) {
        MtpDriverHost &d = e->drv;
        const int p = e->pos;
        if (p < d.q) d.q = p;
        const size_t keep = std::min<size_t>((size_t)std::max(0, p - d.q), d.cu_tok.size());
        d.cu_tok.resize(keep);
        d.cu_h.resize(keep * E);
        if (d.q + (int)d.cu_tok.size() < p) {   // positions the driver did not see: MTP KV stale there
            d.q = p;
            d.cu_tok.clear();
            d.cu_h.clear();
        }
        if (h_prev) d.hl.assign(h_prev, h_prev + E);
        else std::fill(d.hl.begin(), d.hl.end(), 0.0f);
        d.last_n = 0;
    }

    // Engine::reset (engine.rs:1491-1509): empty sequence, zero recurrent state, V^T back to +0
    int reset() {
        lookup_last = 0;
        const size_t conv = (size_t)OXE_NSLOTS * conv_bytes(), ssm = (size_t)OXE_NSLOTS * ssm_bytes();
        if (hipMemsetAsync(e->m.conv_state, 0, conv, e->st) != hipSuccess ||
            hipMemsetAsync(e->m.ssm_state, 0, ssm, e->st) != hipSuccess ||
            hipMemsetAsync(e->m.vcache, 0, (size_t)e->m.n_att * NKV * HD * e->m.n_ctx * 2, e->st) != hipSuccess)
            return -2;
        e->pos = 0;
        e->cur = 0;
        e->pend_n = 0;
        if (mtp) mtp_sync(nullptr);
        return hipStreamSynchronize(e->st) == hipSuccess ? 0 : -2;
    }

    int prefill(const uint32_t *t, int n, float *logits) {
        lookup_last = 0;
        int rc = check_tokens(t, n);
        if (rc) return rc;
        uint32_t next = 0;
        if (mtp) rc = n == 1 ? e->drv.step_plain(*e, t[0], &next) : e->drv.prefill_batched(*e, t, n, &next);
        else if (n == 1) {
            rc = e->verify(t, 1, &next);
            if (!rc) rc = e->commit(1);
        } else {
            rc = e->prefill(t, n, &next, nullptr);
        }
        if (rc) return rc;
        return logits_row(logits);
    }

    int decode_argmax(uint32_t tok, uint32_t *out) {
        lookup_last = 0;
        int rc = check_one(tok);
        if (rc) return rc;
        uint32_t g = 0;
        if (mtp) rc = e->drv.step_plain(*e, tok, &g);
        else {
            rc = e->verify(&tok, 1, &g);
            if (!rc) rc = e->commit(1);
        }
        if (!rc && out) *out = g;
        return rc;
    }

    // decode_spec_argmax: `extra` = accepted drafts (now in the state), `argmax` = the argmax of
    // every committed row (the last one is the bonus token, not yet in the state); rows (optional):
    // those rows' logits (decode_spec)
    int decode_spec_argmax(uint32_t tok, uint32_t *extra, int *n_extra, uint32_t *argmax, int *n_argmax,
                           float *rows = nullptr) {
        if (!mtp) return 1;   // unsupported: the caller decodes one token
        int rc = check_one(tok);
        if (rc) return rc;
        uint32_t out[MTP_MAX_DEPTH + 1];
        int n = 0;
        if ((rc = e->drv.step_k(*e, tok, out, &n, nullptr, 0, rows))) return rc;
        for (int i = 0; i < n; i++) argmax[i] = out[i];
        for (int i = 0; i + 1 < n; i++) extra[i] = out[i];
        *n_argmax = n;
        *n_extra = n - 1;
        return 0;
    }

    int spec_rewind(int keep) {
        if (lookup_last) {
            const int n = lookup_last;
            lookup_last = 0;
            if (keep < 1) return fail(-1, "spec_rewind: keep out of range");
            return keep < n ? e->commit(keep) : 0;   // commit again with a smaller count
        }
        if (!mtp) return 0;
        if (e->drv.last_n == 0) return fail(-1, "rewind without a step");
        if (keep < 1 || keep > e->drv.last_n) return fail(-1, "spec_rewind: keep out of range");
        return keep == e->drv.last_n ? 0 : e->drv.rewind(*e, keep);
    }

    // prompt-lookup drafts on the plain engine: verify [tok, drafts[0..k)], accept the prefix that
    // equals greedy decoding, commit it (oxe_engine.rs:593-619); k <= verify lanes - 1
    int decode_verify(uint32_t tok, const uint32_t *drafts, int nd, uint32_t *acc, int *n_acc, uint32_t *argmax,
                      int *n_argmax) {
        if (mtp || nd < 1) return 1;
        if (tok >= (uint32_t)e->d.n_vocab) return fail(-1, "token out of vocab");
        for (int i = 0; i < nd; i++)
            if (drafts[i] >= (uint32_t)e->d.n_vocab) return fail(-1, "token out of vocab");
        const int k = std::min(std::min(nd, OXE_NL - 1), std::max(0, e->m.n_ctx - (e->pos + 1)));
        if (k == 0) return 1;
        uint32_t vt[OXE_NL], g[OXE_NL];
        vt[0] = tok;
        for (int i = 0; i < k; i++) vt[1 + i] = drafts[i];
        int rc = e->verify(vt, k + 1, g);
        if (rc) return rc;
        int a = 0;
        while (a < k && drafts[a] == g[a]) a++;
        if ((rc = e->commit(a + 1))) return rc;
        lookup_last = a + 1;
        lookup_drafted += k;
        lookup_accepted += a;
        for (int i = 0; i < a; i++) acc[i] = drafts[i];
        for (int i = 0; i <= a; i++) argmax[i] = g[i];
        *n_acc = a;
        *n_argmax = a + 1;
        return 0;
    }

    int snapshot(SrvSnapshot *s) {
        const size_t conv = conv_bytes(), ssm = ssm_bytes();
        if (!s->conv) {
            if (hipMalloc(&s->conv, conv) != hipSuccess || hipMalloc(&s->ssm, ssm) != hipSuccess)
                return fail(-3, "out of device memory for a snapshot");
            s->conv_bytes = conv;
            s->ssm_bytes = ssm;
        } else if (s->conv_bytes != conv || s->ssm_bytes != ssm) {
            return fail(-1, "snapshot from another model");
        }
        if (hipMemcpyAsync(s->conv, (const char *)e->m.conv_state + e->cur * conv, conv, hipMemcpyDeviceToDevice, e->st) !=
                hipSuccess ||
            hipMemcpyAsync(s->ssm, (const char *)e->m.ssm_state + e->cur * ssm, ssm, hipMemcpyDeviceToDevice, e->st) !=
                hipSuccess)
            return -2;
        s->pos = e->pos;
        s->has_mtp = mtp;
        if (mtp) {
            s->q = e->drv.q;
            s->cu_tok = e->drv.cu_tok;
            s->cu_h = e->drv.cu_h;
            s->hl = e->drv.hl;
        }
        return hipStreamSynchronize(e->st) == hipSuccess ? 0 : -2;
    }

    size_t conv_bytes() const { return (size_t)e->m.n_rec * NCH * (KC - 1) * 4; }
    size_t ssm_bytes() const { return (size_t)e->m.n_rec * NVH * HV * HV * 4; }

    // Engine::restore_recurrent (engine.rs:1643-1659): the current slot's conv and S from `conv` /
    // `ssm` (device or host memory, by `kind`), V^T of the main attention layers at positions
    // [pos, current) back to +0, the position becomes pos
    int restore_rec(int pos, const void *conv, const void *ssm, hipMemcpyKind kind) {
        lookup_last = 0;
        if (hipMemcpyAsync((char *)e->m.conv_state + e->cur * conv_bytes(), conv, conv_bytes(), kind, e->st) !=
                hipSuccess ||
            hipMemcpyAsync((char *)e->m.ssm_state + e->cur * ssm_bytes(), ssm, ssm_bytes(), kind, e->st) != hipSuccess)
            return -2;
        if (e->pos > pos) launch_zero_v(e->m, e->n_att_main, pos, e->pos, e->st);
        e->pos = pos;
        e->pend_n = 0;
        return hipStreamSynchronize(e->st) == hipSuccess ? 0 : -2;
    }
    // OxeEngine::restore_mtp (oxe_engine.rs:304-311): the snapshot's exact driver state when it
    // fits the engine (MtpDriver::import_state, mtp.rs:391-401), else a re-sync from its h_prev
    void restore_mtp(bool has, int q, const std::vector<uint32_t> &cu_tok, const std::vector<float> &cu_h,
                     const std::vector<float> &hl) {
        if (!mtp) return;
        MtpDriverHost &d = e->drv;
        if (has && cu_h.size() == cu_tok.size() * E && hl.size() == (size_t)E && q + (int)cu_tok.size() == e->pos) {
            d.q = q;
            d.cu_tok = cu_tok;
            d.cu_h = cu_h;
            d.hl = hl;
            d.last_n = 0;
        } else {
            mtp_sync(has && hl.size() == (size_t)E ? hl.data() : nullptr);
        }
    }
    int restore(const SrvSnapshot *s) {
        if (s->pos < 0 || s->conv_bytes != conv_bytes() || s->ssm_bytes != ssm_bytes())
            return fail(-1, "snapshot from another model");
        if (s->pos > e->pos) return fail(-1, "restore of a snapshot ahead of the current position");
        const int rc = restore_rec(s->pos, s->conv, s->ssm, hipMemcpyDeviceToDevice);
        if (rc) return rc;
        restore_mtp(s->has_mtp, s->q, s->cu_tok, s->cu_h, s->hl);
        return 0;
    }

    // Snapshot file (OxeEngine::snap_save / snap_save_live, oxe_engine.rs:428-450):
    // RecurrentSnapshot::write_to (engine.rs:572-582: u64 pos, u64 conv length, u64 ssm length,
    // conv f32, ssm f32), a tag byte (0: no MTP state, 2: MTP driver state) and with tag 2
    // MtpState::write (oxe_engine.rs:108-119: u64 q, u64 n, n u32 tokens, n rows of n_embd f32,
    // h_prev), little-endian
    static int64_t snap_file_bytes(size_t conv_b, size_t ssm_b, bool has_mtp, size_t n) {
        return 24 + (int64_t)(conv_b + ssm_b) + 1 + (has_mtp ? 16 + (int64_t)n * 4 + ((int64_t)n + 1) * E * 4 : 0);
    }
    int snap_write(int pos, const void *conv, const void *ssm, bool has_mtp, int q, const std::vector<uint32_t> &cu_tok,
                   const std::vector<float> &cu_h, const std::vector<float> &hl, void *buf, int64_t cap,
                   int64_t *written) {
        const int64_t need = snap_file_bytes(conv_bytes(), ssm_bytes(), has_mtp, cu_tok.size());
        if (!buf || cap < need) return fail(-1, "save snapshot: buffer smaller than the snapshot");
        char *o = (char *)buf;
        const uint64_t hdr[3] = {(uint64_t)pos, conv_bytes() / 4, ssm_bytes() / 4};
        std::memcpy(o, hdr, 24);
        o += 24;
        if (hipMemcpyAsync(o, conv, conv_bytes(), hipMemcpyDeviceToHost, e->st) != hipSuccess) return -2;
        o += conv_bytes();
        if (hipMemcpyAsync(o, ssm, ssm_bytes(), hipMemcpyDeviceToHost, e->st) != hipSuccess) return -2;
        o += ssm_bytes();
        *o++ = has_mtp ? 2 : 0;
        if (has_mtp) {
            const uint64_t qn[2] = {(uint64_t)q, (uint64_t)cu_tok.size()};
            std::memcpy(o, qn, 16);
            o += 16;
            std::memcpy(o, cu_tok.data(), cu_tok.size() * 4);
            o += cu_tok.size() * 4;
            std::memcpy(o, cu_h.data(), cu_h.size() * 4);
            o += cu_h.size() * 4;
            std::memcpy(o, hl.data(), (size_t)E * 4);
        }
        if (hipStreamSynchronize(e->st) != hipSuccess) return -2;
        if (written) *written = need;
        return 0;
    }
    int snap_save(const SrvSnapshot *s, void *buf, int64_t cap, int64_t *written) {
        if (s->conv_bytes != conv_bytes() || s->ssm_bytes != ssm_bytes()) return fail(-1, "snapshot from another model");
        return snap_write(s->pos, s->conv, s->ssm, s->has_mtp, s->q, s->cu_tok, s->cu_h, s->hl, buf, cap, written);
    }
    int64_t snap_live_bytes() const {
        return snap_file_bytes(conv_bytes(), ssm_bytes(), mtp, mtp ? e->drv.cu_tok.size() : 0);
    }
    int snap_save_live(void *buf, int64_t cap, int64_t *written) {
        static const std::vector<uint32_t> no_tok;
        static const std::vector<float> no_f;
        const MtpDriverHost &d = e->drv;
        return snap_write(e->pos, (const char *)e->m.conv_state + e->cur * conv_bytes(),
                          (const char *)e->m.ssm_state + e->cur * ssm_bytes(), mtp, d.q, mtp ? d.cu_tok : no_tok,
                          mtp ? d.cu_h : no_f, d.hl, buf, cap, written);
    }
    // OxeEngine::snap_load (oxe_engine.rs:451-467) with RecurrentSnapshot::read_from (engine.rs:585-602)
    // and MtpState::read (oxe_engine.rs:120-137): the KV rows of positions < n_pos are already in
    // place (kv rows load); the whole file is checked before any state changes
    int snap_load(const void *buf, int64_t nbytes, int n_pos) {
        const char *in = (const char *)buf;
        if (!buf || nbytes < 25 || n_pos < 0 || n_pos > e->m.n_ctx) return fail(-1, "load snapshot: truncated");
        uint64_t hdr[3];
        std::memcpy(hdr, in, 24);
        if (hdr[1] != conv_bytes() / 4 || hdr[2] != ssm_bytes() / 4)
            return fail(-1, "load snapshot: snapshot of another recurrent layout");
        if (nbytes < (int64_t)(24 + conv_bytes() + ssm_bytes() + 1)) return fail(-1, "load snapshot: truncated");
        if (hdr[0] != (uint64_t)n_pos) return fail(-1, "load snapshot: position does not match its rows");
        const char *conv = in + 24, *ssm = conv + conv_bytes(), *t = ssm + ssm_bytes();
        const uint8_t tag = (uint8_t)*t++;
        if (!((tag == 0 && !mtp) || (tag == 2 && mtp))) return fail(-1, "load snapshot: MTP state does not match this engine");
        uint64_t q = 0, n = 0;
        if (tag == 2) {
            if (nbytes < (int64_t)(t - in) + 16) return fail(-1, "load snapshot: truncated");
            std::memcpy(&q, t, 8);
            std::memcpy(&n, t + 8, 8);
            // each term bounded first, so the sum cannot wrap (as load_state checks it)
            if (n > 4096 || n > (uint64_t)n_pos || q > (uint64_t)n_pos || q + n != (uint64_t)n_pos)
                return fail(-1, "load snapshot: MTP state does not match the snapshot position");
            t += 16;
        }
        if (nbytes != snap_file_bytes(conv_bytes(), ssm_bytes(), tag == 2, n)) return fail(-1, "load snapshot: size does not match");
        int rc = restore_rec(n_pos, conv, ssm, hipMemcpyHostToDevice);
        if (rc) return rc;
        if (tag == 2) {
            std::vector<uint32_t> ct((const uint32_t *)t, (const uint32_t *)t + n);
            t += n * 4;
            std::vector<float> ch((const float *)t, (const float *)t + n * E);
            t += n * E * 4;
            std::vector<float> hl((const float *)t, (const float *)t + E);
            restore_mtp(true, (int)q, ct, ch, hl);
        }
        return 0;
    }
    // Engine::state_layout (engine.rs:1669-1677), the f16 KV form: a state written by one engine
    // is read by another whose layout string is equal
    std::string state_layout() const {
        return "att=" + std::to_string(e->m.n_att) + " kv_heads=" + std::to_string(NKV) + " head_dim=" +
               std::to_string(HD) + " conv=" + std::to_string(conv_bytes() / 4) + " ssm=" + std::to_string(ssm_bytes() / 4) +
               " f16kv";
    }

    int64_t state_size_hint() const {
        return oxe_engine_state_bytes((const oxe_engine *)e) + (mtp ? (int64_t)e->pos * 4 * E : 0);
    }
    // save_state (oxe_engine.rs:492-507): write_state, then with MTP on: u64 q, u64 n, n u32
    // pending tokens, their n h rows and h_prev (f32, little-endian)
    int64_t save_bytes() const {
        int64_t b = oxe_engine_state_bytes((const oxe_engine *)e);
        if (mtp) b += 16 + (int64_t)e->drv.cu_tok.size() * 4 + ((int64_t)e->drv.cu_tok.size() + 1) * E * 4;
        return b;
    }
    int save_state(void *buf, int64_t cap, int64_t *written) {
        const int64_t need = save_bytes();
        if (!buf || cap < need) return fail(-1, "save_state: buffer smaller than the state");
        const int64_t sb = oxe_engine_state_bytes((const oxe_engine *)e);
        int rc = oxe_engine_write_state((oxe_engine *)e, buf, sb);
        if (rc) return rc;
        char *o = (char *)buf + sb;
        if (mtp) {
            const MtpDriverHost &d = e->drv;
            const uint64_t q = (uint64_t)d.q, n = d.cu_tok.size();
            std::memcpy(o, &q, 8);
            std::memcpy(o + 8, &n, 8);
            o += 16;
            std::memcpy(o, d.cu_tok.data(), n * 4);
            o += n * 4;
            std::memcpy(o, d.cu_h.data(), n * E * 4);
            o += n * E * 4;
            std::memcpy(o, d.hl.data(), E * 4);
        }
        if (written) *written = need;
        return 0;
    }
    int load_state(const void *buf, int64_t nbytes, int n_pos) {
        lookup_last = 0;
        if (!buf || n_pos < 0 || n_pos > e->m.n_ctx) return fail(-1, "load_state: bad arguments");
        const int64_t sb = oxe_engine_kv_row_bytes((const oxe_engine *)e) * n_pos + (int64_t)(conv_bytes() + ssm_bytes());
        if (nbytes < sb) return fail(-1, "load_state: truncated state");
        const char *in = (const char *)buf;
        uint64_t q = 0, n = 0;
        if (mtp) {
            if (nbytes < sb + 16) return fail(-1, "load state: bad MTP header");
            std::memcpy(&q, in + sb, 8);
            std::memcpy(&n, in + sb + 8, 8);
            if (n > (uint64_t)n_pos || q + n != (uint64_t)n_pos ||
                nbytes != sb + 16 + (int64_t)n * 4 + ((int64_t)n + 1) * E * 4)
                return fail(-1, "load state: bad MTP header");
        } else if (nbytes != sb) {
            return fail(-1, "load_state: size does not match the state");
        }
        int rc = oxe_engine_read_state((oxe_engine *)e, buf, sb, n_pos);
        if (rc) return rc;
        if (mtp) {
            MtpDriverHost &d = e->drv;
            const char *p = in + sb + 16;
            d.q = (int)q;
            d.cu_tok.assign((const uint32_t *)p, (const uint32_t *)p + n);
            p += n * 4;
            d.cu_h.assign((const float *)p, (const float *)p + n * E);
            p += n * E * 4;
            d.hl.assign((const float *)p, (const float *)p + E);
            d.last_n = 0;
        }
        return 0;
    }
};

}  // namespace oxe

using oxe::SrvEngine;
using oxe::SrvSnapshot;

// every call starts with no error message, so a failure reports its own
static SrvEngine *srv(oxe_srv *s) {
    oxe::set_err("");
    return (SrvEngine *)s;
}

extern "C" {

// the ranking file's ids: the first field of each line that parses as an unsigned integer, in file
// order, the first k of them when k >= 0 (apply_draft_vocab, mtp.rs:199-212)
static int read_ranking(const char *path, long long k, std::vector<uint32_t> &ids) {
    std::ifstream f(path);
    if (!f) {
        oxe::set_err(std::string(path) + ": cannot be read");
        return -1;
    }
    std::string line;
    while (std::getline(f, line)) {
        std::istringstream ls(line);
        std::string w;
        if (!(ls >> w) || w.empty() || w.size() > 10 || w.find_first_not_of("0123456789") != std::string::npos) continue;
        const unsigned long long v = std::stoull(w);
        if (v > 0xffffffffull) continue;
        ids.push_back((uint32_t)v);
    }
    if (k >= 0 && (long long)ids.size() > k) ids.resize((size_t)k);
    return 0;
}

int oxe_srv_create(oxe_engine *engine, int mtp, oxe_srv **out) {
    if (!engine || !out) return -1;
    oxe::Engine *e = (oxe::Engine *)engine;
    if (mtp) {
        if (const char *rk = std::getenv("OXE_MTP_DRAFT_VOCAB")) {
            long long k = -1;
            if (const char *ks = std::getenv("OXE_MTP_DRAFT_K")) {
                char *end = nullptr;
                const long long v = std::strtoll(ks, &end, 10);
                if (end && *end == 0 && v >= 0) k = v;   // unparsable: no cut, as the reference's .ok()
            }
            std::vector<uint32_t> ids;
            if (read_ranking(rk, k, ids)) return -1;
            if (ids.empty()) {
                oxe::set_err("empty draft vocabulary");
                return -1;
            }
            const int rows = e->set_draft_vocab(ids.data(), (int)ids.size());
            if (rows < 0) {
                if (rows == -1) oxe::set_err("empty draft vocabulary");
                return rows;
            }
            if (rows > 0) fprintf(stderr, "oxe-server: MTP draft head restricted to %d rows\n", rows);
        }
    }
    SrvEngine *s = new SrvEngine();
    s->e = e;
    s->mtp = mtp != 0;
    if (s->mtp) s->mtp_sync(nullptr);
    *out = (oxe_srv *)s;
    return 0;
}
void oxe_srv_destroy(oxe_srv *s) { delete (SrvEngine *)s; }
oxe_engine *oxe_srv_engine(oxe_srv *s) { return (oxe_engine *)srv(s)->e; }
int oxe_srv_n_ctx(const oxe_srv *s) { return ((const SrvEngine *)s)->e->m.n_ctx; }
int oxe_srv_n_vocab(const oxe_srv *s) { return ((const SrvEngine *)s)->e->d.n_vocab; }
int oxe_srv_n_past(const oxe_srv *s) { return ((const SrvEngine *)s)->e->pos; }
int oxe_srv_reset(oxe_srv *s) { return srv(s)->reset(); }
int oxe_srv_prefill(oxe_srv *s, const uint32_t *toks, int n, float *logits) {
    return srv(s)->prefill(toks, n, logits);
}
int oxe_srv_decode(oxe_srv *s, uint32_t tok, float *logits) { return srv(s)->prefill(&tok, 1, logits); }
int oxe_srv_decode_argmax(oxe_srv *s, uint32_t tok, uint32_t *out) { return srv(s)->decode_argmax(tok, out); }
int oxe_srv_decode_spec_argmax(oxe_srv *s, uint32_t tok, uint32_t *extra, int *n_extra, uint32_t *argmax, int *n_argmax) {
    if (!extra || !n_extra || !argmax || !n_argmax) return -1;
    return srv(s)->decode_spec_argmax(tok, extra, n_extra, argmax, n_argmax);
}
int oxe_srv_decode_spec(oxe_srv *s, uint32_t tok, uint32_t *extra, int *n_extra, float *rows, int rows_cap) {
    if (!extra || !n_extra || !rows) return -1;
    // a step commits up to depth + 1 rows: refuse a buffer that could not hold them, before any work
    const SrvEngine *v = srv(s);
    if (v->mtp && rows_cap < v->e->drv.depth + 1) {
        oxe::set_err("decode_spec: rows buffer holds " + std::to_string(rows_cap) + " rows, a depth-" +
                  std::to_string(v->e->drv.depth) + " step needs " + std::to_string(v->e->drv.depth + 1));
        return -1;
    }
    uint32_t g[oxe::MTP_MAX_DEPTH + 1];
    int ng = 0;
    return srv(s)->decode_spec_argmax(tok, extra, n_extra, g, &ng, rows);
}
int oxe_srv_spec_rewind(oxe_srv *s, int keep) { return srv(s)->spec_rewind(keep); }
int oxe_srv_decode_verify(oxe_srv *s, uint32_t tok, const uint32_t *drafts, int n_drafts, uint32_t *accepted, int *n_acc,
                          uint32_t *argmax, int *n_argmax) {
    if (!drafts || !accepted || !n_acc || !argmax || !n_argmax) return -1;
    return srv(s)->decode_verify(tok, drafts, n_drafts, accepted, n_acc, argmax, n_argmax);
}
int oxe_srv_spec_max_depth(const oxe_srv *s) { return ((const SrvEngine *)s)->mtp ? oxe::MTP_MAX_DEPTH : 0; }
// spec_set_depth (oxe_engine.rs:623-627): clamped to 1..max; no effect without MTP
int oxe_srv_spec_set_depth(oxe_srv *s, int depth) {
    SrvEngine *v = srv(s);
    if (v->mtp) v->e->drv.depth = depth < 1 ? 1 : (depth > oxe::MTP_MAX_DEPTH ? oxe::MTP_MAX_DEPTH : depth);
    return 0;
}
int oxe_srv_spec_counters(const oxe_srv *s, uint64_t *drafted, uint64_t *accepted) {
    const SrvEngine *v = (const SrvEngine *)s;
    if (!drafted || !accepted) return -1;
    if (v->mtp) {
        *drafted = (uint64_t)v->e->drv.drafted;
        *accepted = (uint64_t)v->e->drv.accepted;
    } else {
        *drafted = v->lookup_drafted;
        *accepted = v->lookup_accepted;
    }
    return 0;
}
int oxe_srv_snapshot(oxe_srv *s, oxe_snapshot **inout) {
    if (!inout) return -1;
    SrvSnapshot *sn = *inout ? (SrvSnapshot *)*inout : new SrvSnapshot();
    const int rc = srv(s)->snapshot(sn);
    if (rc) {
        if (!*inout) delete sn;
        return rc;
    }
    *inout = (oxe_snapshot *)sn;
    return 0;
}
int oxe_srv_restore(oxe_srv *s, const oxe_snapshot *sn) {
    if (!sn) return -1;
    return srv(s)->restore((const SrvSnapshot *)sn);
}
int64_t oxe_snapshot_bytes(const oxe_snapshot *sn) {
    const SrvSnapshot *v = (const SrvSnapshot *)sn;
    return (int64_t)(v->conv_bytes + v->ssm_bytes + 4 * (v->cu_tok.size() + v->cu_h.size() + v->hl.size()) + 8);
}
int oxe_snapshot_pos(const oxe_snapshot *sn) { return ((const SrvSnapshot *)sn)->pos; }
void oxe_snapshot_free(oxe_snapshot *sn) { delete (SrvSnapshot *)sn; }
int64_t oxe_srv_state_size_hint(const oxe_srv *s) { return ((const SrvEngine *)s)->state_size_hint(); }
int64_t oxe_srv_save_bytes(const oxe_srv *s) { return ((const SrvEngine *)s)->save_bytes(); }
int oxe_srv_save_state(oxe_srv *s, void *buf, int64_t cap, int64_t *written) {
    return srv(s)->save_state(buf, cap, written);
}
int oxe_srv_load_state(oxe_srv *s, const void *buf, int64_t nbytes, int n_pos) {
    return srv(s)->load_state(buf, nbytes, n_pos);
}
int64_t oxe_srv_snap_file_bytes(const oxe_srv *s, const oxe_snapshot *sn) {
    const SrvSnapshot *v = (const SrvSnapshot *)sn;
    (void)s;
    return SrvEngine::snap_file_bytes(v->conv_bytes, v->ssm_bytes, v->has_mtp, v->cu_tok.size());
}
int oxe_srv_snap_save(oxe_srv *s, const oxe_snapshot *sn, void *buf, int64_t cap, int64_t *written) {
    if (!sn) return -1;
    return srv(s)->snap_save((const SrvSnapshot *)sn, buf, cap, written);
}
int64_t oxe_srv_snap_live_bytes(const oxe_srv *s) { return ((const SrvEngine *)s)->snap_live_bytes(); }
int oxe_srv_snap_save_live(oxe_srv *s, void *buf, int64_t cap, int64_t *written) {
    return srv(s)->snap_save_live(buf, cap, written);
}
int oxe_srv_snap_load(oxe_srv *s, const void *buf, int64_t nbytes, int n_pos) {
    return srv(s)->snap_load(buf, nbytes, n_pos);
}
int oxe_srv_state_layout(const oxe_srv *s, char *buf, int cap) {
    const std::string l = ((const SrvEngine *)s)->state_layout();
    if (!buf || cap < (int)l.size() + 1) return (int)l.size() + 1;
    std::memcpy(buf, l.c_str(), l.size() + 1);
    return 0;
}

}  // extern "C"
