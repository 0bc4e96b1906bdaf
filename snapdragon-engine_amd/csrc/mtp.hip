// MTP speculative decoding (crates/model/src/mtp.rs:314-608, MtpDriver):
//  * a host-driven driver with the reference's semantics (catch-up pairs, draft chain, verify,
//    greedy accept, commit, rewind) over the engine's host-driven calls, depth 1..3, and
//  * the device-driven step at depth 1 or 2: the same state machine held in device memory
//    (MtpState), one step = draft(s) (depth 1: with the pending pair as an extra lane; depth 2: after
//    a seeding run) -> verify -> accept/commit, all decided on the GPU and captured once as a HIP
//    graph; K steps are K graph launches with no host round-trip.
#include <hip/hip_runtime.h>

#include <cstring>
#include <vector>

#include "../../include/oxe_amd.h"
#include "oxe_engine.h"
#include "oxe_engine_host.h"
#include "oxe_model_kernels.h"
#include "oxe_mtp_dev.h"
#include "oxe_shape.h"

namespace oxe {

using namespace shp;


// ---- device-driven step kernels ----------------------------------------------------------------

// per-phase runs: the draft run reads ctl
__global__ void mtp_prep_draft_kernel(MtpState *ms, RunCtl *ctl, int n_ctx) { *ctl = draft_ctl(ms, n_ctx); }
// fused runs: the first step's draft control block (the commit kernel fills it for the next)
__global__ void mtp_prep_step_kernel(MtpState *ms, RunCtl *cd, int n_ctx) { *cd = draft_ctl(ms, n_ctx); }

// the largest of n argmax keys (one wave: lanes stride the keys, then a shuffle tree)
__device__ unsigned long long wave_key_max(const unsigned long long *keys, int n) {
    unsigned long long k = 0ull;
    for (int i = threadIdx.x & 63; i < n; i += 64) k = keys[i] > k ? keys[i] : k;
    for (int m = 32; m >= 1; m >>= 1) {
        const unsigned long long o = __shfl_xor(k, m, 64);
        k = o > k ? o : k;
    }
    return k;
}

// per-phase runs: the verify's control block from the draft's argmax (the fused draft run does this
// in its last stage)
__global__ void mtp_prep_verify_kernel(MtpState *ms, RunCtl *ctl, const unsigned long long *keys, int nkeys,
                                       const int32_t *force_d1, int force_n, int n_ctx) {
    const unsigned long long k0 = wave_key_max(keys + (ms->pending != 0 ? nkeys : 0), nkeys);  // the draft's lane
    if (threadIdx.x == 0) *ctl = mtp_after_draft(ms, k0, force_d1, force_n, n_ctx);
}

// per-phase runs: accept / commit after the verify (the fused verify run does this in its last
// stage), then the next step's draft control block (cd)
__global__ void mtp_commit_kernel(MtpState *ms, const unsigned long long *keys, int nkeys, float *hid, int n_ctx,
                                  uint32_t *out_tok, int out_cap, RunCtl *cd) {
    __shared__ CommitSm sm;
    __shared__ uint32_t s_g[2];
    const int t = threadIdx.x;
    if (t < 64) {
        const unsigned long long k0 = wave_key_max(keys, nkeys), k1 = wave_key_max(keys + nkeys, nkeys);
        if (t == 0) {
            s_g[0] = decode_key(k0);
            s_g[1] = decode_key(k1);
        }
    }
    __syncthreads();
    mtp_commit(ms, true, s_g[0], s_g[1], hid, n_ctx, out_tok, out_cap, cd, sm);
}

// ---- the device-driven step at depth 2 (mtp.rs:522-592 with k = 2) --------------------------------
// seed (the pending pairs, up to 2) -> draft 1 (x, hl) at p -> draft 2 (d1, draft 1's MTP h) at p + 1
// -> verify piece 1 (x, d1) at p, p + 1 -> commit 1 -> verify piece 2 (d2 at p + 2; active when d1
// was accepted and d2 equals piece 1's second argmax) -> commit 2. The reference's 3-lane verify runs
// as these two pieces (the kernels' lane count), committed one after the other and stopped at the
// first rejected draft, as the host driver's step_k does. Every run reads ctl, written just before it.

// draft i of the current step, or the test hook's forced value (force[steps * 2 + i] >= 0)
__device__ uint32_t forced2(const MtpState *ms, const int32_t *force, int force_n, int i, uint32_t d) {
    const int j = ms->steps * 2 + i;
    return (force && j < force_n && force[j] >= 0) ? (uint32_t)force[j] : d;
}

__global__ void mtp2_prep_seed_kernel(MtpState *ms, RunCtl *ctl) {
    const int np = ms->pending;
    RunCtl r{};
    r.nl = np > 1 ? 2 : 1;
    r.pos0 = ms->pos - np;
    r.cur = ms->cur;
    r.tok[0] = ms->pend_tok;
    r.tok[1] = ms->pend_tok2;
    r.hin_sel[0] = HID_PEND;
    r.hin_sel[1] = HID_PEND2;
    r.head_mask = 0;
    r.active = np > 0 && ms->err == 0;
    *ctl = r;
}

__global__ void mtp2_prep_draft1_kernel(MtpState *ms, RunCtl *ctl, int n_ctx) {
    if (ms->pos + 3 > n_ctx) ms->err |= 2;  // no room for the 3 positions of a depth-2 step: stop
    RunCtl r{};
    r.nl = 1;
    r.pos0 = ms->pos;
    r.cur = ms->cur;
    r.tok[0] = ms->x;
    r.hin_sel[0] = HID_HL;
    r.head_mask = 1;
    r.active = ms->err == 0;
    *ctl = r;
}

// d1 from draft 1's argmax; draft 1's MTP h (hid[0]) kept in HID_M as draft 2's input
__global__ void mtp2_prep_draft2_kernel(MtpState *ms, RunCtl *ctl, const unsigned long long *keys, int nkeys, float *hid,
                                        const int32_t *force, int force_n) {
    const int t = threadIdx.x;
    if (t < 64) {
        const unsigned long long k0 = wave_key_max(keys, nkeys);
        if (t == 0) {
            const uint32_t d1 = forced2(ms, force, force_n, 0, decode_key(k0));
            ms->d1 = d1;
            RunCtl r{};
            r.nl = 1;
            r.pos0 = ms->pos + 1;
            r.cur = ms->cur;
            r.tok[0] = d1;
            r.hin_sel[0] = HID_M;
            r.head_mask = 1;
            r.active = ms->err == 0;
            *ctl = r;
        }
    }
    for (int i = t; i < E; i += blockDim.x) hid[(int64_t)HID_M * E + i] = hid[i];
}

__global__ void mtp2_prep_verify1_kernel(MtpState *ms, RunCtl *ctl, const unsigned long long *keys, int nkeys,
                                         const int32_t *force, int force_n) {
    const unsigned long long k0 = wave_key_max(keys, nkeys);
    if (threadIdx.x != 0) return;
    ms->d2 = forced2(ms, force, force_n, 1, decode_key(k0));
    RunCtl r{};
    r.nl = 2;
    r.pos0 = ms->pos;
    r.cur = ms->cur;
    r.tok[0] = ms->x;
    r.tok[1] = ms->d1;
    r.head_mask = 3;
    r.hin_sel[0] = HID_HL;
    r.hin_sel[1] = HID_PEND;
    r.active = ms->err == 0;
    *ctl = r;
}

// piece 1: lane 0 is committed; lane 1 when d1 == g0 (else its V^T column goes back to +0). The
// pairs of the committed drafts wait for seeding (note_with: (d1, h after x), (d2, h after d1)).
// Writes piece 2's control block: d2 at p + 2 when d1 was accepted and d2 == g1.
__global__ void mtp2_commit1_kernel(MtpState *ms, RunCtl *ctl, const unsigned long long *keys, int nkeys, float *hid,
                                    uint16_t *vcache, int64_t vrows, int n_ctx, uint32_t *out_tok, int out_cap) {
    __shared__ int s_a, s_p2, s_ok, s_pos0;
    __shared__ uint32_t s_g[2];
    const int t = threadIdx.x;
    if (t < 64) {
        const unsigned long long k0 = wave_key_max(keys, nkeys), k1 = wave_key_max(keys + nkeys, nkeys);
        if (t == 0) {
            s_g[0] = decode_key(k0);
            s_g[1] = decode_key(k1);
            s_ok = ms->err == 0;
            s_a = s_ok && ms->d1 == s_g[0];
            s_p2 = s_a && ms->d2 == s_g[1];
            s_pos0 = ms->pos;
        }
    }
    __syncthreads();
    if (!s_ok) {
        if (t == 0) {
            ms->piece2 = 0;
            RunCtl r{};
            r.nl = 1;
            r.active = 0;
            *ctl = r;
        }
        return;
    }
    const int a = s_a, p2 = s_p2, pos0 = s_pos0;
    for (int i = t; i < E; i += blockDim.x) {
        const float h0 = hid[i], h1 = hid[E + i];
        if (!a) hid[(int64_t)HID_HL * E + i] = h0;
        if (a) hid[(int64_t)HID_PEND * E + i] = h0;
        if (a && !p2) hid[(int64_t)HID_HL * E + i] = h1;
        if (p2) hid[(int64_t)HID_PEND2 * E + i] = h1;
    }
    if (!a)
        for (int64_t r = t; r < vrows; r += blockDim.x) vcache[r * n_ctx + pos0 + 1] = 0;
    if (t == 0) {
        int n = ms->n_out;
        if (n < out_cap) out_tok[n++] = s_g[0];
        if (a && n < out_cap) out_tok[n++] = s_g[1];
        ms->n_out = n;
        ms->pending = a ? 1 + p2 : 0;
        ms->pend_tok = ms->d1;
        ms->pend_tok2 = ms->d2;
        ms->pos = pos0 + a + 1;
        ms->cur = (ms->cur + a + 1) % OXE_NSLOTS;
        ms->piece2 = p2;
        if (!p2) {
            ms->x = a ? s_g[1] : s_g[0];
            ms->steps += 1;
            ms->accepted += a;
        }
        RunCtl r{};
        r.nl = 1;
        r.pos0 = ms->pos;
        r.cur = ms->cur;
        r.tok[0] = ms->d2;
        r.head_mask = 1;
        r.hin_sel[0] = HID_HL;
        r.active = p2;
        *ctl = r;
    }
}

// piece 2 (one lane, always committed): g2 is the bonus token, hl the h after d2
__global__ void mtp2_commit2_kernel(MtpState *ms, const unsigned long long *keys, int nkeys, float *hid, uint32_t *out_tok,
                                    int out_cap) {
    __shared__ int s_on;
    __shared__ uint32_t s_g;
    const int t = threadIdx.x;
    if (t < 64) {
        const unsigned long long k0 = wave_key_max(keys, nkeys);
        if (t == 0) {
            s_on = ms->piece2 != 0 && ms->err == 0;
            s_g = decode_key(k0);
        }
    }
    __syncthreads();
    if (!s_on) return;
    for (int i = t; i < E; i += blockDim.x) hid[(int64_t)HID_HL * E + i] = hid[i];
    if (t == 0) {
        int n = ms->n_out;
        if (n < out_cap) out_tok[n++] = s_g;
        ms->n_out = n;
        ms->x = s_g;
        ms->pos += 1;
        ms->cur = (ms->cur + 1) % OXE_NSLOTS;
        ms->piece2 = 0;
        ms->steps += 1;
        ms->accepted += 2;
    }
}

// ---- host side ---------------------------------------------------------------------------------

void MtpDriverHost::note(Engine &e, int p0, const uint32_t *toks, int n) {
    std::vector<float> h((size_t)n * E);
    for (int i = 0; i < n; i++) e.hidden_host(i, h.data() + (size_t)i * E);
    note_h(p0, toks, n, h.data());
}

// MtpDriver::note_with (mtp.rs:415-432): the pairs (toks[i], h_nextn before toks[i]) of positions
// not yet in the MTP KV join the catch-up; hl becomes the h_nextn of the last token
void MtpDriverHost::note_h(int p0, const uint32_t *toks, int n, const float *h) {
    for (int i = 0; i < n; i++) {
        const int p = p0 + i;
        if (p >= q) {
            cu_tok.push_back(toks[i]);
            if (i == 0) cu_h.insert(cu_h.end(), hl.begin(), hl.end());
            else cu_h.insert(cu_h.end(), h + (size_t)(i - 1) * E, h + (size_t)i * E);
        }
    }
    hl.assign(h + (size_t)(n - 1) * E, h + (size_t)n * E);
}

void MtpDriverHost::remember(Engine &e, int p0, int n) {
    last_cur0 = (e.cur - n % OXE_NSLOTS + OXE_NSLOTS) % OXE_NSLOTS;   // n lanes committed from there
    last_p0 = p0;
    last_n = n;
    last_h.resize((size_t)n * E);
    for (int i = 0; i < n; i++) e.hidden_host(i, last_h.data() + (size_t)i * E);
}

int MtpDriverHost::flush(Engine &e, size_t keep) {
    while (cu_tok.size() > keep) {
        const int n = (int)std::min<size_t>(OXE_NL, cu_tok.size());
        const int rc = e.mtp_seed(cu_tok.data(), n, q, cu_h.data());
        if (rc) return rc;
        cu_tok.erase(cu_tok.begin(), cu_tok.begin() + n);
        cu_h.erase(cu_h.begin(), cu_h.begin() + (size_t)n * E);
        q += n;
    }
    return 0;
}

int MtpDriverHost::prefill(Engine &e, const uint32_t *toks, int n, uint32_t *next) {
    uint32_t nx = 0xffffffffu;
    for (int c0 = 0; c0 < n; c0 += OXE_NL) {
        const int c = std::min(OXE_NL, n - c0);
        const int p0 = e.pos;
        uint32_t g[OXE_NL];
        int rc = e.verify(toks + c0, c, g);
        if (!rc) rc = e.commit(c);
        if (rc) return rc;
        nx = g[c - 1];
        note(e, p0, toks + c0, c);
        if ((rc = flush(e, 7))) return rc;  // the reference keeps up to mtp_lanes - 1 = 7 pairs pending
    }
    last_n = 0;
    if (next) *next = nx;
    return 0;
}

// MtpDriver::prefill_batched (mtp.rs:468-500): the batched prefill with every position's h_nextn,
// then the catch-up pairs seeded into the MTP KV in one batched pass (the same K / V rows as
// 2-lane seeding runs: every pair's rows depend on that pair only). One token: step_plain.
int MtpDriverHost::prefill_batched(Engine &e, const uint32_t *toks, int n, uint32_t *next) {
    if (n == 1) {
        uint32_t g;
        const int rc = step_plain(e, toks[0], &g);
        if (rc) return rc;
        last_n = 0;
        if (next) *next = g;
        return 0;
    }
    std::vector<float> h;
    uint32_t g = 0;
    for (int c0 = 0; c0 < n; c0 += PF_CHUNK) {
        const int c = std::min(PF_CHUNK, n - c0);
        const int p0 = e.pos;
        h.resize((size_t)c * E);
        int rc = e.prefill(toks + c0, c, &g, h.data());
        if (rc) return rc;
        note_h(p0, toks + c0, c, h.data());
        const size_t keep = 7;
        if (cu_tok.size() > keep) {
            const int ns = (int)(cu_tok.size() - keep);
            if ((rc = e.seed_batched(cu_tok.data(), ns, q, cu_h.data()))) return rc;
            cu_tok.erase(cu_tok.begin(), cu_tok.begin() + ns);
            cu_h.erase(cu_h.begin(), cu_h.begin() + (size_t)ns * E);
            q += ns;
        }
    }
    last_n = 0;
    if (next) *next = g;
    return 0;
}

int MtpDriverHost::step(Engine &e, uint32_t x, uint32_t *out, int *n_out, int64_t override_d1) {
    return step_k(e, x, out, n_out, &override_d1, 1, nullptr);
}

// MtpDriver::step (mtp.rs:522-592) at depth k = min(depth, room): the catch-up seeded, the draft
// chain d_1 = MTP(x, h_prev) at p, d_i = MTP(d_{i-1}, h of the previous MTP run) at p + i - 1;
// force[i] >= 0 replaces d_{i+1} after the chain (the draft_override hook, mtp.rs:554-558); then
// the verify of [x, d_1..d_k] with greedy acceptance. The verify runs in pieces of at most OXE_NL
// lanes, each committed before the next, and stops at the first rejected draft: a run of n lanes
// computes exactly n steps, so the committed state, argmaxes, hidden rows and logits are those of
// the reference's single (k+1)-lane verify and commit(a+1). rows (optional, host [k+1][n_vocab]):
// the logits of every committed lane.
int MtpDriverHost::step_k(Engine &e, uint32_t x, uint32_t *out, int *n_out, const int64_t *force, int nforce,
                          float *rows) {
    const int p = e.pos, cur0 = e.cur;
    const int k = std::min(depth, std::max(0, e.m.n_ctx - (p + 1)));
    int rc = flush(e, 7);
    if (rc) return rc;
    if (k == 0) {
        uint32_t g;
        if ((rc = e.verify(&x, 1, &g)) || (rc = e.commit(1))) return rc;
        note(e, p, &x, 1);
        remember(e, p, 1);
        if (rows && hipMemcpy(rows, e.b.logits, (size_t)e.d.n_vocab * 4, hipMemcpyDeviceToHost) != hipSuccess) return -2;
        out[0] = g;
        *n_out = 1;
        return 0;
    }
    if ((rc = flush(e, 0))) return rc;
    uint32_t d[MTP_MAX_DEPTH];
    if ((rc = e.mtp_run(&x, 1, p, hl.data(), 1, &d[0]))) return rc;
    q = p + 1;
    std::vector<float> h(E);
    for (int i = 1; i < k; i++) {
        if ((rc = e.hidden_host(0, h.data()))) return rc;
        if ((rc = e.mtp_run(&d[i - 1], 1, p + i, h.data(), 1, &d[i]))) return rc;
    }
    for (int i = 0; i < k && i < nforce; i++)
        if (force[i] >= 0) d[i] = (uint32_t)force[i];
    uint32_t vt[MTP_MAX_DEPTH + 1], g[MTP_MAX_DEPTH + 1];
    vt[0] = x;
    for (int i = 0; i < k; i++) vt[1 + i] = d[i];
    std::vector<float> hs((size_t)(k + 1) * E);
    int done = 0;
    for (bool more = true; more;) {
        const int n = std::min(OXE_NL, k + 1 - done);
        if ((rc = e.verify(vt + done, n, g + done))) return rc;
        int m = 0;   // lanes of this piece to commit: lane j, then j + 1 while d_{j+1} == g_j
        for (int j = done; j < done + n; j++) {
            m++;
            if (j >= k || vt[j + 1] != g[j]) {
                more = false;
                break;
            }
        }
        for (int j = 0; j < m; j++) {
            if ((rc = e.hidden_host(j, hs.data() + (size_t)(done + j) * E))) return rc;
            if (rows && hipMemcpy(rows + (size_t)(done + j) * e.d.n_vocab, e.b.logits + (size_t)j * e.d.n_vocab,
                                  (size_t)e.d.n_vocab * 4, hipMemcpyDeviceToHost) != hipSuccess)
                return -2;
        }
        if ((rc = e.commit(m))) return rc;
        done += m;
    }
    const int a = done - 1;
    note_h(p, vt, a + 1, hs.data());
    last_p0 = p;
    last_n = a + 1;
    last_cur0 = cur0;
    last_h.assign(hs.begin(), hs.begin() + (size_t)(a + 1) * E);
    steps++;
    drafted += k;
    accepted += a;
    for (int i = 0; i <= a; i++) out[i] = g[i];
    *n_out = a + 1;
    return 0;
}

// MtpDriver::step_plain (mtp.rs:504-515): one target step that keeps the MTP catch-up in sync
int MtpDriverHost::step_plain(Engine &e, uint32_t x, uint32_t *out) {
    const int p = e.pos;
    uint32_t g;
    int rc;
    if ((rc = e.verify(&x, 1, &g)) || (rc = e.commit(1))) return rc;
    note(e, p, &x, 1);
    remember(e, p, 1);
    if ((rc = flush(e, 7))) return rc;
    *out = g;
    return 0;
}

// MtpDriver::rewind (mtp.rs:596-608): keep the first m committed tokens of the last step. Inside
// the step's last verify piece this is a smaller commit; before it, a rollback to the slot that
// holds the state after token m (the step began at slot last_cur0; lane j wrote slot + j + 1).
int MtpDriverHost::rewind(Engine &e, int m) {
    if (last_n == 0 || m < 1 || m > last_n) return -1;
    if (m == last_n) return 0;
    const int target = last_p0 + m;
    int rc = (e.pend_n > 0 && target > e.pend_pos0) ? e.commit(target - e.pend_pos0)
                                                     : e.rollback(target, (last_cur0 + m) % OXE_NSLOTS);
    if (rc) return rc;
    const size_t keep = std::min<size_t>((size_t)std::max(0, last_p0 + m - q), cu_tok.size());
    cu_tok.resize(keep);
    cu_h.resize(keep * E);
    hl.assign(last_h.begin() + (size_t)(m - 1) * E, last_h.begin() + (size_t)m * E);
    last_n = m;
    return 0;
}

// device-driven: hand the host driver state to the device, run K graph steps, read it back
int MtpDriverHost::dev_begin(Engine &e, uint32_t x) {
    last_n = 0;  // rewind applies to host-driven steps only
    int rc = flush(e, 0);  // at most the pairs the next step seeds stay pending: none here
    if (rc) return rc;
    if (e.dev_depth != depth) {  // a captured step is for one depth
        if (e.graph_exec) (void)hipGraphExecDestroy(e.graph_exec);
        e.graph_exec = nullptr;
        e.dev_depth = depth;
    }
    MtpState s{};
    s.pos = e.pos;
    s.cur = e.cur;
    s.x = x;
    s.pending = 0;
    s.n_out = 0;
    s.zcol = -1;
    if (hipMemcpyAsync(e.mtp_state, &s, sizeof(s), hipMemcpyHostToDevice, e.st) != hipSuccess) return -2;
    if (hipMemcpyAsync(e.b.hid + (size_t)HID_HL * E, hl.data(), (size_t)E * 4, hipMemcpyHostToDevice, e.st) != hipSuccess) return -2;
    hipLaunchKernelGGL(mtp_prep_step_kernel, dim3(1), dim3(1), 0, e.st, e.mtp_state, e.ctl_draft, e.m.n_ctx);
    return hipStreamSynchronize(e.st) == hipSuccess ? 0 : -2;
}

int MtpDriverHost::dev_end(Engine &e, uint32_t *out_tok, int cap, int *n_out, uint32_t *next_x) {
    MtpState s{};
    if (hipMemcpyAsync(&s, e.mtp_state, sizeof(s), hipMemcpyDeviceToHost, e.st) != hipSuccess) return -2;
    if (hipStreamSynchronize(e.st) != hipSuccess) return -2;
    // An aborted run (-5) commits nothing, and every step after it in this batch is inactive: the
    // device state is that of the last step that ran, and is handed back below like any other.
    const int abort_rc = e.fused_check();
    if (abort_rc != 0 && abort_rc != -5) return abort_rc;
    const bool aborted = abort_rc == -5 || (s.err & 4) != 0;
    if (s.zcol >= 0 && s.zcol < e.m.n_ctx) {   // the last rejected lane's V^T column (zero_v)
        launch_zero_v(e.m, e.n_att_main, s.zcol, s.zcol + 1, e.st);
        if (hipStreamSynchronize(e.st) != hipSuccess) return -2;
    }
    if (aborted && s.pos < e.m.n_ctx) {
        // the V^T columns an aborted verify (up to 3 lanes from pos) may have written go back to +0
        launch_zero_v(e.m, e.n_att_main, s.pos, std::min(s.pos + 3, e.m.n_ctx), e.st);
        if (hipStreamSynchronize(e.st) != hipSuccess) return -2;
    }
    const int n = std::min(s.n_out, cap);
    if (n > 0 && hipMemcpy(out_tok, e.out_tok, (size_t)n * 4, hipMemcpyDeviceToHost) != hipSuccess) return -2;
    *n_out = n;
    *next_x = s.x;
    hl.resize(E);
    if (hipMemcpy(hl.data(), e.b.hid + (size_t)HID_HL * E, (size_t)E * 4, hipMemcpyDeviceToHost) != hipSuccess) return -2;
    cu_tok.clear();
    cu_h.clear();
    const int np = std::max(0, std::min(s.pending, 2));
    if (np > 0) {
        const uint32_t pt[2] = {s.pend_tok, s.pend_tok2};
        const int hb[2] = {HID_PEND, HID_PEND2};
        cu_h.resize((size_t)np * E);
        for (int i = 0; i < np; i++) {
            cu_tok.push_back(pt[i]);
            if (hipMemcpy(cu_h.data() + (size_t)i * E, e.b.hid + (size_t)hb[i] * E, (size_t)E * 4, hipMemcpyDeviceToHost) !=
                hipSuccess)
                return -2;
        }
    }
    q = s.pos - np;
    e.pos = s.pos;
    e.cur = s.cur;
    e.pend_n = 0;
    steps += s.steps;
    accepted += s.accepted;
    drafted += (int64_t)s.steps * e.dev_depth;   // dev_depth drafts per device-driven step
    if (aborted) {
        if (abort_rc == 0) set_err("fused run aborted: an exchange poll timed out (nothing committed)");
        return -5;
    }
    return s.err ? -4 : 0;
}

void Engine::enqueue_mtp_device_step() {
    if (fused) {
        // two launches: the draft run (with the pending pair, if any) reads its control block, filled
        // by the previous step's verify run (or dev_begin), and its last stage prepares the verify's;
        // the verify run's last stage accepts / commits and fills the next draft's
        enqueue_mtp_run(ctl_draft);
        enqueue_verify();
        return;
    }
    hipLaunchKernelGGL(mtp_prep_draft_kernel, dim3(1), dim3(1), 0, st, mtp_state, ctl, m.n_ctx);
    enqueue_mtp_run();
    hipLaunchKernelGGL(mtp_prep_verify_kernel, dim3(1), dim3(64), 0, st, mtp_state, ctl, keys(), nkeys(),
                       (const int32_t *)force_d1, force_n, m.n_ctx);
    enqueue_verify();
    hipLaunchKernelGGL(mtp_commit_kernel, dim3(1), dim3(256), 0, st, mtp_state, keys(), nkeys(), b.hid, m.n_ctx,
                       out_tok, out_cap, ctl_draft);
}

void Engine::enqueue_mtp_device_step2() {
    const int32_t *force = (const int32_t *)force_d1;
    hipLaunchKernelGGL(mtp2_prep_seed_kernel, dim3(1), dim3(1), 0, st, mtp_state, ctl);
    enqueue_mtp_seed();
    hipLaunchKernelGGL(mtp2_prep_draft1_kernel, dim3(1), dim3(1), 0, st, mtp_state, ctl, m.n_ctx);
    enqueue_mtp_run();
    hipLaunchKernelGGL(mtp2_prep_draft2_kernel, dim3(1), dim3(256), 0, st, mtp_state, ctl, keys(), nkeys(), b.hid, force,
                       force_n);
    enqueue_mtp_run();
    hipLaunchKernelGGL(mtp2_prep_verify1_kernel, dim3(1), dim3(64), 0, st, mtp_state, ctl, keys(), nkeys(), force, force_n);
    enqueue_verify();
    hipLaunchKernelGGL(mtp2_commit1_kernel, dim3(1), dim3(256), 0, st, mtp_state, ctl, keys(), nkeys(), b.hid, m.vcache,
                       (int64_t)n_att_main * NKV * HD, m.n_ctx, out_tok, out_cap);
    enqueue_verify();
    hipLaunchKernelGGL(mtp2_commit2_kernel, dim3(1), dim3(256), 0, st, mtp_state, keys(), nkeys(), b.hid, out_tok, out_cap);
}

int Engine::mtp_steps_async(int k, bool use_graph) {
    if (!use_graph) {
        for (int i = 0; i < k; i++) {
            if (dev_depth == 2) enqueue_mtp_device_step2();
            else enqueue_mtp_device_step();
        }
        return hipGetLastError() == hipSuccess ? 0 : -2;
    }
    if (!graph_exec) {
        if (!st) {
            set_err("graph steps need a created stream: this engine runs on the null stream");
            return -1;
        }
        if (hipStreamBeginCapture(st, hipStreamCaptureModeThreadLocal) != hipSuccess) return -2;
        fz_capturing = true;
        if (dev_depth == 2) enqueue_mtp_device_step2();
        else enqueue_mtp_device_step();
        fz_capturing = false;
        hipGraph_t g;
        if (hipStreamEndCapture(st, &g) != hipSuccess) return -2;
        if (hipGraphInstantiate(&graph_exec, g, nullptr, nullptr, 0) != hipSuccess) return -2;
        (void)hipGraphDestroy(g);
    }
    for (int i = 0; i < k; i++) {
        if (fused) fz_account(dev_depth == 2 ? 5 : 2);   // the fused launches of one step
        if (hipGraphLaunch(graph_exec, st) != hipSuccess) return -2;
    }
    return 0;
}

}  // namespace oxe

using oxe::Engine;

extern "C" {

// Eagerly enqueue k device-driven MTP steps with HIP events around every launch of kernel `kind`
// (engine stream); *avg_us = mean launch duration, *n = launches timed. For the bench's roofline.
int oxe_mtp_device_probe(oxe_engine *e, int k, int kind, float *avg_us, int *n) {
    Engine *g = (Engine *)e;
    if (k < 1 || kind < 0 || !avg_us || !n) return -1;
    g->probe_kind = kind;
    g->probe_used = 0;
    int rc = g->mtp_steps_async(k, false);
    g->probe_kind = -1;
    if (rc) return rc;
    if (hipStreamSynchronize(g->st) != hipSuccess) return -2;
    if ((rc = g->fused_check())) return rc;
    double tot = 0.0;
    int cnt = 0;
    for (size_t i = 0; i + 1 < g->probe_used; i += 2) {
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, g->probe_ev[i], g->probe_ev[i + 1]) != hipSuccess) return -2;
        tot += ms;
        cnt++;
    }
    *avg_us = cnt ? (float)(tot * 1000.0 / cnt) : 0.0f;
    *n = cnt;
    return 0;
}

int oxe_mtp_prefill(oxe_engine *e, const uint32_t *toks, int n, uint32_t *next) {
    Engine *g = (Engine *)e;
    if (n < 1 || !g->toks_ok(toks, n) || g->pos + n > g->m.n_ctx) return -1;
    return g->drv.prefill(*g, toks, n, next);
}

int oxe_mtp_prefill_batched(oxe_engine *e, const uint32_t *toks, int n, uint32_t *next) {
    Engine *g = (Engine *)e;
    if (n < 1 || !g->toks_ok(toks, n) || g->pos + n > g->m.n_ctx) return -1;
    return g->drv.prefill_batched(*g, toks, n, next);
}

int oxe_engine_prefill(oxe_engine *e, const uint32_t *toks, int n, uint32_t *next, float *hidden) {
    Engine *g = (Engine *)e;
    if (n < 1 || !g->toks_ok(toks, n) || g->pos + n > g->m.n_ctx) return -1;
    return g->prefill(toks, n, next, hidden);
}

int oxe_mtp_step(oxe_engine *e, uint32_t x, uint32_t *out, int *n_out, int64_t override_d1) {
    Engine *g = (Engine *)e;
    if (!g->toks_ok(&x, 1) || override_d1 >= g->d.n_vocab || !out || !n_out) return -1;
    return g->drv.step(*g, x, out, n_out, override_d1);
}

int oxe_mtp_step_force(oxe_engine *e, uint32_t x, uint32_t *out, int *n_out, const int64_t *force, int nforce) {
    Engine *g = (Engine *)e;
    if (!g->toks_ok(&x, 1) || !out || !n_out || nforce < 0 || (nforce > 0 && !force)) return -1;
    for (int i = 0; i < nforce; i++)
        if (force[i] >= g->d.n_vocab) return -1;
    return g->drv.step_k(*g, x, out, n_out, force, nforce, nullptr);
}

int oxe_mtp_set_depth(oxe_engine *e, int depth) {
    Engine *g = (Engine *)e;
    if (depth < 1 || depth > oxe::MTP_MAX_DEPTH) return -1;
    g->drv.depth = depth;
    return 0;
}

int oxe_mtp_step_plain(oxe_engine *e, uint32_t x, uint32_t *out) {
    Engine *g = (Engine *)e;
    if (!g->toks_ok(&x, 1) || !out) return -1;
    return g->drv.step_plain(*g, x, out);
}

int oxe_mtp_rewind(oxe_engine *e, int m) {
    Engine *g = (Engine *)e;
    return g->drv.rewind(*g, m);
}

int oxe_mtp_set_force(oxe_engine *e, const int32_t *force_d1, int n) {
    Engine *g = (Engine *)e;
    return g->set_force(force_d1, n);
}

int oxe_mtp_set_draft_vocab(oxe_engine *e, const uint32_t *ids, int n) {
    Engine *g = (Engine *)e;
    if (!g) return -1;
    return g->set_draft_vocab(ids, n);
}

int oxe_mtp_device_begin(oxe_engine *e, uint32_t x, int out_cap) {
    Engine *g = (Engine *)e;
    if (out_cap < 1 || !g->toks_ok(&x, 1)) return -1;
    if (g->drv.depth != 1 && g->drv.depth != 2) {
        oxe::set_err("device-driven MTP steps are depth 1 or 2");
        return -1;
    }
    if (g->ensure_out(out_cap)) return -3;
    return g->drv.dev_begin(*g, x);
}

int oxe_mtp_device_steps(oxe_engine *e, int k, int use_graph) {
    Engine *g = (Engine *)e;
    if (k < 0) return -1;
    return g->mtp_steps_async(k, use_graph != 0);
}

int oxe_mtp_device_end(oxe_engine *e, uint32_t *out_tok, int cap, int *n_out, uint32_t *next_x) {
    Engine *g = (Engine *)e;
    return g->drv.dev_end(*g, out_tok, cap, n_out, next_x);
}

int oxe_mtp_stats(const oxe_engine *e, int64_t *st) {
    const Engine *g = (const Engine *)e;
    st[0] = g->drv.steps;
    st[1] = g->drv.accepted;
    st[2] = g->drv.drafted;
    return 0;
}

int oxe_engine_sync(oxe_engine *e) {
    Engine *g = (Engine *)e;
    return hipStreamSynchronize(g->st) == hipSuccess ? 0 : -2;
}

void *oxe_engine_stream(oxe_engine *e) { return (void *)((Engine *)e)->st; }

}  // extern "C"
