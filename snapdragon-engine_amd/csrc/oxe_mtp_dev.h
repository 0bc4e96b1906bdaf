// The device-driven MTP depth-1 step's decisions (crates/model/src/mtp.rs:522-591 with depth 1,
// engine.rs:2030-2039), shared by the one-workgroup control kernels (per-phase runs) and the last
// stage of the fused runs (workgroup 0, after every other workgroup of the launch is done).
#pragma once
#include <hip/hip_runtime.h>

#include "oxe_engine.h"
#include "oxe_shape.h"

namespace oxe {

// the argmax key's row (keys: largest value, then smallest row; 0 = none)
__host__ __device__ inline uint32_t decode_key(unsigned long long k) { return k == 0 ? 0u : 0xffffffffu - (uint32_t)(k & 0xffffffffu); }

// The draft run's control block of the step about to start. A pending catch-up pair (the accepted
// draft of the previous step with the target h before it) rides along as lane 0 at pos - 1 and the
// draft (x, hl) is the last lane: the pair's MTP K / V rows are written by the same run that reads
// them (lanes are independent but for the attention over earlier positions, which includes the
// run's own rows), as the reference's batched MTP call takes its pending pairs with the draft. Only
// the last lane's LM-head argmax is wanted. Inactive when the 2-lane verify has no room (the step
// then stops the driver, as the reference's k = 0; mtp_after_draft records it). stage 1: a fused
// draft run prepares the verify itself.
__device__ inline RunCtl draft_ctl(const MtpState *ms, int n_ctx) {
    const int np = ms->pending != 0 ? 1 : 0;
    RunCtl r{};
    r.nl = 1 + np;
    r.pos0 = ms->pos - np;
    r.cur = ms->cur;
    r.tok[0] = np ? ms->pend_tok : ms->x;
    r.tok[1] = ms->x;
    r.hin_sel[0] = np ? HID_PEND : HID_HL;
    r.hin_sel[1] = HID_HL;
    r.head_mask = 1 << np;
    r.active = ms->err == 0 && ms->pos + 2 <= n_ctx;
    r.stage = 1;
    return r;
}

// After the draft run (one thread): d1 from the draft lane's largest key (the test hook force[step]
// >= 0 replaces it, mtp.rs:554-558), the context check, and the verify's control block (stage 2: a
// fused verify run commits itself).
__device__ inline RunCtl mtp_after_draft(MtpState *ms, unsigned long long kmax, const int32_t *force, int force_n,
                                         int n_ctx) {
    if (ms->pos + 2 > n_ctx) ms->err |= 1;  // no room for the 2-lane verify: stop (reference: k = 0)
    uint32_t d1 = decode_key(kmax);
    if (force && ms->steps < force_n && force[ms->steps] >= 0) d1 = (uint32_t)force[ms->steps];
    ms->d1 = d1;
    RunCtl r{};
    r.nl = 2;
    r.pos0 = ms->pos;
    r.cur = ms->cur;
    r.tok[0] = ms->x;
    r.tok[1] = d1;
    r.head_mask = 3;
    r.hin_sel[0] = HID_HL;
    r.hin_sel[1] = HID_PEND;
    r.active = ms->err == 0;
    r.stage = 2;
    return r;
}

struct CommitSm {
    int a, ok, pos0;
};

// Accept / commit / note after the verify (mtp.rs:564-591): a = (d1 == g0). Every thread of one
// workgroup calls it; ran: the verify ran to its end. hl becomes the h_nextn after the last committed
// token, the accepted draft's pair (d1, h after x) waits for seeding, the committed argmax tokens are
// emitted, and the next step's draft control block goes to cd. A rejected lane's V^T column of the
// main attention layers must go back to +0 (zero_v, engine.rs:2030-2039) before anything reads it:
// the next step's verify writes that column (its lane 0 sits at that position) before any of its
// phases reads it, so the column is only recorded (zcol) and zeroed by dev_end when no further step
// ran.
__device__ inline void mtp_commit(MtpState *ms, bool ran, uint32_t g0, uint32_t g1, float *hid, int n_ctx,
                                  uint32_t *out_tok, int out_cap, RunCtl *cd, CommitSm &sm) {
    const int t = threadIdx.x;
    if (t == 0) {
        sm.ok = ran && ms->err == 0;
        sm.a = sm.ok && ms->d1 == g0;
        sm.pos0 = ms->pos;
    }
    __syncthreads();
    if (!sm.ok) {
        if (t == 0) *cd = draft_ctl(ms, n_ctx);
        return;
    }
    const int a = sm.a, pos0 = sm.pos0;
    for (int i = t; i < shp::E; i += blockDim.x) {
        const float h0 = hid[i], h1 = hid[shp::E + i];
        hid[(int64_t)HID_HL * shp::E + i] = a ? h1 : h0;
        if (a) hid[(int64_t)HID_PEND * shp::E + i] = h0;
    }
    if (t == 0) {
        ms->zcol = a ? -1 : pos0 + 1;
        int n = ms->n_out;
        if (n < out_cap) out_tok[n++] = g0;
        if (a && n < out_cap) out_tok[n++] = g1;
        ms->n_out = n;
        ms->x = a ? g1 : g0;
        ms->pending = a;
        ms->pend_tok = ms->d1;
        ms->pos = pos0 + a + 1;
        ms->cur = (ms->cur + a + 1) % OXE_NSLOTS;
        ms->steps += 1;
        ms->accepted += a;
        *cd = draft_ctl(ms, n_ctx);
    }
}

}  // namespace oxe
