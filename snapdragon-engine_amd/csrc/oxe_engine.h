// Device-resident state of the MI355X decode engine: weight arena, recurrent slots, KV cache,
// per-lane activations and the run control block every kernel reads.
//
// Reference state (crates/model/src/engine.rs:393-560, 918-953): conv/ssm state [slot][layer],
// K cache [layer][kv head][pos][head_dim] f16, V^T cache [layer][kv head*head_dim + dim][pos] f16,
// lanes of up to MAX_LANES tokens. Here all of it lives in HBM; the host never reads it on the hot
// path. Lanes per kernel launch: at most OXE_NL (2, the verify width of depth-1 MTP).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include <vector>

#include "../../include/oxe_model.h"

namespace oxe {

constexpr int OXE_NL = 2;           // lanes per launch (verify width; MTP seeding batches by 2)
constexpr int OXE_MAX_EXP_USED = 8; // top-k of the router
constexpr int OXE_MAX_UNION = 16;   // union of two lanes' top-8

// Q8_0 matrix in this build's layout: int8 codes [rows][k] + fp16 scales [rows][k/32]
struct Q8W {
    int8_t *q = nullptr;
    uint16_t *d = nullptr;
    int64_t rows = 0, k = 0;
};

// A matrix kept in a model file's own blocks: K-quant rows of k / 256 ggml blocks (type 11..14), or
// F32 rows (type 0). type 8: not used (the matrix is Q8_0, in the Q8W beside it).
struct RawW {
    uint8_t *w = nullptr;
    int type = 8;
    int64_t rows = 0, k = 0;   // per expert for the expert tensors
};
__host__ __device__ inline int kq_block_bytes(int type) {
    return type == 11 ? 110 : type == 12 ? 144 : type == 13 ? 176 : type == 14 ? 210 : 0;
}
__host__ __device__ inline int64_t raw_row_bytes(const RawW &r) {
    return r.type == 0 ? r.k * 4 : r.k / 256 * kq_block_bytes(r.type);
}

// ggml types of the matrices that may be other than Q8_0 (the reference's mv dispatches every type,
// crates/model/src/engine.rs:2270-2343): K-quant experts, shared expert, mixer projections, output
// projections, token embedding and LM head; F32 or K-quant ssm_beta / ssm_alpha. Gate and up of one
// expert kind are both Q8_0 or both K-quants; a layer's projection parts are all Q8_0 (beta / alpha
// Q8_0 or F32) or all in the file's blocks.
struct LayerTypes {
    int gate = 8, up = 8, down = 8, sh_gate = 8, sh_up = 8, sh_down = 8, beta = 8, alpha = 8;
    // the mixer's projections (delta-net qkv / z, attention q / k / v) and output projection
    int qkv = 8, z = 8, q = 8, k = 8, v = 8, out = 8;
    bool any() const {
        return gate != 8 || up != 8 || down != 8 || sh_gate != 8 || sh_up != 8 || sh_down != 8 || beta != 8 || alpha != 8 ||
               qkv != 8 || z != 8 || q != 8 || k != 8 || v != 8 || out != 8;
    }
};
struct ModelTypes {
    std::vector<LayerTypes> layer;   // n_layer + 1 (the MTP block last)
    int output = 8, tok_embd = 8;
    bool any() const {
        for (const LayerTypes &t : layer)
            if (t.any()) return true;
        return output != 8 || tok_embd != 8;
    }
};

// recurrent slots: lane i reads slot cur+i, writes cur+i+1 (never in place). Five keep the state
// after every position of an MTP depth-3 step (4 lanes verified in pieces of OXE_NL), so a rewind
// can return to any committed prefix of it.
constexpr int OXE_NSLOTS = 5;

// Run control (device memory). Written by the host through a tiny kernel for host-driven calls and,
// for the device-driven MTP step, by the step's decision code (the control kernels of per-phase runs,
// the last stage of fused draft and verify runs); read by every kernel of a run.
struct RunCtl {
    int32_t nl;          // lanes of this run (1..OXE_NL)
    int32_t pos0;        // position of lane 0
    int32_t cur;         // recurrent slot holding the state before lane 0 (lane i writes slot (cur + i + 1) % OXE_NSLOTS)
    int32_t head_mask;   // lanes whose LM-head argmax is wanted
    uint32_t tok[OXE_NL];
    int32_t hin_sel[OXE_NL]; // MTP entry: which hidden buffer feeds lane i (index into hid[])
    int32_t active;      // 0: every kernel of this run returns at once (conditional MTP seeding)
    int32_t stage;       // fused runs of the device-driven MTP step: 1 after a draft run (prepare the
                         // verify), 2 after a verify run (accept / commit); 0 otherwise
};

// Device-driven MTP state (crates/model/src/mtp.rs:314-340 MtpDriver, depth 1 or 2)
struct MtpState {
    int32_t pos;         // committed position P (tokens in the target)
    int32_t cur;         // current recurrent slot
    uint32_t x;          // next token (not yet in the target)
    int32_t pending;     // pairs waiting for MTP seeding at pos - pending .. pos - 1 (0..depth):
    uint32_t pend_tok;   // (pend_tok, hidden buffer HID_PEND), then (pend_tok2, HID_PEND2)
    int32_t n_out;       // tokens emitted so far (ring position in out_tok)
    int32_t steps, accepted;
    uint32_t d1;         // drafts of the current step
    int32_t err;         // sticky error bits (1: context full; 2: no room for a depth-2 step)
    uint32_t pend_tok2;
    uint32_t d2;
    int32_t piece2;      // depth 2: the current step verifies d2 in a second piece
    int32_t zcol;        // depth 1: a rejected lane's V^T column not yet back to +0 (-1: none); the
                         // next step's verify overwrites it, dev_end zeroes it if no step did
};

// hidden-state buffers ([HID_N][n_embd] floats): 0..NL-1 h_nextn per lane of the last run, HID_HL
// the target h of position pos-1 (MtpDriver.hl), HID_PEND / HID_PEND2 the pending catch-up pairs'
// h, HID_M the first draft run's MTP h (the second draft's input at depth 2).
constexpr int HID_HL = OXE_NL;
constexpr int HID_PEND = OXE_NL + 1;
constexpr int HID_PEND2 = OXE_NL + 2;
constexpr int HID_M = OXE_NL + 3;
constexpr int HID_N = OXE_NL + 4;

struct LayerW {
    int att = 0;    // 1: full attention (+ MTP block), 0: gated delta-net
    int index = 0;  // recurrent or attention index
    float *attn_norm = nullptr, *post_norm = nullptr;
    Q8W proj;       // DN: [qkv | z | beta | alpha]; ATT: [q(+gate) | k | v]
    Q8W out;        // ssm_out / attn_output [n_embd][4096]
    float *conv = nullptr, *ssm_a = nullptr, *dt_bias = nullptr, *ssm_norm = nullptr;  // DN
    float *q_norm = nullptr, *k_norm = nullptr;                                          // ATT
    float *router = nullptr, *shexp_gate = nullptr;  // [n_expert][n_embd], [n_embd]
    Q8W shexp_gu;   // shared gate/up, rows interleaved per 16-row tile: 8 gate rows then 8 up rows
    Q8W shexp_down; // [n_embd][ff_shexp]
    Q8W exp_gu;     // [n_expert][2*ff_exp][n_embd], per expert interleaved like shexp_gu
    Q8W exp_down;   // [n_expert][n_embd][ff_exp]
    Q8W eh_proj;    // MTP block only: [n_embd][2*n_embd]
    float *enorm = nullptr, *hnorm = nullptr, *head_norm = nullptr;
    // matrices of other types (a model file's), used in place of the Q8W ones above when their type
    // is not 8: experts [n_expert][rows][k], the shared expert, ssm_beta / ssm_alpha [n_vheads][n_embd]
    RawW exp_gate_r, exp_up_r, exp_down_r, sh_gate_r, sh_up_r, sh_down_r, beta_r, alpha_r;
    // K-quant mixer matrices: delta-net qkv / z, attention q (+ gate) / k / v, the output projection
    RawW qkv_r, z_r, q_r, k_r, v_r, out_r;
    bool kq_moe() const {
        return exp_gate_r.type != 8 || exp_down_r.type != 8 || sh_gate_r.type != 8 || sh_down_r.type != 8;
    }
    // the projection's parts in the file's blocks, with no Q8_0 projection matrix: a delta-net
    // layer's qkv and z (its beta / alpha then K-quants or F32), an attention layer's q, k and v
    bool kq_proj() const { return qkv_r.type != 8 || q_r.type != 8; }
};

// Per-lane activation buffers, all [OXE_NL][...]
struct ActBufs {
    float *x;          // layer input
    float *x1;         // after the mixer residual
    float *x2;         // after the MoE (next layer input)
    int8_t *xq;        // quantized normalized activations [NL][2*n_embd] (+ scales xd)
    uint16_t *xd;
    float *xn;         // normalized f32 (router input) [NL][n_embd]
    float *proj;       // projection outputs [NL][proj_max]
    float *gdn;        // delta-net outputs before the gated norm [NL][d_inner]
    int8_t *oq;        // quantized mixer output [NL][4096] (+ od)
    uint16_t *od;
    float *scores;     // attention scores [NL][n_head][n_ctx]
    float *router_lg;  // [NL][n_expert]
    float *sh_gate;    // [NL]
    float *hsh;        // shared expert swiglu [NL][ff_shexp]
    float *hexp;       // routed expert swiglu [NL][k_used][ff_exp]
    int32_t *route_ids;   // [NL][k_used]
    float *route_w;       // [NL][k_used]
    int32_t *uni;         // [OXE_MAX_UNION + 1]: count, then expert ids in first-use order
    float *hid;           // [HID_N][n_embd]
    float *logits;        // [NL][n_vocab] (optional)
    unsigned long long *amax_key;  // [NL] packed argmax keys
    uint8_t *xk;          // q8_K blocks of xn [NL][n_embd / 256] (K-quant matrices)
    uint8_t *hk;          // q8_K blocks of hexp [NL][k_used][ff_exp / 256]
    uint8_t *hshk;        // q8_K blocks of hsh [NL][ff_shexp / 256]
    float *o32;           // the mixer's gated outputs in f32 [NL][4096] (a K-quant output projection)
    uint8_t *ok;          // their q8_K blocks [NL][4096 / 256]
    float *emb;           // the lanes' embedded tokens [NL][n_embd] (a K-quant token embedding)
    uint32_t *counters;   // per-kernel completion counters (zeroed at allocation; self-resetting)
};

}  // namespace oxe
