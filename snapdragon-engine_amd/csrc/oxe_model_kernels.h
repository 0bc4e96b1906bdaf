// Argument blocks and launchers of the per-layer decode kernels (k_layer.hip, k_attn.hip,
// k_moe.hip). Each launcher enqueues one kernel on `st`; kernels read the run's lanes, positions
// and slots from the device-side RunCtl, so a whole step can be captured once in a HIP graph.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oxe_engine.h"

namespace oxe {

// ids of the self-resetting completion counters in ActBufs::counters
enum CounterId { CNT_DN = 0, CNT_ERR_TIE = 64, CNT_ROUTE = 65, CNT_UNI_SUM = 66, CNT_EXP_CALLS = 67, CNT_N = 128 };

struct ModelRt {
    // runtime shape
    int n_layer, n_vocab, n_ctx, n_att;
    float eps;
    // global tensors
    Q8W tok_embd, output;
    RawW output_r;         // the LM head in another type (output_r.type != 8), else unused
    RawW tok_embd_r;       // a K-quant token embedding (tok_embd_r.type != 8), else unused
    float *out_norm;
    // state
    float *conv_state;     // [NSLOTS][n_rec][NCH][KC-1]
    float *ssm_state;      // [NSLOTS][n_rec][NVH][HV][HV]
    uint16_t *kcache;      // [n_att][NKV][n_ctx][HD]
    uint16_t *vcache;      // [n_att][NKV*HD][n_ctx]
    float *rope;           // [n_ctx][NROT] (cos, sin pairs)
    int n_rec;
};

void launch_set_run(RunCtl *ctl, const RunCtl &v, hipStream_t st);

// layer input of the verify: layer 0 embeds the lanes' tokens (the Q8_0 embedding, or b.emb when the
// embedding is a K-quant)
void launch_proj(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const float *x, bool embed, float *x_store,
                 const ActBufs &b, hipStream_t st, int64_t row_begin = 0);
void launch_zero_v(const ModelRt &m, int n_att_main, int p0, int p1, hipStream_t st);
// o32 (optional): the gated outputs also as f32 (for a K-quant output projection)
void launch_dn(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st, float *o32 = nullptr);
void launch_out(const RunCtl *ctl, const LayerW &w, const float *x, const ActBufs &b, hipStream_t st);
void launch_kwrite(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st);
void launch_scores(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st);
void launch_pv(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st, float *o32 = nullptr);
void launch_router(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st);
void launch_route(const RunCtl *ctl, const ActBufs &b, hipStream_t st);
void launch_experts(const RunCtl *ctl, const LayerW &w, const ActBufs &b, hipStream_t st);
void launch_down(const RunCtl *ctl, const LayerW &w, const ActBufs &b, hipStream_t st);
// w / ids: a restricted draft head (rows of the output matrix, local row r = token ids[r]); null: the
// output matrix, row r = token r
void launch_head(const RunCtl *ctl, const ModelRt &m, const float *norm_w, const ActBufs &b, bool store_logits,
                 hipStream_t st, const Q8W *w = nullptr, const uint32_t *ids = nullptr);
// emb (optional): the lanes' embedded tokens [NL][n_embd] (a K-quant token embedding), else the
// Q8_0 embedding is read directly
void launch_entry(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st,
                  const float *emb = nullptr);

// K-quant / F32 matrices in the per-phase runs (k_kquant.hip): F32 ssm_beta / ssm_alpha rows after
// the projection; the MoE's gate / up and down of a layer with any K-quant expert or shared matrix;
// the LM head over a K-quant output matrix. Each returns 0 or -2 (a launch failed).
int launch_ba_f32(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const float *x, const ActBufs &b, hipStream_t st);
int launch_kq_moe(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const ActBufs &b, hipStream_t st);
int launch_kq_head(const RunCtl *ctl, const ModelRt &m, const float *norm_w, const ActBufs &b, hipStream_t st,
                   const RawW *w = nullptr, const uint32_t *ids = nullptr);
// The projection of a layer whose parts are in the file's blocks (w.kq_proj()): the lanes' input
// (the embedding when embed, stored to x_store; else x) normed into b.xn and quantised to q8_K, then
// each K-quant part's rows into b.proj at the part's offset (V rows also to V^T); F32 beta / alpha
// rows follow with launch_ba_f32. row_begin: only the parts at or after it (MTP seeding: K and V).
int launch_kq_proj(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const float *x, bool embed, float *x_store,
                   const ActBufs &b, hipStream_t st, int64_t row_begin = 0);
// The K-quant output projection: the mixer's f32 gated outputs (b.o32) quantised to q8_K, the
// GEMV, + the residual x into x1.
int launch_kq_out(const RunCtl *ctl, const ModelRt &m, const LayerW &w, const float *x, const ActBufs &b, hipStream_t st);
// the lanes' tokens of a K-quant token embedding, dequantised into out [NL][n_embd]
int launch_kq_embed(const RunCtl *ctl, const ModelRt &m, float *out, hipStream_t st);

}  // namespace oxe
