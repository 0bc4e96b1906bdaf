// TEST INFRASTRUCTURE ONLY (see oxo.h). C API of the oracle engine and MTP driver (model.cpp).
#pragma once
#include <stdint.h>
#include "../include/oxe_model.h"

#ifdef __cplusplus
extern "C" {
#endif
typedef struct oxo_engine oxo_engine;
typedef struct oxo_driver oxo_driver;

oxo_engine *oxo_engine_new(const oxe_model_desc *d, uint64_t seed, int64_t n_ctx);
// with n_slots recurrent slots (verify lanes; 2 by default, 4 for MTP depth 3)
oxo_engine *oxo_engine_new_lanes(const oxe_model_desc *d, uint64_t seed, int64_t n_ctx, int n_slots);
// with per-matrix ggml types types[layer * 64 + kind] (K-quant experts, shared experts and LM head;
// F32 ssm_beta / ssm_alpha; Q8_0 elsewhere); null for a type this model cannot take there
// restricted-vocabulary draft head (mtp.rs:166-197): MTP draft runs' argmax over `ids` only
int oxo_set_draft_vocab(oxo_engine *e, const uint32_t *ids, int n);
oxo_engine *oxo_engine_new_typed(const oxe_model_desc *d, uint64_t seed, int64_t n_ctx, int n_slots, const int32_t *types);
void oxo_engine_free(oxo_engine *e);
void oxo_engine_reset(oxo_engine *e);
int oxo_verify(oxo_engine *e, const uint32_t *toks, int n, uint32_t *out);      // engine.rs:2002-2025
int oxo_commit(oxo_engine *e, int m);                                          // engine.rs:2030-2039
uint32_t oxo_step(oxo_engine *e, uint32_t tok);                                // engine.rs:1991-1997
uint32_t oxo_mtp_run(oxo_engine *e, const uint32_t *toks, int n, int64_t pos0, const float *hs, int head_last); // engine.rs:2044-2071
void oxo_mtp_seed(oxo_engine *e, const uint32_t *toks, int n, int64_t pos0, const float *hs); // engine.rs:2077-2091
int64_t oxo_pos(const oxo_engine *e);
int oxo_cur_slot(const oxo_engine *e);
int oxo_tie_count(const oxo_engine *e);
const float *oxo_hidden(const oxo_engine *e, int lane);
const float *oxo_logits(const oxo_engine *e, int lane);
int64_t oxo_n_ctx(const oxo_engine *e);
void oxo_set_keep_logits(oxo_engine *e, int on);
double oxo_gen_seconds(const oxo_engine *e);  // time spent generating synthetic experts
int oxo_pin_team(int on);  // pin (1) / unpin (0) the OpenMP team, one thread per CPU of the caller's mask
const uint16_t *oxo_kcache(const oxo_engine *e);
const uint16_t *oxo_vcache(const oxo_engine *e);
float *oxo_conv_state(oxo_engine *e);
float *oxo_ssm_state(oxo_engine *e);
uint16_t *oxo_kcache_mut(oxo_engine *e);
uint16_t *oxo_vcache_mut(oxo_engine *e);
void oxo_set_pos(oxo_engine *e, int64_t pos);
void oxo_mixer(oxo_engine *e, int l, int nl, int64_t pos0, const float *x, float *x1);
void oxo_moe(oxo_engine *e, int l, int nl, const float *x1, float *x2);
void oxo_engine_set_router(oxo_engine *e, int l, int row0, int nrows, const float *src);
void oxo_mtp_entry(oxo_engine *e, const uint32_t *toks, int nl, const float *hs, float *x);

void oxo_synth_q8(uint64_t seed, int layer, int kind, int64_t expert, int64_t rows, int64_t k, int8_t *q, uint16_t *d);
void oxo_synth_f32(uint64_t seed, int layer, int kind, int64_t n, float *out);
void oxo_synth_normal(uint64_t seed, uint64_t uid, int64_t n, float mu, float sigma, float *out);

oxo_driver *oxo_driver_new(oxo_engine *e, int depth);                          // mtp.rs:348-362
void oxo_driver_free(oxo_driver *d);
void oxo_driver_import(oxo_driver *d, int64_t q, const float *hl);
int oxo_engine_read_state(oxo_engine *e, const uint8_t *buf, int64_t nbytes, int64_t n_pos);
uint32_t oxo_driver_prefill(oxo_driver *d, const uint32_t *toks, int n);      // mtp.rs:450-463
int oxo_driver_step(oxo_driver *d, uint32_t x, uint32_t *out, int64_t override_d1); // mtp.rs:522-592
// the same with force[i] >= 0 replacing draft i (i < nforce) after the chain (draft_override, mtp.rs:554-558)
int oxo_driver_step_force(oxo_driver *d, uint32_t x, uint32_t *out, const int64_t *force, int nforce);
uint32_t oxo_driver_step_plain(oxo_driver *d, uint32_t x);                           // mtp.rs:504-515
int oxo_driver_rewind(oxo_driver *d, int m);                                        // mtp.rs:596-608
void oxo_driver_stats(const oxo_driver *d, int64_t *st);
#ifdef __cplusplus
}
#endif
