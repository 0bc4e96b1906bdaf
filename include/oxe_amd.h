/* oxe_amd.h - C ABI of the MI355X (gfx950) MTP depth-1 decode step.
 *
 * Drop-in boundary for the hot path of n0rpan/snapdragon-engine's `oxe` engine. The reference's
 * Rust host (crates/model, crates/sched, crates/oxe-cli) calls its CPU kernels through the
 * extern "C" block of crates/kernels-sys/src/lib.rs:36-333; this header is the device counterpart
 * a Rust (or any C-ABI) host links instead. Plain C: device pointers, sizes, a stream handle
 * (hipStream_t passed as void*), int status codes. No allocation inside kernel-level calls.
 *
 * Status codes: 0 ok, -1 bad shape/argument (nothing written, like the reference's
 * oxe_repack_q8_0_4x8 returning -1), -2 HIP launch/runtime error, -3 out of device memory,
 * -4 device-side stop (a device-driven step that does not fit the context), -5 a fused run aborted
 * (one of its exchange polls timed out; oxe_last_error() names the word): the run commits nothing,
 * the engine keeps the state before it, and the call may be repeated.
 *
 * Every declaration names the reference interface it replaces (file:line in the reference tree).
 */
#ifndef OXE_AMD_H
#define OXE_AMD_H
#include <stdint.h>
#include "oxe_model.h"

#ifdef __cplusplus
extern "C" {
#endif

#define OXE_API

typedef struct oxe_engine oxe_engine;

/* ---- kernel level (device pointers, async on `stream`) -------------------------------------- */

/* Q8_0 activation quantizer: nrows rows of k floats -> int8 codes [nrows][k] + fp16 scales
 * [nrows][k/32]. Replaces quantize_row_q8_0 (crates/kernels-sys/src/lib.rs:62; NEON body
 * vendor/ggml-subset/generated/quants_subset.c:6-42). */
OXE_API int oxe_hip_quantize_row_q8_0(const float *x, int64_t k, int64_t nrows, int8_t *q, uint16_t *d, void *stream);

/* Q8_0 lane GEMV: y[l][r] = W[r] . x[l] for nl = 1..4 lanes in one weight pass, each lane bit for
 * bit the per-lane GEMV; weights as int8 codes [nr][k] + fp16 scales [nr][k/32] (this build's
 * layout; see oxe_hip_repack_q8_0), lanes as produced by oxe_hip_quantize_row_q8_0; k any multiple
 * of 32 (tuned kernels for 512, 2048 and 4096, a one-wave-per-row kernel otherwise, up to 131072 /
 * nl ... 32768 at 4 lanes). isum (optional, may be NULL): the exact int32 block dots [nl][nr][k/32].
 * Replaces oxe_vl_gemv type 80 (lib.rs:113; csrc/oxe_vl.inc:78-107) with its return convention:
 * 1 = done, 0 = not handled with nothing written (nl outside 1..4, nr <= 0, k not a positive
 * multiple of 32 or past the limit), -2 launch error; and ggml_gemv_q8_0_4x8_q8_0 (lib.rs:75). */
OXE_API int oxe_hip_gemv_q8_0(int64_t k, int64_t nr, int nl, const int8_t *wq, const uint16_t *wd, const int8_t *xq,
                              const uint16_t *xd, float *y, int32_t *isum, void *stream);

/* Routing of n_rows rows of 256 router logits (f32): probabilities = softmax, the top 8 expert ids
 * (ids [n_rows][8]) in the reference's order, including libstdc++ std::sort's order of tied
 * probabilities, and their weights renormalised by the clamped sum (w [n_rows][8]). *tie_count
 * (device memory) is incremented once per row that took the sort path. Replaces Engine::route
 * (crates/model/src/engine.rs:3414-3429) over oxe_soft_max_f32 and oxe_argsort_top_k_f32
 * (crates/kernels-sys/src/lib.rs:129-130; oxe_ops.cpp:101-165). */
OXE_API int oxe_hip_route_f32(const float *logits, int64_t n_rows, int32_t *ids, float *w, uint32_t *tie_count,
                              void *stream);

/* Q8_0 GEMM for prefill: y[t][r] (row stride ldy >= nr) = W[r] . x[t] for nt token rows of
 * activations (oxe_hip_quantize_row_q8_0 output) against nr weight rows (layout as in
 * oxe_hip_gemv_q8_0); k a multiple of 128. Each output equals the GEMV's bit for bit (block dots
 * and scale products on the matrix cores, the fp32 chain over blocks in order). Replaces
 * ggml_gemm_q8_0_4x8_q8_0 (crates/kernels-sys/src/lib.rs:95;
 * vendor/ggml-subset/generated/repack_subset.cpp:3804-3954). wq, wd, xq and xd must be 16-byte
 * aligned, and nr * k and nt * k below 2^32 (the kernel addresses codes with 32-bit offsets).
 * Returns 0, -1 (bad shape, alignment or null pointer) or -2 (launch error). */
OXE_API int oxe_hip_gemm_q8_0(int64_t k, int64_t nr, int64_t nt, const int8_t *wq, const uint16_t *wd, const int8_t *xq,
                              const uint16_t *xd, float *y, int64_t ldy, void *stream);

/* Q8_0 weight repack: nrows rows of ggml Q8_0 blocks (34 bytes: fp16 d, 32 int8 codes; device memory)
 * into this build's layout, int8 codes [nrows][k] + fp16 scales [nrows][k/32], which every GEMV /
 * GEMM entry point here reads. Replaces oxe_repack_q8_0_4x8 (crates/kernels-sys/src/lib.rs:59, the
 * reference's 4-row interleave for its NEON GEMV); -1 on a bad shape (k not a multiple of 32),
 * nothing written. */
OXE_API int oxe_hip_repack_q8_0(const void *src, int64_t nrows, int64_t k, int8_t *q, uint16_t *d, void *stream);

/* K-quant activation quantizer: nrows rows of k floats (k a multiple of 256; x 16-byte aligned) ->
 * ggml block_q8_K blocks (float d, int8 qs[256], int16 bsums[16]; 292 bytes each) [nrows][k/256].
 * Replaces quantize_row_q8_K (on ARM the reference's is quantize_row_q8_K_ref,
 * vendor/ggml-subset/generated/quants_base.c:14-48, ggml_subset.h:18-19); an all-zero block gets
 * zero sums (the reference leaves them unwritten). 0, -1 bad shape, -2 launch error. */
OXE_API int oxe_hip_quantize_row_q8_K(const float *x, int64_t k, int64_t nrows, void *y, void *stream);

/* K-quant lane GEMV: s[l][r] = W[r] . y[l] for nl = 1..4 lanes, bit for bit the reference's
 * per-lane result. type 3 Q3_K, 4 Q4_K, 5 Q5_K, 6 Q6_K; w = nr rows of k/256 ggml blocks of the type
 * (the GGUF file's bytes, 4-byte aligned; no repack), y = nl lanes of k/256 block_q8_K (as
 * oxe_hip_quantize_row_q8_K writes them: the kernels use their bsums), s = float [nl][nr]. Replaces
 * oxe_vl_gemv (crates/kernels-sys/src/lib.rs:113; csrc/oxe_vl.inc:78-107 and oxe_vl_q{3,4,5,6}k.inc),
 * whose weights are its 8-row interleaved repack, and its per-lane fallback ggml_gemv_q*_K_8x8_q8_K.
 * Returns as the reference: 1 = done, 0 = not handled, nothing written (another type, nl outside
 * 1..4, k not a multiple of 256 or above 8192, Q3_K / Q6_K with an odd number of blocks per row);
 * -2 launch error. */
OXE_API int oxe_hip_vl_gemv(int type, int64_t k, int64_t nr, int nl, const void *w, const void *y, float *s,
                            void *stream);

/* Parity hook (no counterpart in the reference): y[i] = f(x) for the float x with bits
 * start + i*stride, i < n, on the device; f: 0 expf and 1 log1pf (the C library functions the
 * reference calls, oxe_ops.cpp:80-89), 2 ggml_v_expf (vec.h:1154-1175), 3 the sigmoid and
 * 4 the softplus of oxe_ops.cpp:80-89, 5 ggml_v_silu (vec.h:1178-1185). */
OXE_API int oxe_hip_eval_unary(int fn, uint32_t start, int64_t n, int64_t stride, float *y, void *stream);

/* ---- engine level (crates/model/src/engine.rs Engine; one engine per stream) -------------- */

/* Last error message of a failed call on this host thread (no exceptions cross the C ABI). */
OXE_API const char *oxe_last_error(void);

/* Create an engine for `desc` (the kernels are specialised for the 35B-A3B per-layer shape; layer
 * count and vocabulary are free) with a context of n_ctx positions (rounded up to 256), all state in
 * device memory. Replaces Engine::with_options (crates/model/src/engine.rs:869-1000) with
 * verify_lanes 2 and an MTP head. */
OXE_API int oxe_engine_create(const oxe_model_desc *desc, uint64_t seed, int n_ctx, oxe_engine **out);
/* oxe_engine_create on the caller's stream (hipStream_t as void*, the null stream included; the
 * device-driven steps' graph capture needs a created stream): every launch and copy of the engine,
 * weight synthesis and loading included, goes to it, and destroy leaves it to the caller. The
 * reference's engine runs on the caller's thread (Engine::with_options, engine.rs:869); this is its
 * device counterpart. */
OXE_API int oxe_engine_create_on(const oxe_model_desc *desc, uint64_t seed, int n_ctx, void *stream,
                                 oxe_engine **out);
/* An engine whose matrices take other types than Q8_0, as a model file's do, without the file:
 * types[layer * 64 + kind] (layer 63 = the global tensors; kinds of include/oxe_model.h) holds a ggml
 * type id per matrix, 8 where it is Q8_0: K-quants (11..14) for the experts, shared expert, mixer
 * and output projections, token embedding and LM head, F32 (0) or K-quants for ssm_beta /
 * ssm_alpha, in the combinations oxe_engine_create_from_gguf takes (-1 naming any other).
 * oxe_engine_synth_weights then fills each matrix in its type (the oracle's synthetic K-quant
 * blocks). The reference builds such an engine only from a file (WeightStore::load, weights.rs:556);
 * this is that engine with synthetic weights, for tests and benchmarks of the files' types. */
OXE_API int oxe_engine_create_typed(const oxe_model_desc *desc, uint64_t seed, int n_ctx, const int32_t *types,
                                    oxe_engine **out);
OXE_API void oxe_engine_destroy(oxe_engine *e);
/* Fill every weight with the synthetic model of include/oxe_model.h (the benchmark's model), each
 * matrix of a typed engine in its type. */
OXE_API int oxe_engine_synth_weights(oxe_engine *e);

/* Run n (1..2) tokens at positions pos..pos+n-1 as one batch-invariant run; argmax per lane.
 * Replaces Engine::verify (engine.rs:2002-2025). The position moves only on commit. */
OXE_API int oxe_engine_verify(oxe_engine *e, const uint32_t *toks, int n, uint32_t *argmax_out);
/* Keep the first m tokens of the last verify (engine.rs:2030-2039): position pos0+m, recurrent
 * state of lane m-1, V^T of rejected positions zeroed. */
OXE_API int oxe_engine_commit(oxe_engine *e, int m);
/* verify + commit(1) (engine.rs:1991-1997). */
OXE_API int oxe_engine_step(oxe_engine *e, uint32_t tok, uint32_t *argmax_out);
/* MTP head over toks at pos0.. with input hidden states hs [n][n_embd] (host memory); argmax of the
 * last lane when head_last (engine.rs:2044-2071). */
OXE_API int oxe_engine_mtp_run(oxe_engine *e, const uint32_t *toks, int n, int pos0, const float *hs, int head_last,
                               uint32_t *argmax_out);
/* MTP KV seeding of the pairs (toks[i], hs[i]) at pos0.. (engine.rs:2077-2091). */
OXE_API int oxe_engine_mtp_seed(oxe_engine *e, const uint32_t *toks, int n, int pos0, const float *hs);
OXE_API int oxe_engine_pos(const oxe_engine *e);
OXE_API int oxe_engine_n_ctx(const oxe_engine *e);
/* h_nextn of lane `lane` of the last run (Engine::hidden, engine.rs:1941-1945), host copy. */
OXE_API int oxe_engine_hidden(oxe_engine *e, int lane, float *out);
/* Logits of lane `lane` of the last verify (Engine::logits_lane, engine.rs:1934-1937), host copy. */
OXE_API int oxe_engine_logits(oxe_engine *e, int lane, float *out);
/* Overwrite router rows [row0, row0 + nrows) of layer `layer` (n_layer: the MTP block) with host f32
 * rows of n_embd values (a test hook for exact routing ties; no counterpart in the reference). */
OXE_API int oxe_engine_set_router(oxe_engine *e, int layer, int row0, int nrows, const float *host);
/* Diagnostic counters (64: routings that took the reference's std::sort path for tied probabilities). */
OXE_API int oxe_engine_counter(oxe_engine *e, int which, uint32_t *out);
/* State copy for parity checks / hand-off (see engine.hip for the regions). */
OXE_API int oxe_engine_state_copy(oxe_engine *e, int which, int dir, int64_t offset, void *host, int64_t nbytes);
OXE_API int oxe_engine_set_pos(oxe_engine *e, int pos);
/* Sequence state in the reference's byte order (prefix store / prefill hand-off): Engine::state_bytes
 * (engine.rs:1570-1576); Engine::write_state (1682-1722): per attention layer (the MTP layer's
 * included) the f16 K rows of positions < pos per KV head, then the f16 V^T rows (kv head *
 * head_dim + dim) of those positions, then the current slot's conv state [n_rec][8192][3] and
 * delta-net S [n_rec][32][128][128] (s[j*128+i] = S[i][j]), f32; write_state needs cap >=
 * state_bytes (-1 otherwise). Engine::read_state (1819-1871): the same bytes for n_pos positions
 * (nbytes must match exactly); V^T of positions [n_pos, pos) zeroed, position = n_pos. */
OXE_API int64_t oxe_engine_state_bytes(const oxe_engine *e);
OXE_API int oxe_engine_write_state(oxe_engine *e, void *host, int64_t cap);
OXE_API int oxe_engine_read_state(oxe_engine *e, const void *host, int64_t nbytes, int n_pos);
/* KV rows of positions [a, b) in the write_state order (the prefix store's row segments):
 * Engine::kv_row_bytes (engine.rs:1812-1814) = bytes per position; Engine::write_kv_rows
 * (1727-1767), b <= pos, cap >= (b - a) * kv_row_bytes; Engine::read_kv_rows (1769-1810), b <=
 * n_ctx, nbytes == (b - a) * kv_row_bytes, the position does not change. */
OXE_API int64_t oxe_engine_kv_row_bytes(const oxe_engine *e);
OXE_API int oxe_engine_write_kv_rows(oxe_engine *e, int a, int b, void *host, int64_t cap);
OXE_API int oxe_engine_read_kv_rows(oxe_engine *e, int a, int b, const void *host, int64_t nbytes);
OXE_API int64_t oxe_engine_device_bytes(const oxe_engine *e);
/* Run mode (no counterpart in the reference, whose runs are thread-team phases): 1 = every run
 * as one persistent launch of the fused run kernel (the default where the device has exactly 256
 * CUs), 0 = one launch per phase. Both compute the same bits. -1 when 1 is not available. */
OXE_API int oxe_engine_set_fused(oxe_engine *e, int on);
OXE_API int oxe_engine_fused(const oxe_engine *e);
/* Phase trace of the fused run kernel (diagnostic, no counterpart in the reference, whose Trace at
 * crates/model/src/engine.rs:324-340 records tensors, not time): when on, every run records per workgroup and
 * phase (phase id, start, barrier released, end) in device wall-clock ticks (100 MHz);
 * read_trace copies the last run's records ([grid][2048][4] u64) and returns their count. */
OXE_API int oxe_engine_set_trace(oxe_engine *e, int on);
OXE_API int64_t oxe_engine_read_trace(oxe_engine *e, unsigned long long *host, int64_t cap);

/* Batched prefill of n prompt tokens at pos..pos+n-1 (all layers over the whole batch: int8
 * matrix-core GEMMs for every weight matrix, token-parallel norms / routing / attention, the conv
 * and delta-net recurrences token by token). KV cache, recurrent state, logits and hidden state of
 * the last token are those of n decode steps, bit for bit; *next = argmax of the last token.
 * hidden (optional host [n][n_embd]): every position's h_nextn. Replaces Engine::prefill_ext
 * (crates/model/src/engine/prefill.rs:763). */
OXE_API int oxe_engine_prefill(oxe_engine *e, const uint32_t *toks, int n, uint32_t *next, float *hidden);
/* oxe_engine_prefill with HIP events around every launch of one kernel kind (12 every matrix-core
 * GEMM, 13 the grouped expert GEMMs, 14 attention, 15 the delta rule): *total_us = their summed
 * duration, *n_launch = launches timed (diagnostic for the prefill roofline; no counterpart in the
 * reference). */
OXE_API int oxe_engine_prefill_probe(oxe_engine *e, const uint32_t *toks, int n, int kind, float *total_us,
                                     int *n_launch);

/* ---- GGUF model files (crates/gguf/src/lib.rs, crates/model/src/desc.rs, weights.rs) --------- */

typedef struct oxe_gguf oxe_gguf;

/* Memory-map and parse a GGUF v2/v3 file: header, metadata, tensor table, data alignment
 * (general.alignment, default 32, a power of two), every tensor inside the file. Replaces
 * Gguf::open (gguf/src/lib.rs:345-355) with parse_header (268-316) and check_bounds (320-330):
 * the same checks and the same error cases (bad magic, version, counts the file cannot hold, more
 * than 4 dimensions, dimensions above 2^63, unknown types, element counts not a multiple of the
 * type's block, overflowing sizes, data beyond the end of the file). -1 with oxe_last_error(). */
OXE_API int oxe_gguf_open(const char *path, oxe_gguf **out);
/* parse_header of an in-memory file image (no bounds check; file_bytes = len) */
OXE_API int oxe_gguf_parse(const void *buf, uint64_t len, oxe_gguf **out);
/* check_bounds against a file of file_bytes bytes */
OXE_API int oxe_gguf_check_bounds(const oxe_gguf *g, uint64_t file_bytes);
OXE_API void oxe_gguf_close(oxe_gguf *g);
OXE_API int oxe_gguf_info(const oxe_gguf *g, uint32_t *version, uint64_t *n_tensors, uint64_t *n_meta,
                          uint64_t *data_offset, uint64_t *header_bytes, uint64_t *file_bytes);
/* tensor i: name (valid until close), ggml type id, dims, shape (unused dims 1), offset in the data
 * section, bytes (TensorInfo, lib.rs:136-166) */
OXE_API int oxe_gguf_tensor(const oxe_gguf *g, uint64_t i, const char **name, uint32_t *type, uint32_t *n_dims,
                            uint64_t *shape4, uint64_t *offset, uint64_t *bytes);
/* metadata entry i: key and GGUF value type; typed lookups by key (first match, Header::get), with
 * Value::as_u64 / as_f64 semantics (lib.rs:113-134); arrays: item type, length, and whether the
 * items were kept (arrays longer than 4096 items are counted only) */
OXE_API int oxe_gguf_meta(const oxe_gguf *g, uint64_t i, const char **key, uint32_t *type);
OXE_API int oxe_gguf_meta_u64(const oxe_gguf *g, const char *key, uint64_t *out);
OXE_API int oxe_gguf_meta_f64(const oxe_gguf *g, const char *key, double *out);
OXE_API int oxe_gguf_meta_str(const oxe_gguf *g, const char *key, const char **out);
OXE_API int oxe_gguf_meta_array(const oxe_gguf *g, const char *key, uint32_t *item_type, uint64_t *len, int *kept);
OXE_API int oxe_gguf_meta_array_f64(const oxe_gguf *g, const char *key, uint64_t i, double *out);
/* ModelDesc::from_header + check (desc.rs:69-178): qwen35moe only, layer kinds from the tensors
 * (ssm_a / attn_q) checked against full_attention_interval, shape cross-checks. */
OXE_API int oxe_gguf_model_desc(const oxe_gguf *g, oxe_model_desc *out);
/* Every weight of the engine from the file (WeightStore::load, weights.rs:556-700): Q8_0 matmul
 * weights split on the device into this build's codes + scales layout (the reference repacks into
 * 4-row interleaved blocks, oxe_repack_q8_0_4x8, lib.rs:59), F32 norms, routers and state
 * parameters copied, BF16 ones widened to f32 (as the reference converts BF16 small tensors,
 * crates/model/src/mtp.rs:109-128). K-quant (Q3_K..Q6_K) expert, shared-expert and output matrices
 * and F32 ssm_beta / ssm_alpha (a Qwen3.6 file's types; the reference's mv dispatches every type,
 * engine.rs:2270-2343) are copied in the file's blocks into an engine created with those types,
 * which oxe_engine_create_from_gguf reads from the file; into an engine created for Q8_0 they are
 * refused by name (-1), as is any other tensor type. An engine with such matrices runs its runs per
 * phase (oxe_engine_set_fused(e, 1) returns -1: the fused run kernel reads Q8_0 matrices only) and
 * its batched prefill as decode runs of two positions (the same state and h_nextn). */
OXE_API int oxe_engine_load_gguf(oxe_engine *e, const oxe_gguf *g);
/* oxe_engine_load_gguf without any device allocation: no counterpart in the reference; for callers
 * that cannot allocate device memory (code under HIP graph capture, serving loops, harnesses that
 * forbid hipMalloc). Uploads are staged through a 16 MiB device array of the library (one per GPU,
 * held until the process ends) instead of a 256 MiB buffer allocated per call; a tensor that must be
 * staged whole above 16 MiB (one expert's matrix, an interleaved gate / up matrix) is refused by
 * name (-1). The engine's device must be current. Calls on one GPU share the array: a per-device
 * lock makes overlapping calls (other threads, other streams) run one after another. */
OXE_API int oxe_engine_load_gguf_noalloc(oxe_engine *e, const oxe_gguf *g);
/* open + model_desc + engine_create with the file's matrix types + load_gguf */
OXE_API int oxe_engine_create_from_gguf(const char *path, int n_ctx, oxe_engine **out);

/* ---- MTP depth-1 speculative decoding (crates/model/src/mtp.rs MtpDriver, depth 1) --------- */

/* Append prompt tokens through 2-token verify runs and the MTP catch-up (MtpDriver::prefill,
 * mtp.rs:450-463); *next = argmax after the last token. */
OXE_API int oxe_mtp_prefill(oxe_engine *e, const uint32_t *toks, int n, uint32_t *next);
/* Append a prompt with the batched prefill, then seed the MTP KV from every position's h_nextn in
 * one batched pass (MtpDriver::prefill_batched, mtp.rs:468-500; one token: step_plain). Same
 * engine state, MTP KV and *next as oxe_mtp_prefill. */
OXE_API int oxe_mtp_prefill_batched(oxe_engine *e, const uint32_t *toks, int n, uint32_t *next);
/* One speculative step from token x (MtpDriver::step, mtp.rs:522-592), host-driven: out[0..n_out)
 * = the greedy tokens that follow (accepted drafts + bonus; room for depth + 1). override_d1 >= 0
 * replaces the first draft (the reference's draft_override test hook, mtp.rs:328-330). */
OXE_API int oxe_mtp_step(oxe_engine *e, uint32_t x, uint32_t *out, int *n_out, int64_t override_d1);
/* One plain target step from x that keeps the MTP catch-up in sync (MtpDriver::step_plain,
 * mtp.rs:504-515); *out = argmax after x. */
OXE_API int oxe_mtp_step_plain(oxe_engine *e, uint32_t x, uint32_t *out);
/* Drafts per host-driven step, 1..3 (MtpDriver.depth, mtp.rs:314-360; the reference's MAX_LANES
 * verify of depth + 1 lanes runs here as pieces of at most 2 lanes, each committed before the next,
 * stopping at the first rejected draft: the same committed state, tokens, hidden rows and logits).
 * The device-driven step (oxe_mtp_device_*) runs depth 1 or 2 (the depth set when begin is called)
 * and refuses depth 3. */
OXE_API int oxe_mtp_set_depth(oxe_engine *e, int depth);
/* oxe_mtp_step with force[i] >= 0 (i < nforce) replacing draft i + 1 after the draft chain is formed
 * (the reference's draft_override hook, mtp.rs:328-330, 554-558); out has room for depth + 1 tokens */
OXE_API int oxe_mtp_step_force(oxe_engine *e, uint32_t x, uint32_t *out, int *n_out, const int64_t *force, int nforce);
/* Keep only the first m (1..committed) tokens of the last host-driven step (MtpDriver::rewind,
 * mtp.rs:596-608; the server's spec_rewind, crates/server/src/engine.rs:100-104). -1 without a
 * step to rewind. */
OXE_API int oxe_mtp_rewind(oxe_engine *e, int m);
/* Device-driven steps: begin hands the driver state to the GPU; each of the k steps then runs
 * draft (the pending catch-up pair, if any, as an extra lane) -> 2-lane verify -> greedy
 * accept/commit on the GPU (one HIP graph per step, no host round-trip); end synchronises and
 * returns the emitted tokens and the next x. At depth 2 a step
 * runs two drafts and verifies x, d1 and then d2 in pieces of at most two lanes, the second piece
 * only when d1 was accepted and d2 matches (mtp.rs:522-592). A step that does not fit the context
 * (depth 1: 2 positions, depth 2: 3) stops the steps: end returns -4, and the caller continues with
 * host-driven steps (which shorten the draft chain to the room left, as the reference does). A run
 * that aborted stops the steps as well: end returns -5 after handing back the state of the last step
 * that ran (tokens, position, pending pairs), so decoding continues from there. */
OXE_API int oxe_mtp_device_begin(oxe_engine *e, uint32_t x, int out_cap);
OXE_API int oxe_mtp_device_steps(oxe_engine *e, int k, int use_graph);
OXE_API int oxe_mtp_device_end(oxe_engine *e, uint32_t *out_tok, int cap, int *n_out, uint32_t *next_x);
/* Forced drafts for the device-driven steps (test hook): force_d1[i * depth + j] >= 0 replaces draft
 * j + 1 of step i. */
OXE_API int oxe_mtp_set_force(oxe_engine *e, const int32_t *force_d1, int n);
/* Restricted-vocabulary draft head (MtpWeights::set_draft_vocab, crates/model/src/mtp.rs:166-197,
 * WP-D3b): the output matrix's rows of `ids` (ids >= n_vocab dropped, sorted, duplicates removed,
 * padded by repeating the last id) become every MTP draft run's LM head, its argmax mapped back to
 * token ids; verify runs keep the whole head, so the output is unchanged and only the drafts (and
 * acceptance) can differ. n = 0 restores the whole head. Returns the draft head's rows (0 after a
 * restore), -1 (no id below n_vocab: "empty draft vocabulary"), -2 or -3. */
OXE_API int oxe_mtp_set_draft_vocab(oxe_engine *e, const uint32_t *ids, int n);
/* k eager device-driven steps with HIP events around each launch of one kernel kind (0 LM head,
 * 1 experts gate/up, 2 down, 3 projections, 4 mixer out, 5 delta-net, 6 router, 7 scores, 8 pv,
 * 9 MTP entry; in the fused run mode 10 the verify run, 11 the draft run, each one launch): mean
 * kernel duration in microseconds (roofline measurement). */
OXE_API int oxe_mtp_device_probe(oxe_engine *e, int k, int kind, float *avg_us, int *n);
/* oxe_engine_verify with the same HIP-event timing of one kernel kind (*count launches timed):
 * the bench's per-config lines. No counterpart in the reference (a measurement hook). */
OXE_API int oxe_engine_verify_probe(oxe_engine *e, const uint32_t *toks, int n, int kind, uint32_t *argmax_out,
                                    float *avg_us, int *count);
/* st[0] steps, st[1] accepted drafts, st[2] drafted tokens (MtpStats, mtp.rs:273-290) */
OXE_API int oxe_mtp_stats(const oxe_engine *e, int64_t *st);
OXE_API int oxe_engine_sync(oxe_engine *e);
/* the engine's HIP stream (hipStream_t) */
OXE_API void *oxe_engine_stream(oxe_engine *e);

/* ---- the server's engine (crates/server/src/engine.rs:28-190 trait Engine, implemented for oxe
 * by crates/server/src/oxe_engine.rs:317-634 OxeEngine) ---------------------------------------
 * An oxe_srv borrows an engine (destroy the oxe_srv first) and, with mtp != 0, drives it through
 * the MTP depth-1 driver; then OXE_MTP_DRAFT_VOCAB=<ranking file> [OXE_MTP_DRAFT_K=<k>] restricts
 * the engine's draft head as the reference's adapter does (oxe_engine.rs:215-222; see
 * oxe_mtp_set_draft_vocab). Errors: -1 with oxe_last_error() (the reference's EngineError text),
 * -2 HIP error; 1 = "not supported here" (the trait's Ok(None)). */
typedef struct oxe_srv oxe_srv;
typedef struct oxe_snapshot oxe_snapshot;

OXE_API int oxe_srv_create(oxe_engine *engine, int mtp, oxe_srv **out);
OXE_API void oxe_srv_destroy(oxe_srv *s);
OXE_API oxe_engine *oxe_srv_engine(oxe_srv *s);
/* n_ctx / n_vocab / n_past (Engine::n_ctx, n_vocab, n_past) */
OXE_API int oxe_srv_n_ctx(const oxe_srv *s);
OXE_API int oxe_srv_n_vocab(const oxe_srv *s);
OXE_API int oxe_srv_n_past(const oxe_srv *s);
/* reset (OxeEngine::reset, oxe_engine.rs:336-341; Engine::reset, engine.rs:1491-1509): empty
 * sequence, recurrent state and V^T zeroed, MTP driver re-synced with h_prev = 0 */
OXE_API int oxe_srv_reset(oxe_srv *s);
/* prefill (oxe_engine.rs:342-374): append n >= 1 tokens ("empty prefill", "context full", "token
 * T out of vocab"); with MTP the batched prefill seeds the MTP KV (one token: step_plain); logits
 * (optional, host [n_vocab]) = the last token's row. logits NULL = prefill_quiet (375-390). */
OXE_API int oxe_srv_prefill(oxe_srv *s, const uint32_t *toks, int n, float *logits);
/* decode (the trait's default: prefill of one token) */
OXE_API int oxe_srv_decode(oxe_srv *s, uint32_t tok, float *logits);
/* decode_argmax (oxe_engine.rs:544-562): one step (MTP: step_plain), *out = the first maximum of
 * the logits row */
OXE_API int oxe_srv_decode_argmax(oxe_srv *s, uint32_t tok, uint32_t *out);
/* decode_spec_argmax (oxe_engine.rs:563-578): one MTP step from tok; extra[0..n_extra) = accepted
 * drafts (in the state), argmax[0..n_argmax) = the argmax of every committed row (the last is the
 * bonus token, not yet in the state); both arrays sized spec_max_depth() + 1 (4). 1 without MTP. */
OXE_API int oxe_srv_decode_spec_argmax(oxe_srv *s, uint32_t tok, uint32_t *extra, int *n_extra, uint32_t *argmax,
                                       int *n_argmax);
/* decode_spec (oxe_engine.rs:530-543): as decode_spec_argmax with the committed rows' logits in
 * rows = host [rows_cap][n_vocab]; rows [0, n_extra] are written. A step commits up to depth + 1
 * rows, so rows_cap must be at least the current depth + 1 (spec_max_depth() + 1 covers every depth):
 * a smaller buffer is refused (-1) before any work. extra holds up to depth values. */
OXE_API int oxe_srv_decode_spec(oxe_srv *s, uint32_t tok, uint32_t *extra, int *n_extra, float *rows, int rows_cap);
/* spec_rewind (oxe_engine.rs:579-592): keep the first `keep` tokens the last lookup verify or MTP
 * step committed (MtpDriver::rewind, mtp.rs:596-608) */
OXE_API int oxe_srv_spec_rewind(oxe_srv *s, int keep);
/* decode_verify (oxe_engine.rs:593-619): caller drafts on the plain engine (1 with MTP on, no
 * drafts or no room): verify [tok, drafts[0..k)], k = min(n_drafts, verify lanes - 1 = 1, room), accept the prefix
 * equal to greedy decoding, commit it; accepted[0..n_acc), argmax[0..n_acc] as decode_spec_argmax */
OXE_API int oxe_srv_decode_verify(oxe_srv *s, uint32_t tok, const uint32_t *drafts, int n_drafts, uint32_t *accepted,
                                  int *n_acc, uint32_t *argmax, int *n_argmax);
/* spec_set_depth (oxe_engine.rs:623-627): drafts per step, clamped to 1..spec_max_depth (3 with MTP);
 * spec_max_depth / spec_counters (oxe_engine.rs:620-633): MTP (drafted, accepted) or the lookup
 * counts of decode_verify */
OXE_API int oxe_srv_spec_max_depth(const oxe_srv *s);
OXE_API int oxe_srv_spec_set_depth(oxe_srv *s, int depth);
OXE_API int oxe_srv_spec_counters(const oxe_srv *s, uint64_t *drafted, uint64_t *accepted);
/* snapshot / snapshot_reuse (oxe_engine.rs:391-397; Engine::save_recurrent, engine.rs:1525-1531):
 * the current slot's conv + delta-net state (a device copy) and the position, plus the MTP
 * driver's state; *inout NULL allocates a snapshot, else it is reused. restore (oxe_engine.rs:
 * 402-409; Engine::restore_recurrent, engine.rs:1643-1659): refused for a snapshot ahead of the
 * position; V^T of the positions beyond it back to +0; the MTP driver imports the snapshot's
 * state when it fits (MtpDriver::import_state, mtp.rs:391-401), else re-syncs (363-382). */
OXE_API int oxe_srv_snapshot(oxe_srv *s, oxe_snapshot **inout);
OXE_API int oxe_srv_restore(oxe_srv *s, const oxe_snapshot *snap);
/* snapshot_bytes (oxe_engine.rs:410-412), the snapshot's position, free */
OXE_API int64_t oxe_snapshot_bytes(const oxe_snapshot *snap);
OXE_API int oxe_snapshot_pos(const oxe_snapshot *snap);
OXE_API void oxe_snapshot_free(oxe_snapshot *snap);
/* state_size_hint (oxe_engine.rs:398-401); save_state / load_state (oxe_engine.rs:492-529):
 * Engine::write_state bytes, then with MTP u64 q, u64 n, n u32 catch-up tokens, their n h rows and
 * h_prev (f32); save_bytes = the exact size save_state writes; load_state checks the whole buffer
 * before it changes any state */
OXE_API int64_t oxe_srv_state_size_hint(const oxe_srv *s);
OXE_API int64_t oxe_srv_save_bytes(const oxe_srv *s);
OXE_API int oxe_srv_save_state(oxe_srv *s, void *buf, int64_t cap, int64_t *written);
OXE_API int oxe_srv_load_state(oxe_srv *s, const void *buf, int64_t nbytes, int n_pos);
/* snapshot files (snap_save / snap_save_live / snap_load, oxe_engine.rs:428-467):
 * RecurrentSnapshot::write_to (engine.rs:572-582) + tag byte (0 / 2) + MtpState::write
 * (oxe_engine.rs:108-119); snap_load needs the KV rows of positions < n_pos in place
 * (oxe_engine_read_kv_rows) and the file's position equal to n_pos */
OXE_API int64_t oxe_srv_snap_file_bytes(const oxe_srv *s, const oxe_snapshot *snap);
OXE_API int oxe_srv_snap_save(oxe_srv *s, const oxe_snapshot *snap, void *buf, int64_t cap, int64_t *written);
OXE_API int64_t oxe_srv_snap_live_bytes(const oxe_srv *s);
OXE_API int oxe_srv_snap_save_live(oxe_srv *s, void *buf, int64_t cap, int64_t *written);
OXE_API int oxe_srv_snap_load(oxe_srv *s, const void *buf, int64_t nbytes, int n_pos);
/* Engine::state_layout (engine.rs:1669-1677), f16 KV: "att=A kv_heads=H head_dim=D conv=C ssm=S
 * f16kv"; returns 0, or the bytes needed when cap is too small */
OXE_API int oxe_srv_state_layout(const oxe_srv *s, char *buf, int cap);

#ifdef __cplusplus
}
#endif
#endif /* OXE_AMD_H */
