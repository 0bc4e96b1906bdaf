// The fused run kernel: one persistent launch per engine run (verify of 1-2 lanes over every layer
// + the LM head; the MTP draft run; the MTP seeding run) instead of one launch per phase.
//
// Workgroups (one per CU, all resident) walk the run's phases in the same order as the reference's
// static plan (crates/model/src/plan.rs:171-261). Where the reference's thread team meets at a
// barrier between dependent phases (crates/sched/src/lib.rs:43-84), a workgroup here waits only for
// the tagged values it reads (FzXch). Each workgroup issues a phase's weight loads before it waits
// for the phase's inputs, so weight streaming overlaps the wait. Activations exchanged between
// workgroups inside the launch are written and read with device-scope (coherent) accesses; nothing
// relies on a cache flush.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "oxe_engine.h"
#include "oxe_model_kernels.h"

namespace oxe {

// per-layer weight table in device memory (the fused kernel indexes it by layer)
struct LayerDev {
    int32_t att, index;
    const float *attn_norm, *post_norm;
    Q8W proj, out;
    const float *conv, *ssm_a, *dt_bias, *ssm_norm;
    const float *q_norm, *k_norm;
    const float *router, *shexp_gate;
    Q8W shexp_gu, shexp_down, exp_gu, exp_down, eh_proj;
    const float *enorm, *hnorm, *head_norm;
};

enum FusedMode { FM_VERIFY = 0, FM_DRAFT = 1, FM_SEED = 2 };

// sync words (uint32): the launch's tag base at [288] (read by every workgroup at its start; the
// last workgroup to finish advances it by FZ_TAG_STRIDE), the finished-workgroup counter at [256],
// the sticky error word at [320]
constexpr int FZ_SYNC_WORDS = 384;
constexpr int FZ_W_DONE = 256, FZ_W_FLAG = 288, FZ_W_ERR = 320;
constexpr int FZ_W_HEADQ = 352;   // the LM head's tile-pair counter (cleared by the last workgroup out)
constexpr uint32_t FZ_TAG_STRIDE = 1024;   // > 8 phases x (n_layer + 2)

// Tagged exchange buffers of the fused kernel. Every 32-bit value one workgroup passes to another
// inside a launch travels as a 64-bit word, the value in the low half and the tag of the phase that
// wrote it in the high half, stored and loaded whole (device scope); a reader spins until the tag it
// expects appears, so no grid barrier separates the phases and no writer waits for its stores to
// complete. Tags are launch base + 1 + 8 k + phase (k: the run's layer index), unique across
// launches. Each buffer has two copies, by the parity of k: a write of layer k + 2 depends, through
// the all-to-all exchanges of layer k + 1 (every workgroup reads every workgroup's x and x1), on every
// read of layer k having been made.
struct FzXch {
    uint64_t *x;      // [2][NL][E]               the residual stream: layer inputs (x2 of the layer before)
    uint64_t *x1;     // [2][NL][E]               after the mixer
    uint64_t *p;      // [2][NL][DN_ROWS]         projection outputs
    uint64_t *g;      // [2][NL][MIX_W]           delta-rule outputs / gated attention outputs (f32)
    uint64_t *o;      // [2][NL][MIX_W / 4]       the delta-net mixer output, Q8_0 codes, 4 per word
    uint64_t *od;     // [2][NL][MIX_W / 32]      its fp16 scales
    uint64_t *lg;     // [2][NL][NEXP]            router logits
    uint64_t *sg;     // [2][NL]                  shared-expert gate (sigmoid)
    uint64_t *hsh;    // [2][NL][FFSH]            shared-expert h
    uint64_t *hq;     // [2][NL][MAX_UNION][FF/4] routed experts' h, Q8_0 codes, 4 per word
    uint64_t *hd;     // [2][NL][MAX_UNION][FF/32] their fp16 scales
    uint64_t *sc;     // [2][NL][NH][n_ctx]       attention scores
    uint64_t *kx;     // [NL][grid][2]            the LM head's per-workgroup argmax keys (low, high half)
};

// The device-driven MTP step's state and outputs, for the last stage of a fused draft or verify run
// whose control block has stage 1 or 2 (device memory; the host rewrites it when out_tok or the
// forced drafts change)
struct MtpHooks {
    MtpState *ms;
    RunCtl *ctl_verify;       // stage 1 writes the verify's control block here
    RunCtl *ctl_draft;        // stage 2 writes the next step's draft control block here
    uint32_t *out_tok;
    const int32_t *force;
    int32_t out_cap, force_n, n_ctx, pad;
};

struct FusedArgs {
    int32_t mode, n_layer, keep_logits, grid;
    const LayerDev *layers;        // [n_layer + 1] (the last one is the MTP block)
    ModelRt m;
    ActBufs b;
    uint32_t *sync;                // [FZ_SYNC_WORDS]
    FzXch xc;                      // tagged exchange buffers
    const uint64_t *xbase;         // the one allocation holding every exchange buffer, and its size
    uint32_t xbytes;
    unsigned long long *keys;      // [NL][grid] per-workgroup argmax keys of the LM head
    unsigned long long *trace;     // optional [grid][FZ_TRACE_EV][4]: phase id, start, barrier passed, end
    const MtpHooks *mh;            // the device-driven MTP step's stages
    // the LM head of this run: the output matrix, or (draft runs) the restricted draft head's rows,
    // whose local row r is token head_ids[r] (null: row r is token r)
    Q8W head_w;
    const uint32_t *head_ids;
};

constexpr int FZ_TRACE_EV = 2048;  // trace events per workgroup and run

size_t fused_lds_bytes(int n_ctx);
// workgroups of the fused kernel one CU holds with `lds` bytes of dynamic LDS (must be >= 1)
int fused_blocks_per_cu(size_t lds);
// dev_args: the run's FusedArgs in device memory
void launch_fused(const RunCtl *ctl, const FusedArgs *dev_args, int grid, size_t lds, hipStream_t st);
// after an aborted run: clear the error word and the finished counter and advance the tag base past
// every tag of the aborted launch (a fill kernel, no memset node)
void launch_fused_sync_reset(uint32_t *sync, hipStream_t st);
// every exchange word (xch: `words` 64-bit words) and sync word to zero: tag 0 is never live
void launch_fused_xch_clear(uint64_t *xch, size_t words, uint32_t *sync, hipStream_t st);

}  // namespace oxe
