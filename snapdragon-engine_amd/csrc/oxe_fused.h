// The fused run kernel: one persistent launch per engine run (verify of 1-2 lanes over every layer
// + the LM head; the MTP draft run; the MTP seeding run) instead of one launch per phase.
//
// Workgroups (one per CU, all resident) walk the run's phases in the same order as the reference's
// static plan (crates/model/src/plan.rs:171-261) and meet at a grid barrier between dependent
// phases, as the reference's thread team meets at its phase barriers (crates/sched/src/lib.rs:43-84).
// Each workgroup issues the next phase's weight loads before it waits at the barrier, so weight
// streaming overlaps the barrier latency. Activations exchanged between workgroups inside the launch
// are written and read with device-scope (coherent) accesses; nothing relies on a cache flush.
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

// barrier words (uint32): per-XCD arrival counters at [32 x] (x = 0..7, one 128-byte line each),
// the global arrival counter at [256], the release round at [288] (read at launch), the sticky
// error word at [320], per-XCD copies of the release round at [384 + 32 x], and the delta-net
// per-value-head arrival counters at [640 + 32 h] (h = 0..31)
constexpr int FZ_SYNC_WORDS = 640 + 32 * 32;
constexpr int FZ_XCD = 8;
constexpr int FZ_W_GLOB = 256, FZ_W_FLAG = 288, FZ_W_ERR = 320, FZ_W_REL = 384, FZ_W_HEAD = 640;

struct FusedArgs {
    int32_t mode, n_layer, keep_logits, grid;
    const LayerDev *layers;        // [n_layer + 1] (the last one is the MTP block)
    ModelRt m;
    ActBufs b;
    uint32_t *sync;                // [FZ_SYNC_WORDS]
    int8_t *hq;                    // [NL][OXE_MAX_UNION][FF] routed experts' h, Q8_0 codes
    uint16_t *hd;                  // [NL][OXE_MAX_UNION][FF/32] scales
    unsigned long long *keys;      // [NL][grid] per-workgroup argmax keys of the LM head
    unsigned long long *trace;     // optional [grid][FZ_TRACE_EV][4]: phase id, start, barrier passed, end
};

constexpr int FZ_TRACE_EV = 1024;  // trace events per workgroup and run

size_t fused_lds_bytes(int n_ctx);
// workgroups of the fused kernel one CU holds with `lds` bytes of dynamic LDS (must be >= 1)
int fused_blocks_per_cu(size_t lds);
// dev_args: the run's FusedArgs in device memory
void launch_fused(const RunCtl *ctl, const FusedArgs *dev_args, int grid, size_t lds, hipStream_t st);
// zero the barrier words (after an aborted run); a fill kernel, no memset node
void launch_fused_sync_reset(uint32_t *sync, hipStream_t st);

}  // namespace oxe
