// The fused run kernel (see oxe_fused.h): every phase of one engine run in one persistent launch.
//
// Arithmetic is the per-phase kernels' (k_layer.hip, k_attn.hip, k_moe.hip) with the reference's
// float order; only the distribution of work over threads differs:
//   * 512-thread workgroups, one per CU; in the norm prologues lane l of the run is handled by
//     threads [256 l, 256 l + 256) (8 elements each), and the exact double sums use the same
//     bracket test, so their result does not depend on the reduction order;
//   * Q8_0 GEMV slices: a workgroup owns a contiguous range of rows (or a fixed row list), loads all
//     of its 16-byte code chunks and scale rows into registers before it polls for the activations,
//     then forms the exact int32 block dots and runs one serial fp32 FMA chain per (row, lane) in
//     block order, as the reference's NEON GEMV;
//   * no grid barrier: every value a phase passes to another workgroup is a tagged 64-bit word
//     (FzXch, oxe_fused.h), and a reader polls the words it needs until they carry the tag of the
//     phase that writes them. A workgroup therefore waits only for its own inputs, and a phase of
//     one workgroup overlaps the previous phase of the others.
// Every poll is bounded: a poll that times out sets the sticky error word, and every workgroup
// that sees it leaves the run.
#include "oxe_fused.h"
#include "oxe_gemv.h"
#include "oxe_mtp_dev.h"
#include "oxe_prologue.h"
#include "oxe_route.h"
#include "oxe_shape.h"

namespace oxe {

using namespace shp;

namespace fz {

constexpr int FT = 512;                       // threads per workgroup
constexpr int SC_P = 16;                      // positions per scores chunk (workgroup step)
constexpr int SC_KS = HD + 32;                // LDS row stride of cached K rows in halves (576 B: the 16 rows of a
                                              // wave quarter fall on distinct banks)
constexpr uint32_t SPIN_MAX = 400000;         // ~0.4 s at one device-scope load per iteration
constexpr int POLL_SLEEP = 1;                 // s_sleep between polls of a missing word (units of 64 clocks)

// ---- address-space views ------------------------------------------------------------------------
// Each layer's phases form one non-inlined function, so pointers reach it as generic pointers and
// plain accesses compile to flat instructions. A flat access counts on both the vector-memory and
// the LDS wait counters, so an LDS wait would also wait for every weight load in flight. Device
// memory is therefore read and written through global-space views, and the run's arguments and run
// control (written by the host or the control kernels before the launch, never during it) through a
// uniform constant-space view (scalar loads; every dispatch starts with the scalar cache invalidated,
// so the values written before the launch are the ones read).
#define FZ_GAS __attribute__((address_space(1)))
#define FZ_CAS __attribute__((address_space(4)))
#define FZ_LDS __attribute__((address_space(3)))
template <int N> struct RawOf;   // a plain type of N bytes (no constructors, so it loads from any space)
template <> struct RawOf<2> { using T = uint16_t; };
template <> struct RawOf<4> { using T = uint32_t; };
template <> struct RawOf<8> { using T = uint32_t __attribute__((ext_vector_type(2))); };
template <> struct RawOf<16> { using T = uint32_t __attribute__((ext_vector_type(4))); };
template <class T>
OXE_DEV T gld(const T *p) {
    using R = typename RawOf<sizeof(T)>::T;
    return __builtin_bit_cast(T, *(const FZ_GAS R *)p);
}
// streamed once per run (weights, cache rows): a non-temporal load. Measured on MI355X: 256
// workgroups each reading 136 KB never read before take 14 us with plain loads and 6.5 us with
// non-temporal ones (the L2 does not allocate the lines).
template <class T>
OXE_DEV T gldn(const T *p) {
    using R = typename RawOf<sizeof(T)>::T;
    return __builtin_bit_cast(T, __builtin_nontemporal_load((const FZ_GAS R *)p));
}
template <class T>
OXE_DEV const FZ_CAS T *uni(const T *p) {
    const uint64_t v = (uint64_t)p;
    return (const FZ_CAS T *)(((uint64_t)__builtin_amdgcn_readfirstlane((uint32_t)(v >> 32)) << 32) |
                              (uint32_t)__builtin_amdgcn_readfirstlane((uint32_t)v));
}

// ---- device-scope accesses for data exchanged inside the launch -----------------------------
OXE_DEV void cst(float *p, float v) { __hip_atomic_store((FZ_GAS float *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
OXE_DEV float cld(const float *p) { return __hip_atomic_load((FZ_GAS float *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
OXE_DEV void cst32(void *p, uint32_t v) { __hip_atomic_store((FZ_GAS uint32_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
OXE_DEV uint32_t cld32(const void *p) { return __hip_atomic_load((FZ_GAS uint32_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
OXE_DEV void cst16(uint16_t *p, uint16_t v) { __hip_atomic_store((FZ_GAS uint16_t *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
OXE_DEV uint16_t cld16(const uint16_t *p) { return __hip_atomic_load((FZ_GAS uint16_t *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }
OXE_DEV void cst64(void *p, unsigned long long v) {
    __hip_atomic_store((FZ_GAS unsigned long long *)p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
OXE_DEV unsigned long long cld64(const void *p) {
    return __hip_atomic_load((FZ_GAS unsigned long long *)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
OXE_DEV uint4 cld128(const void *p) {
    const unsigned long long a = cld64(p), b = cld64((const char *)p + 8);
    return make_uint4((uint32_t)a, (uint32_t)(a >> 32), (uint32_t)b, (uint32_t)(b >> 32));
}
OXE_DEV void cst128(void *p, uint4 v) {
    cst64(p, (unsigned long long)v.x | ((unsigned long long)v.y << 32));
    cst64((char *)p + 8, (unsigned long long)v.z | ((unsigned long long)v.w << 32));
}

// ---- tagged exchange (FzXch) ----------------------------------------------------------------
// phases of run layer k (the verify's layer il: k = il; the MTP layer of a draft / seed run: k = 1,
// its entry acting as the "down" phase of k = 0)
enum { PH_PROJ = 0, PH_MIX = 1, PH_PV = 2, PH_OUT = 3, PH_ROUTER = 4, PH_EXP = 5, PH_DOWN = 6, PH_HEAD = 7 };

OXE_DEV unsigned long long ll_pack(uint32_t v, uint32_t tag) { return ((unsigned long long)tag << 32) | v; }
OXE_DEV void ll_st(uint64_t *p, uint32_t v, uint32_t tag) { cst64(p, ll_pack(v, tag)); }
OXE_DEV void ll_stf(uint64_t *p, float v, uint32_t tag) { ll_st(p, __builtin_bit_cast(uint32_t, v), tag); }
OXE_DEV bool ll_ok(unsigned long long w, uint32_t tag) { return (uint32_t)(w >> 32) == tag; }

// A thread's tagged inputs: word i at at(i).p with tag at(i).tag, wanted when at(i).on. While word 0
// (list the word expected last first) is missing, only it is polled (one load in flight per thread,
// so waiting workgroups do not flood the memory system with re-reads of data they already hold);
// every wanted word is loaded once, and missing ones again until all are there. SENT: poll word 0
// before the first load of the others (inputs that are usually not ready yet); otherwise every word
// is loaded at once first (inputs that usually are). Every poll is bounded: past SPIN_MAX polls the
// sticky error word is set; a poll also stops when another workgroup set it. false: the run was
// aborted.
struct LLW {
    const uint64_t *p;
    uint32_t tag;
    bool on;
};
// err[0]: the sticky error word; on a timeout err[1..4] note the word polled (expected tag, the tag
// seen, the low 32 bits of its address, the workgroup)
OXE_DEV bool ll_spin(uint32_t &spins, uint32_t *err, const uint64_t *p, uint32_t tag, unsigned long long seen) {
    if (++spins > SPIN_MAX) {
        cst32(err + 1, tag);
        cst32(err + 2, (uint32_t)(seen >> 32));
        cst32(err + 3, (uint32_t)(uintptr_t)p);
        cst32(err + 4, blockIdx.x);
        cst32(err, 1u);
        return false;
    }
    if ((spins & 31) == 0 && cld32(err)) return false;
    __builtin_amdgcn_s_sleep(POLL_SLEEP);
    return true;
}
// The exchange buffers as a buffer resource: two adjacent tagged words in one 16-byte device-scope
// load. A wave's loads of 8 bytes per lane are served at about a third of the rate of 16-byte ones
// when every workgroup reads the same words (measured: 32 KB read by 255 workgroups in 2.4 us with
// 8-byte loads, 0.7 us with 16-byte loads). Each 8-byte half is written by one 8-byte store and
// checked against its own tag, so a load that sees one half before the other only polls again.
struct XR {
    __amdgpu_buffer_rsrc_t r;
    const uint64_t *base;
};
OXE_DEV XR make_xr(const uint64_t *base, uint32_t bytes) {
    return XR{__builtin_amdgcn_make_buffer_rsrc((void *)base, (short)0, (int)bytes, 0x00020000), base};
}
OXE_DEV void cld128x(const XR &xr, const uint64_t *p, unsigned long long &w0, unsigned long long &w1) {
    typedef uint32_t u4 __attribute__((ext_vector_type(4)));
    // cache policy 16: sc1 (device scope, as the relaxed agent-scope atomic loads above)
    const u4 v = __builtin_amdgcn_raw_buffer_load_b128(xr.r, (int)((const char *)p - (const char *)xr.base), 0, 16);
    w0 = ((unsigned long long)v.y << 32) | v.x;
    w1 = ((unsigned long long)v.w << 32) | v.z;
}

// NP: words [0, 2 NP) come in adjacent pairs (at(2 m + 1).p == at(2 m).p + 1, 16-byte aligned, the
// same `on`), loaded 16 bytes at a time through xr in the first round.
template <int N, int NP, bool SENT, class At>
OXE_DEV bool ll_gather(At at, uint32_t (&v)[N], uint32_t *err, const XR *xr) {
    static_assert(N <= 32 && 2 * NP <= N, "mask of 32 words");
    uint32_t miss = 0;
    if (SENT && at(0).on) {
        const LLW x = at(0);
        uint32_t spins = 0;
        unsigned long long y;
        while (!ll_ok(y = cld64(x.p), x.tag))
            if (!ll_spin(spins, err, x.p, x.tag, y)) return false;
    }
    {
        unsigned long long w[N];
        // pairs through xr (without it, word by word)
        const int np = xr ? NP : 0;
#pragma unroll
        for (int m = 0; m < NP; m++) {
            w[2 * m] = w[2 * m + 1] = 0ull;
            if (m < np && at(2 * m).on) cld128x(*xr, at(2 * m).p, w[2 * m], w[2 * m + 1]);
        }
#pragma unroll
        for (int i = 0; i < N; i++)
            if (i >= 2 * np) w[i] = at(i).on ? cld64(at(i).p) : 0ull;
#pragma unroll
        for (int i = 0; i < N; i++) {
            v[i] = (uint32_t)w[i];
            if (at(i).on && !ll_ok(w[i], at(i).tag)) miss |= 1u << i;
        }
    }
    if (miss == 0) return true;
    uint32_t spins = 0;
    if (miss & 1u) {
        const LLW x = at(0);
        unsigned long long y;
        while (!ll_ok(y = cld64(x.p), x.tag))
            if (!ll_spin(spins, err, x.p, x.tag, y)) return false;
        v[0] = (uint32_t)y;
        miss &= ~1u;
    }
    const int np = xr ? NP : 0;
    while (miss) {
        unsigned long long w[N];
        // pairs with a missing half again 16 bytes at a time, the other words one by one
#pragma unroll
        for (int m = 0; m < NP; m++) {
            w[2 * m] = w[2 * m + 1] = 0ull;
            if (m < np && ((miss >> (2 * m)) & 3u)) cld128x(*xr, at(2 * m).p, w[2 * m], w[2 * m + 1]);
        }
#pragma unroll
        for (int i = 1; i < N; i++)
            if (i >= 2 * np) w[i] = ((miss >> i) & 1u) ? cld64(at(i).p) : 0ull;
#pragma unroll
        for (int i = 1; i < N; i++)
            if (((miss >> i) & 1u) && ll_ok(w[i], at(i).tag)) {
                v[i] = (uint32_t)w[i];
                miss &= ~(1u << i);
            }
        if (miss) {
            // the first word still missing, for the timeout note
            const uint64_t *mp = nullptr;
            uint32_t mt = 0;
            unsigned long long mw = 0;
#pragma unroll
            for (int i = N - 1; i >= 1; i--)
                if ((miss >> i) & 1u) { mp = at(i).p; mt = at(i).tag; mw = w[i]; }
            if (!ll_spin(spins, err, mp, mt, mw)) return false;
        }
    }
    return true;
}
OXE_DEV float u2f(uint32_t u) { return __builtin_bit_cast(float, u); }

// wait until at most n of this wave's vector memory operations are in flight (the other counters
// unconstrained): the weight loads issued before an input gather are left to finish in part, so
// the gather is issued when its inputs are more likely to be there
template <int N>
OXE_DEV void wait_vm() {
    static_assert(N >= 0 && N < 64, "vmcnt field");
    __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4) | (15 << 8));
}

// every thread's verdict of its polls combined (all threads call): false if any thread of the
// workgroup saw the run aborted. s_fail is sticky (cleared at the launch's start; an aborted
// workgroup leaves the run), and the second barrier keeps a later call's update from reaching a
// thread still reading this one's result.
OXE_DEV bool all_ok(bool ok, int *s_fail) {
    if (!ok) *s_fail = 1;
    __syncthreads();
    const bool r = *s_fail == 0;
    __syncthreads();
    return r;
}

// ---- GEMV slices ------------------------------------------------------------------------------
template <int K>
struct KG {
    static constexpr int NB = K / 32;          // blocks per row
    static constexpr int KCH = K / 16;         // 16-byte code chunks per row
    static constexpr int RPP = FT / KCH;       // rows per pass of the workgroup
    static constexpr int SPR = K / 256;        // 16-byte scale chunks per row
    static constexpr int FS = NB + 4;          // LDS row stride of the chain operands (16-byte rows)
};

template <int K, int MAXP>
struct WSlice {
    uint4 w[MAXP];
    uint4 s;
};

template <int K, int MAXR, int NL>
struct GSm {
    // the serial chain's operands per (lane, row, block): f32 of the int32 block dot, and the scale
    // product h2f(activation scale) * h2f(weight scale)
    alignas(16) float f[NL][MAXR][KG<K>::FS];
    alignas(16) float d[NL][MAXR][KG<K>::FS];
    float out[NL][MAXR];
};

// passes [P0, P1) of the codes (and the scales when SC) into registers, as wload; nr >= 1
template <int K, int MAXP, int P0, int P1, bool SC, class RowOf>
OXE_DEV void wload_part(WSlice<K, MAXP> &s, const int8_t *__restrict__ wq, const uint16_t *__restrict__ wd, int nr,
                        RowOf rowof) {
    using G = KG<K>;
    const int t = threadIdx.x, c = t % G::KCH, rs = t / G::KCH;
#pragma unroll
    for (int p = P0; p < P1; p++) {
        const int rl = p * G::RPP + rs;
        s.w[p] = gldn((const uint4 *)(wq + rowof(rl < nr ? rl : nr - 1) * K + c * 16));
    }
    if (SC) {
        const int sr = t / G::SPR, sk = t % G::SPR;
        s.s = gldn((const uint4 *)(wd + rowof(sr < nr ? sr : nr - 1) * G::NB + sk * 8));
    }
}

// codes of rows rowof(0..nr) and their scales into registers (plain loads: weights are read-only)
template <int K, int MAXP, bool NONEMPTY = false, class RowOf>
OXE_DEV void wload(WSlice<K, MAXP> &s, const int8_t *__restrict__ wq, const uint16_t *__restrict__ wd, int nr,
                   RowOf rowof) {
    using G = KG<K>;
    const int t = threadIdx.x, c = t % G::KCH, rs = t / G::KCH;
    // rows past nr load row nr - 1 again (wdot ignores them): no per-load branch, so the loads are
    // issued back to back without a wait between them; nothing is loaded (or read) when nr = 0
    if (!NONEMPTY && nr <= 0) return;   // NONEMPTY: the caller guarantees nr >= 1 (no branch)
#pragma unroll
    for (int p = 0; p < MAXP; p++) {
        const int rl = p * G::RPP + rs;
        s.w[p] = gldn((const uint4 *)(wq + rowof(rl < nr ? rl : nr - 1) * K + c * 16));
    }
    const int sr = t / G::SPR, sk = t % G::SPR;
    s.s = gldn((const uint4 *)(wd + rowof(sr < nr ? sr : nr - 1) * G::NB + sk * 8));
}

// the serial chain acc = fma(a[i], b[i], acc) for i = 0..N-1 in order, from +0 (N a multiple of 16;
// a, b 16-byte aligned, in LDS): the next sixteen operands of each are read while the current
// sixteen multiply-add, so the chain does not wait for an LDS read every step
template <int N>
OXE_DEV float chain_fma(const float *a, const float *b) {
    static_assert(N % 16 == 0, "sixteen per step");
    constexpr int S = 4;   // float4 pairs per step
    const float4 *a4 = (const float4 *)a, *b4 = (const float4 *)b;
    float4 x[S], y[S];
#pragma unroll
    for (int i = 0; i < S; i++) { x[i] = a4[i]; y[i] = b4[i]; }
    float acc = 0.0f;
    for (int q = 0; q < N / 4; q += S) {
        const int qn = q + S < N / 4 ? q + S : q;   // the last step reads its own operands again
        float4 u[S], v[S];
#pragma unroll
        for (int i = 0; i < S; i++) { u[i] = a4[qn + i]; v[i] = b4[qn + i]; }
        __builtin_amdgcn_sched_barrier(0);   // the reads stay ahead of this step's multiply-adds
#pragma unroll
        for (int i = 0; i < S; i++) {
            acc = __builtin_fmaf(x[i].x, y[i].x, acc);
            acc = __builtin_fmaf(x[i].y, y[i].y, acc);
            acc = __builtin_fmaf(x[i].z, y[i].z, acc);
            acc = __builtin_fmaf(x[i].w, y[i].w, acc);
        }
#pragma unroll
        for (int i = 0; i < S; i++) { x[i] = u[i]; y[i] = v[i]; }
    }
    return acc;
}

// g.out[l][r] = row r . lane l for the slice's nr rows (activation codes xq [NL][xq_ld] and scales
// xd [NL][xd_ld] in LDS). Ends with a barrier.
struct NoMid {
    OXE_DEV void operator()() const {}
};
template <int K, int MAXP, int NL, class Mid = NoMid>
OXE_DEV void wdot(const WSlice<K, MAXP> &s, int nr, const int8_t *xq, int xq_ld, const uint16_t *xd, int xd_ld,
                  GSm<K, MAXP * KG<K>::RPP, NL> &g, Mid mid = Mid()) {
    using G = KG<K>;
    const int t = threadIdx.x, c = t % G::KCH, rs = t / G::KCH;
    // codes first, in load order: each pass waits only for its own chunk; the scales (loaded last)
    // after the dots
    uint4 xa[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) xa[l] = *(const uint4 *)(xq + l * xq_ld + c * 16);
    // branch-free, so the independent dots interleave: both lanes of a pair hold the block's sum and
    // store it to the same word; rows past nr (< MAXP * RPP, inside g) get values nobody reads
#pragma unroll
    for (int p = 0; p < MAXP; p++) {
        const int rl = p * G::RPP + rs;
#pragma unroll
        for (int l = 0; l < NL; l++) {
            int32_t v = dot16(s.w[p], xa[l], 0);
            v += dpp_i<DPP_XOR1>(v);  // the other half of the 32-code block sits in the adjacent lane
            g.f[l][rl][c >> 1] = (float)v;
        }
    }
    {
        // thread (row sr, scale chunk sk) holds the weight scales of blocks [8 sk, 8 sk + 8)
        const int sr = t / G::SPR, sk = t % G::SPR;
        if (sr < nr) {
            const uint32_t sw[4] = {s.s.x, s.s.y, s.s.z, s.s.w};
#pragma unroll
            for (int l = 0; l < NL; l++) {
                float dv[8];
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    const uint16_t wsc = (uint16_t)(sw[q / 2] >> (16 * (q & 1)));
                    dv[q] = h2f(xd[l * xd_ld + 8 * sk + q]) * h2f(wsc);
                }
                *(float4 *)&g.d[l][sr][8 * sk] = make_float4(dv[0], dv[1], dv[2], dv[3]);
                *(float4 *)&g.d[l][sr][8 * sk + 4] = make_float4(dv[4], dv[5], dv[6], dv[7]);
            }
        }
    }
    __syncthreads();
    mid();
    if (t < nr * NL) {
        // one serial FMA chain per (row, lane) in block order, four blocks per LDS read
        const int rl = t % nr, l = t / nr;
        g.out[l][rl] = chain_fma<G::NB>(&g.f[l][rl][0], &g.d[l][rl][0]);
    }
    __syncthreads();
}

// ---- norm prologue (oxe_rms_norm_mul_f32, oxe_ops.cpp:32-42), lane l on threads [256 l, 256 l + 256)
struct NormSm {
    double red[2][4];
    float bc[2];
    double part[2][FT / 64];   // per-wave partial sums of squares of each lane (gathered inputs)
};

// v: this thread's 8 elements; xs: the lane's whole vector in LDS (sequential replay); wv8: this
// thread's 8 weights (loaded ahead by the caller). All threads call.
OXE_DEV void norm8(float v[8], const float *xs, const float wv8[8], float eps, NormSm &ns) {
    const int t = threadIdx.x, h = (t >> 8) & 1, tt = t & 255, wv = (t >> 6) & 3;
    double q = 0.0;
#pragma unroll
    for (int i = 0; i < 8; i++) q += (double)(v[i] * v[i]);
    const double p = wave_sum_d_any(q);
    if ((t & 63) == 0) ns.red[h][wv] = p;
    __syncthreads();
    const double P = ((ns.red[h][0] + ns.red[h][1]) + ns.red[h][2]) + ns.red[h][3];
    float mean;
    const bool ok = bracket_ok_mean(P, P, E, (double)E, &mean);
    if (!ok && tt == 0) {
        double s = 0.0;
        for (int i = 0; i < E; i++) s += (double)(xs[i] * xs[i]);
        ns.bc[h] = (float)(s / (double)E);
    }
    __syncthreads();
    if (!ok) mean = ns.bc[h];
    const float scale = 1.0f / sqrtf(mean + eps);
#pragma unroll
    for (int i = 0; i < 8; i++) v[i] = (v[i] * scale) * wv8[i];
}

// this thread's 8 norm weights (elements [8 tt, 8 tt + 8) of w)
struct W8 {
    float v[8];
};
OXE_DEV W8 wload8(const float *w) {
    W8 r;
    const int tt = threadIdx.x & 255;
    const float4 a = gld((const float4 *)(w + 8 * tt)), b = gld((const float4 *)(w + 8 * tt + 4));
    r.v[0] = a.x; r.v[1] = a.y; r.v[2] = a.z; r.v[3] = a.w; r.v[4] = b.x; r.v[5] = b.y; r.v[6] = b.z; r.v[7] = b.w;
    return r;
}

OXE_DEV void put8(float *x, const float *v) {
    *(float4 *)x = make_float4(v[0], v[1], v[2], v[3]);
    *(float4 *)(x + 4) = make_float4(v[4], v[5], v[6], v[7]);
}
OXE_DEV void get8(const float *x, float v[8]) {
    const float4 a = *(const float4 *)x, b = *(const float4 *)(x + 4);
    v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
}
// dequantize_row_q8_0 (quants_base.c:64-78) of elements [8 tt, 8 tt + 8) of token row tok
OXE_DEV void embed8t(const int8_t *eq, const uint16_t *ed, uint32_t tok, int tt, float v[8]) {
    const int8_t *q = eq + (int64_t)tok * E + 8 * tt;
    const float d = h2f(gld(ed + (int64_t)tok * (E / 32) + (8 * tt) / 32));
    const uint2 c = gld((const uint2 *)q);
#pragma unroll
    for (int i = 0; i < 4; i++) {
        v[i] = (float)(int8_t)(c.x >> (8 * i)) * d;
        v[i + 4] = (float)(int8_t)(c.y >> (8 * i)) * d;
    }
}

// entry l (divergent) of a per-lane array of the run control, from uniform scalar loads
// (each entry made wave-uniform first, so the selection stays a register select and the reads stay
// scalar loads)
template <int NL, class T>
OXE_DEV T lane_pick(const FZ_CAS T *v, int l) {
    static_assert(sizeof(T) == 4, "32-bit entries");
    T r = (T)__builtin_amdgcn_readfirstlane((int)v[0]);
#pragma unroll
    for (int i = 1; i < NL; i++) {
        const T vi = (T)__builtin_amdgcn_readfirstlane((int)v[i]);
        r = l == i ? vi : r;
    }
    return r;
}

// The run's lanes normalised with w and quantised to xq/xd (LDS). Source per lane: the token
// embedding (eq != null) or a tagged exchange buffer (src: [NL][E] words with tag `tag`, read
// coalesced: word t + FT j by thread t, staged in xf). xf: LDS staging of the raw vectors; xn
// (optional): the normalised f32 vectors. false: the run was aborted.
template <int NL, bool SENT = false, class Mid = NoMid>
OXE_DEV bool prologue(int nl, const FZ_CAS RunCtl *ctl, const int8_t *eq, const uint16_t *ed, const uint64_t *src,
                      uint32_t tag, uint32_t *err,
                      const W8 &w, float eps, float (*xf)[E], int8_t *xq, int xq_ld, uint16_t *xd, int xd_ld,
                      NormSm &ns, float (*xn)[E], int *s_ok, const XR *xr = nullptr, Mid mid = Mid()) {
    const int t = threadIdx.x, l = t >> 8, tt = t & 255;
    float v[8];
    const bool act = l < NL && l < nl;
    bool ok = true;
    if (eq) {
        if (act) embed8t(eq, ed, lane_pick<NL>(ctl->tok, l), tt, v);
        else
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.0f;
        if (l < NL) put8(&xf[l][8 * tt], v);
        __syncthreads();
        norm8(v, xf[l < NL ? l : 0], w.v, eps, ns);
    } else {
        static_assert(NL * E == 8 * FT && NL == 2, "8 words per thread, 4 of each lane");
        // word 2 (t + FT m) + h is u[2 m + h]: m < 2 are lane 0's, m >= 2 lane 1's
        auto wi = [&](int j) { return 2 * (t + FT * (j / 2)) + (j & 1); };
        uint32_t u[8];
        ok = ll_gather<8, 4, SENT>([&](int j) { return LLW{src + wi(j), tag, wi(j) / E < nl}; }, u, err, xr);
        // the exact parallel sum of squares (any order: the bracket below decides) from the
        // gathered words; the abort flag and the per-wave partials share one barrier
        double q[2] = {0.0, 0.0};
#pragma unroll
        for (int j = 0; j < 8; j++) {
            const int i = wi(j);
            const float x = i / E < nl ? u2f(u[j]) : 0.0f;
            xf[i / E][i % E] = x;
            q[j / 4] += (double)(x * x);
        }
        const double p0 = wave_sum_d_any(q[0]), p1 = wave_sum_d_any(q[1]);
        if (!ok) *s_ok = 1;
        if ((t & 63) == 0) { ns.part[0][t >> 6] = p0; ns.part[1][t >> 6] = p1; }
        __syncthreads();
        // no thread writes the sticky flag again before the barrier at the end of this prologue
        if (*s_ok != 0) return false;
        mid();   // inputs arrived
        float mean[2];
        bool replay = false;
#pragma unroll
        for (int h = 0; h < 2; h++) {
            double P = 0.0;
#pragma unroll
            for (int i = 0; i < FT / 64; i++) P += ns.part[h][i];
            replay |= !bracket_ok_mean(P, P, E, (double)E, &mean[h]);
        }
        if (replay) {   // uniform: every thread tested both lanes
            if (tt == 0 && l < NL) {
                double sq = 0.0;
                for (int i = 0; i < E; i++) sq += (double)(xf[l][i] * xf[l][i]);
                ns.bc[l] = (float)(sq / (double)E);
            }
            __syncthreads();
#pragma unroll
            for (int h = 0; h < 2; h++) mean[h] = ns.bc[h];
        }
        if (l < NL) get8(&xf[l][8 * tt], v);
        else
#pragma unroll
            for (int i = 0; i < 8; i++) v[i] = 0.0f;
        const float scale = 1.0f / sqrtf((l == 1 ? mean[1] : mean[0]) + eps);
#pragma unroll
        for (int i = 0; i < 8; i++) v[i] = (v[i] * scale) * w.v[i];
    }
    if (l < NL) {
        if (act) {
            quant8(v, xq + l * xq_ld + 8 * tt, xd + l * xd_ld + (8 * tt) / 32);
            if (xn) put8(&xn[l][8 * tt], v);
        } else {
            *(uint2 *)(xq + l * xq_ld + 8 * tt) = make_uint2(0, 0);
            if ((tt & 3) == 0) xd[l * xd_ld + (8 * tt) / 32] = 0;
            if (xn) put8(&xn[l][8 * tt], v);
        }
    }
    __syncthreads();
    return true;
}

// ---- shared memory of the phases -------------------------------------------------------------
template <int NL>
struct ProjSm {
    alignas(16) float xf[NL][E];
    alignas(16) int8_t xq[NL][E];
    uint16_t xd[NL][E / 32];
    NormSm ns;
    GSm<E, 52, NL> g;
};
template <int NL>
struct DnSm {
    float q[NL][DS], k[NL][DS], v[NL][HV], o[NL][HV];
    float g[NL], b[NL];
};
template <int NL>
struct OutSm {
    alignas(16) int8_t xq[NL][MIX_W];
    uint16_t xd[NL][MIX_W / 32];
    GSm<MIX_W, 8, NL> g;
    alignas(16) float stg[NL][MIX_W];   // the attention's f32 outputs, staged from the coalesced reads
};
template <int NL>
struct RouterSm {
    alignas(16) float xf[NL][E];
    alignas(16) float xn[NL][E];
    alignas(16) int8_t xq[NL][E];
    uint16_t xd[NL][E / 32];
    NormSm ns;
    alignas(16) float w[16][E / 16 + 4];    // chain-major: w[c][q] = row[c + 16 q]
    alignas(16) float sg[16][E / 16 + 4];
    alignas(16) float xc[NL][16][E / 16 + 4];
    GSm<E, 8, NL> g;
};
template <int NL>
struct ExpSm {
    float lg[NL][NEXP];
    alignas(16) int8_t xq[NL][E];
    uint16_t xd[NL][E / 32];
    GSm<E, 64, NL> g;
};
constexpr int DW_UNITS = OXE_MAX_UNION + 1;   // union experts + the shared expert
template <int NL>
struct DownSm {
    alignas(16) int8_t hq[NL][DW_UNITS][FF];
    uint16_t hd[NL][DW_UNITS][FF / 32];
    // chain operands per (unit, lane, row, block): f32 of the int32 block dot, scale product
    alignas(16) float f[DW_UNITS][NL][8][FF / 32 + 4];
    alignas(16) float d[DW_UNITS][NL][8][FF / 32 + 4];
    float dn[DW_UNITS][NL][8];
};
template <int NL>
struct ScSm {
    alignas(16) uint16_t q[NL * GQA][HD];
    float tmp[NL * GQA][HD];
    float ktmp[NL][HD];
    alignas(16) uint16_t knew[NL][HD];
    alignas(16) uint16_t krows[SC_P][SC_KS];   // cached K rows of the chunk's positions (padded rows)
};
constexpr int HEAD_P = 8;                   // LM-head tile: 8 passes of 4 rows
constexpr int HEAD_TR = HEAD_P * KG<E>::RPP;
template <int NL>
struct HeadSm {
    alignas(16) float xf[NL][E];
    alignas(16) float xn[NL][E];
    alignas(16) int8_t xq[NL][E];
    uint16_t xd[NL][E / 32];
    NormSm ns;
    GSm<E, HEAD_TR, NL> g;
    unsigned long long key[FT / 64][NL];
    int64_t claim[4];   // first tile of claimed pair k in claim[k & 3]
};
template <int NL>
struct EntrySm {
    alignas(16) float xf[NL][E];
    alignas(16) int8_t xq[NL][2 * E];
    uint16_t xd[NL][2 * E / 32];
    NormSm ns;
    GSm<2 * E, 8, NL> g;
};
template <int NL>
union PhaseSm {
    ProjSm<NL> proj;
    DnSm<NL> dn;
    OutSm<NL> out;
    RouterSm<NL> router;
    ExpSm<NL> exp;
    DownSm<NL> down;
    ScSm<NL> sc;
    HeadSm<NL> head;
    EntrySm<NL> entry;
};

// state that lives across phases of one layer (static LDS)
template <int NL>
struct Persist {
    RouteOut ro;
    int32_t uni[OXE_MAX_UNION];
    int32_t nu;
    int32_t slot[NL][KUSED];   // union slot of each lane's rank-j expert
    alignas(16) int8_t xq[NL][E];    // the post-attention-norm lanes, Q8_0 (router phase -> experts)
    uint16_t xd[NL][E / 32];
    int fail;                        // a poll of this workgroup saw the run aborted (sticky)
    uint32_t base;                   // tag base of the launch
    uint32_t tev;                    // trace: next event index of this workgroup
    uint32_t dyn_off;                // LDS offset of the dynamic LDS (fz_dyn), set by the kernel
    uint64_t exp2tab[32];            // the C-library expf's table (oxe_libm), read from LDS by the gates
    unsigned long long t_start, t_pass, t_mark;
};

}  // namespace fz

// LDS of the fused kernel: the phases' union (dynamic) and the state that lives across phases
extern __shared__ __align__(16) unsigned char fz_dyn[];
__shared__ fz::Persist<OXE_NL> fz_ps;

namespace fz {

// the expf table's LDS copy as an LDS-space pointer (its reads compile to LDS loads)
OXE_DEV const FZ_LDS uint64_t *exp_tab() { return (const FZ_LDS uint64_t *)&fz_ps.exp2tab[0]; }

template <int NL>
struct Ctx {
    const FZ_CAS RunCtl *ctl;   // written by the control kernels before the launch, read-only in it
    const FZ_CAS FusedArgs *a;
    PhaseSm<NL> *sm;
    Persist<NL> *ps;
    unsigned char *dyn;
    uint32_t *err;              // the sticky error word
    uint32_t base;              // tag base of the launch
    int k;                      // run layer index: exchange buffer parity k & 1
    unsigned long long *trace;
    int nl, G, b;
    // tag of phase ph of run layer kk
    OXE_DEV uint32_t tag(int kk, int ph) const { return base + 1u + 8u * (uint32_t)kk + (uint32_t)ph; }
    OXE_DEV int par() const { return k & 1; }
};

template <int NL>
OXE_DEV Ctx<NL> make_ctx(const RunCtl *ctl, const FusedArgs *ap, int k) {
    static_assert(NL == OXE_NL, "one lane count");
    const FZ_CAS FusedArgs *a = uni(ap);
    // the dynamic LDS from its offset (a non-kernel function would otherwise look its base up in a
    // per-kernel table in device memory, a load that may be repeated behind the weight loads in flight)
    unsigned char *dyn = (unsigned char *)(FZ_LDS unsigned char *)(uintptr_t)fz_ps.dyn_off;
    // the phase's LDS aliases the previous phase's: no thread writes it before every thread is done
    // with the previous phase
    __syncthreads();
    Ctx<NL> c{uni(ctl), a, (PhaseSm<NL> *)dyn, &fz_ps, dyn, a->sync + FZ_W_ERR,
              (uint32_t)__builtin_amdgcn_readfirstlane((int)fz_ps.base), k, a->trace, 0, 0, 0};
    c.nl = c.ctl->nl < 1 ? 1 : (c.ctl->nl > NL ? NL : c.ctl->nl);
    c.G = gridDim.x;
    c.b = blockIdx.x;
    return c;
}

// layer il's tensors (il is uniform: read with scalar loads)
template <int NL>
OXE_DEV const FZ_CAS LayerDev &layer_of(const Ctx<NL> &c, int il) {
    return *(uni(c.a->layers) + __builtin_amdgcn_readfirstlane(il));
}

// Phases are inlined into one non-inlined function per layer (run_layer). A call boundary costs a
// wait for every memory operation in flight (the callee's entry waits for all counters), which at a
// phase boundary would hold the next phase's weight loads behind the previous phase's output stores;
// inlining the whole run instead leaves the register allocator with one function too large to
// allocate without spills.
#define FZ_PHASE __device__ __attribute__((always_inline)) inline

// phase trace (optional): thread 0 records the device wall clock (100 MHz) at the phase start,
// when its barrier released, and at its arrival
enum { TP_PROJ = 1, TP_DN, TP_SCORES, TP_PV, TP_OUT, TP_ROUTER, TP_EXPERTS, TP_DOWN, TP_ENTRY, TP_HEAD };
template <int NL>
OXE_DEV void tr_start(Ctx<NL> &c) {
    if (c.trace && threadIdx.x == 0) c.ps->t_start = wall_clock64();
}
template <int NL>
OXE_DEV void tr_pass(Ctx<NL> &c) {
    if (c.trace && threadIdx.x == 0) c.ps->t_mark = c.ps->t_pass = wall_clock64();
}
// sub-step marker inside a phase: an event (id, previous mark, 0, now)
template <int NL>
OXE_DEV void tr_mark(Ctx<NL> &c, int id) {
    if (c.trace && threadIdx.x == 0 && c.ps->tev < FZ_TRACE_EV) {
        const unsigned long long now = wall_clock64();
        unsigned long long *e = c.trace + ((size_t)c.b * FZ_TRACE_EV + c.ps->tev++) * 4;
        e[0] = (unsigned long long)id;
        e[1] = c.ps->t_mark;
        e[2] = 0ull;
        e[3] = now;
        c.ps->t_mark = now;
    }
}
template <int NL>
OXE_DEV void tr_end(Ctx<NL> &c, int id) {
    if (c.trace && threadIdx.x == 0 && c.ps->tev < FZ_TRACE_EV) {
        unsigned long long *e = c.trace + ((size_t)c.b * FZ_TRACE_EV + c.ps->tev++) * 4;
        e[0] = (unsigned long long)id;
        e[1] = c.ps->t_start;
        e[2] = c.ps->t_pass;
        e[3] = wall_clock64();
    }
}

// ---- phases ----------------------------------------------------------------------------------

// proj: rows [r_begin, r_end) of the layer's input projection over the normalised lanes; V rows
// (attention) also go to V^T at pos0 + l (read by later launches; this launch's attention takes the
// new positions' V from the projection outputs). Input: the embedding (layer 0 of a verify) or x.
// A workgroup's projection slice: rows [r0, r0 + nr) of rows [r_begin, r_end) of the layer's
// matrix, its weights and the attention-norm weights, loaded into registers. The down phase of the
// layer before loads it once its own inputs are in, so the slice streams during the down phase's
// work and the exchange of its outputs.
struct ProjPre {
    WSlice<E, 13> ws;
    W8 nw;
    int r0, nr;
};
OXE_DEV void proj_load(const FZ_CAS LayerDev &L, int b, int G, int r_begin, int r_end, ProjPre &pp) {
    const int n = r_end - r_begin;
    pp.r0 = r_begin + (int)((int64_t)n * b / G);
    pp.nr = r_begin + (int)((int64_t)n * (b + 1) / G) - pp.r0;
    const int r0 = pp.r0;
    wload<E, 13>(pp.ws, L.proj.q, L.proj.d, pp.nr, [&](int rl) { return (int64_t)(r0 + rl); });
    pp.nw = wload8(L.attn_norm);
}
OXE_DEV int proj_rows(const FZ_CAS LayerDev &L) { return L.att ? AT_ROWS : DN_ROWS; }
// the same in four parts (passes 0-3, 4-7, 8-11, then 12 with the scales and norm weights), issued
// between steps of the down phase: a wave that issues more loads than the memory pipeline takes at
// once stalls at the issue until earlier ones complete, which would hold the down phase's own work
template <int PART>
OXE_DEV void proj_load_part(const FZ_CAS LayerDev &L, int b, int G, int r_begin, int r_end, ProjPre &pp) {
    if (PART == 0) {
        const int n = r_end - r_begin;
        pp.r0 = r_begin + (int)((int64_t)n * b / G);
        pp.nr = r_begin + (int)((int64_t)n * (b + 1) / G) - pp.r0;
    }
    const int r0 = pp.r0;
    auto rowof = [&](int rl) { return (int64_t)(r0 + rl); };
    if (PART == 0) wload_part<E, 13, 0, 4, false>(pp.ws, L.proj.q, L.proj.d, pp.nr, rowof);
    if (PART == 1) wload_part<E, 13, 4, 8, false>(pp.ws, L.proj.q, L.proj.d, pp.nr, rowof);
    if (PART == 2) wload_part<E, 13, 8, 12, false>(pp.ws, L.proj.q, L.proj.d, pp.nr, rowof);
    if (PART == 3) {
        wload_part<E, 13, 12, 13, true>(pp.ws, L.proj.q, L.proj.d, pp.nr, rowof);
        pp.nw = wload8(L.attn_norm);
    }
}

// ---- delta-net inputs known ahead (the projection phase loads them for the delta-net phase)
constexpr int DN_WPH = 8, DN_RPW = HV / DN_WPH;
// conv channel of thread t (q: t < 128, k: t < 256, the workgroup's 16 v rows: t < 272; others
// re-read the last v row)
OXE_DEV int dn_channel(int vh, int row0, int t) {
    const int kh = vh % NKH;
    if (t < DS) return kh * DS + t;
    if (t < 2 * DS) return NKH * DS + kh * DS + (t - DS);
    const int i = t - 2 * DS < DN_RPW ? t - 2 * DS : DN_RPW - 1;
    return 2 * NKH * DS + vh * HV + row0 + i;
}
// the delta-net phase's inputs known before the layer runs: the thread's state row (slot cur, an
// earlier launch), its conv channel's state and weights, the head's gate constants and the
// gated-norm weights. The projection phase loads them after its block dots (no later wait of that
// phase depends on the count of loads in flight, so the loads may be conditional).
struct DnPre {
    float r[8];
    float s0, s1, s2;
    float4 cw;
    float dtb, sa, nw0, nw1;
};
OXE_DEV void dn_load(const FZ_CAS FusedArgs &a, const FZ_CAS LayerDev &L, int b, int cur, DnPre &dp) {
    const int t = threadIdx.x, lane = t & 63;
    const int vh = (b / DN_WPH) % NVH, row0 = (b % DN_WPH) * DN_RPW;
    const int64_t conv_slot = (int64_t)a.m.n_rec * NCH * (KC - 1);
    const int64_t ssm_slot = (int64_t)a.m.n_rec * NVH * HV * HV;
    const float *conv_state = a.m.conv_state + (int64_t)L.index * NCH * (KC - 1);
    const float *ssm = a.m.ssm_state + (int64_t)L.index * NVH * HV * HV;
    const int rg = (t >> 4) % DN_RPW, cc = t & 15;
    if (t < DN_RPW * 16) {
        const float *src = ssm + (int64_t)cur * ssm_slot + ((int64_t)vh * HV + row0 + rg) * HV;
#pragma unroll
        for (int q = 0; q < 8; q++) dp.r[q] = gldn(src + cc + 16 * q);
    }
    if (t < 2 * DS + DN_RPW) {
        const int ch = dn_channel(vh, row0, t);
        const float *st = conv_state + (int64_t)cur * conv_slot + (int64_t)ch * (KC - 1);
        dp.s0 = gldn(st); dp.s1 = gldn(st + 1); dp.s2 = gldn(st + 2);
        dp.cw = gld((const float4 *)(L.conv + (int64_t)ch * KC));
    }
    if ((t >> 6) == 5) {
        dp.dtb = gld(L.dt_bias + vh);
        dp.sa = gld(L.ssm_a + vh);
    }
    if ((t >> 6) < 2) {
        dp.nw0 = gld(L.ssm_norm + lane);
        dp.nw1 = gld(L.ssm_norm + lane + 64);
    }
}

// pp: the slice (loaded: by the down phase before; otherwise loaded here)
template <int NL>
FZ_PHASE bool phase_proj(const RunCtl *ctl, const FusedArgs *ap, int il, int k, bool embed, int r_begin, int r_end,
                         ProjPre &pp, bool loaded, DnPre &dp) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, k);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    const FZ_CAS LayerDev &L = layer_of(c, il);
    auto &s = c.sm->proj;
    if (!loaded) {
        proj_load(L, c.b, c.G, r_begin, r_end, pp);
        if (!embed) wait_vm<8>();   // about half of the 16 loads above
    }
    const WSlice<E, 13> &ws = pp.ws;
    const W8 &nw = pp.nw;
    const int r0 = pp.r0, nr = pp.nr;
    uint64_t *xin = a.xc.x + (size_t)c.par() * NL * E;
    const XR xr = make_xr(a.xbase, a.xbytes);
    if (!prologue<NL>(c.nl, c.ctl, embed ? a.m.tok_embd.q : nullptr, a.m.tok_embd.d, xin, k > 0 ? c.tag(k - 1, PH_DOWN) : 0u,
                      c.err, nw, a.m.eps, s.xf, &s.xq[0][0], E, &s.xd[0][0], E / 32, s.ns, nullptr, &c.ps->fail, &xr,
                      [&] { tr_pass(c); }))
        return false;
    if (embed) tr_pass(c);
    // a delta-net layer's next phase inputs that do not depend on this one
    tr_mark(c, 111);
    if (embed && c.b == 0) {
        // the embedded input is the residual of layer 0
        const int t = threadIdx.x, l = t >> 8, tt = t & 255;
        if (l < c.nl)
            for (int i = 0; i < 8; i++) ll_stf(xin + l * E + 8 * tt + i, s.xf[l][8 * tt + i], c.tag(k, PH_PROJ));
    }
    // after the block dots (every weight wait of this phase done): a delta-net layer's inputs of the
    // next phase that do not depend on this one
    wdot<E, 13, NL>(ws, nr, &s.xq[0][0], E, &s.xd[0][0], E / 32, s.g, [&] {
        tr_mark(c, 113);
        if (!L.att) dn_load(a, L, c.b, c.ctl->cur, dp);
    });
    tr_mark(c, 112);
    const int t = threadIdx.x;
    uint64_t *po = a.xc.p + (size_t)c.par() * NL * DN_ROWS;
    if (t < NL * 52) {
        const int l = t / 52, rl = t % 52;
        if (l < c.nl && rl < nr) {
            const int row = r0 + rl;
            const float v = s.g.out[l][rl];
            ll_stf(po + (int64_t)l * DN_ROWS + row, v, c.tag(k, PH_PROJ));
            if (L.att && row >= AT_V) {
                uint16_t *vt = a.m.vcache + (int64_t)L.index * NKV * HD * a.m.n_ctx;
                vt[(int64_t)(row - AT_V) * a.m.n_ctx + c.ctl->pos0 + l] = f2h(v);
            }
        }
    }
    tr_end(c, TP_PROJ);
    return true;
}

// Delta-net recurrence (k_layer.hip dn_kernel's arithmetic) over DN_WPH workgroups per value head:
// workgroup b takes value head vh = b / DN_WPH and state rows [16 (b % DN_WPH), +16); thread
// (rg = t/16, c = t%16), t < 256, owns state row 16 (b % DN_WPH) + rg. Every workgroup of a head
// forms the head's conv outputs and normalised q, k (gdn conv + l2 norms, oxe_ops.cpp:218-267) and
// writes its 16 outputs; the head's first workgroup then reads the head's 128 outputs back (tagged)
// and forms their gated norm and Q8_0 quantisation.
OXE_DEV float dot16_tree_f(float acc) { return dot16_tree_dpp(acc); }
OXE_DEV float conv4f(float s0, float s1, float s2, float xn, const float *c) {
    const float p0 = s0 * c[0], p1 = s1 * c[1], p2 = s2 * c[2], p3 = xn * c[3];
    float sumf = 0.0f;
    sumf = sumf + p0;
    sumf = sumf + p1;
    sumf = sumf + p2;
    sumf = sumf + p3;
    return sumf;
}
template <int NL>
FZ_PHASE bool phase_dn(const RunCtl *ctl, const FusedArgs *ap, int il, int k, const DnPre &dp) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, k);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    const FZ_CAS LayerDev &L = layer_of(c, il);
    auto &s = c.sm->dn;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63;
    const int vh = c.b / DN_WPH, row0 = (c.b % DN_WPH) * DN_RPW;
    const bool worker = c.b < NVH * DN_WPH;
    const int cur = c.ctl->cur;
    const int64_t conv_slot = (int64_t)a.m.n_rec * NCH * (KC - 1);
    const int64_t ssm_slot = (int64_t)a.m.n_rec * NVH * HV * HV;
    float *conv_state = a.m.conv_state + (int64_t)L.index * NCH * (KC - 1);
    float *ssm = a.m.ssm_state + (int64_t)L.index * NVH * HV * HV;
    const int rg = t >> 4, cc = t & 15;
    const bool dlt = worker && t < DN_RPW * 16;
    const int ch = dn_channel(vh, row0, t);
    const bool conv = worker && t < 2 * DS + DN_RPW;
    const bool writer = t < 2 * DS ? (vh < NKH && row0 == 0) : true;
    float r[8];
#pragma unroll
    for (int q = 0; q < 8; q++) r[q] = dp.r[q];
    float s0 = dp.s0, s1 = dp.s1, s2 = dp.s2;
    const float cw[KC] = {dp.cw.x, dp.cw.y, dp.cw.z, dp.cw.w};
    // gate thread of lane gl (wave 5) and the gated-norm weights (waves < NL)
    const int gl = t - 5 * 64;
    const bool gate = worker && gl >= 0 && gl < NL;
    const float dtb = dp.dtb, sa = dp.sa, nw0 = dp.nw0, nw1 = dp.nw1;
    const uint64_t *pin = a.xc.p + (size_t)c.par() * NL * DN_ROWS;
    uint64_t *gx = a.xc.g + (size_t)c.par() * NL * MIX_W;
    const uint32_t tp = c.tag(k, PH_PROJ), tg = c.tag(k, PH_MIX);
    if (worker) {
        const int nl = c.nl;
        float xin[NL], ga, gb;
        bool ok;
        {
            uint32_t u[NL + 2];
            const int gl1 = gl < 0 ? 0 : (gl >= NL ? NL - 1 : gl);
            ok = ll_gather<NL + 2, 0, true>(
                [&](int i) {
                    if (i < NL) return LLW{pin + (int64_t)i * DN_ROWS + ch, tp, conv && i < nl};
                    return LLW{pin + (int64_t)gl1 * DN_ROWS + (i == NL ? DN_ALPHA : DN_BETA) + vh, tp, gate && gl < nl};
                },
                u, c.err, nullptr);
#pragma unroll
            for (int l = 0; l < NL; l++) xin[l] = u2f(u[l]);
            ga = u2f(u[NL]);
            gb = u2f(u[NL + 1]);
        }
        if (!all_ok(ok, &c.ps->fail)) return false;
        tr_pass(c);
        if (conv) {
#pragma unroll
            for (int l = 0; l < NL; l++) {
                if (l >= nl) break;
                const float y = v_silu(conv4f(s0, s1, s2, xin[l], cw));
                s0 = s1; s1 = s2; s2 = xin[l];
                if (writer) {
                    float *dst = conv_state + (int64_t)((cur + l + 1) % OXE_NSLOTS) * conv_slot + (int64_t)ch * (KC - 1);
                    dst[0] = s0; dst[1] = s1; dst[2] = s2;
                }
                if (t < DS) s.q[l][t] = y;
                else if (t < 2 * DS) s.k[l][t - DS] = y;
                else s.v[l][t - 2 * DS] = y;
            }
        }
        __syncthreads();
        tr_mark(c, 121);
        // the gates (wave 5) beside the l2 norms of q (wave 2 l) and k (wave 2 l + 1)
        if (gate && gl < nl) {
            s.g[gl] = oxe_libm::expf_t(softplus_t(ga + dtb, exp_tab()) * sa, exp_tab());
            s.b[gl] = sigmoid_t(gb, exp_tab());
        }
        if (w < 2 * NL && (w >> 1) < nl) {
            const int l = w >> 1;
            float *xv = (w & 1) ? s.k[l] : s.q[l];
            const float a0 = xv[lane], a1 = xv[lane + 64];
            const float nf = (float)DS;
            const float mean = wave_mean_sq_128(a0, a1, xv);
            const float scale = 1.0f / sqrtf(mean + a.m.eps / nf);
            const float sq = 1.0f / sqrtf(nf);
            xv[lane] = (a0 * scale) * sq;
            xv[lane + 64] = (a1 * scale) * sq;
        }
        __syncthreads();
        tr_mark(c, 122);
        // delta rule per lane; the new states are kept in registers and stored after the count
        const float scale = 1.0f / sqrtf((float)HV);
        float stl[NL][8];
        if (dlt) {
#pragma unroll
            for (int l = 0; l < NL; l++) {
                if (l >= nl) break;
                const float eg = s.g[l], beta = s.b[l];
                float acc = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    r[q] = r[q] * eg;
                    acc = __builtin_fmaf(r[q], s.k[l][cc + 16 * q], acc);
                }
                const float sk = dot16_tree_f(acc);
                const float delta = (s.v[l][rg] - sk) * beta;
                acc = 0.0f;
#pragma unroll
                for (int q = 0; q < 8; q++) {
                    r[q] = __builtin_fmaf(s.k[l][cc + 16 * q], delta, r[q]);
                    acc = __builtin_fmaf(r[q], s.q[l][cc + 16 * q], acc);
                    stl[l][q] = r[q];
                }
                const float sq = dot16_tree_f(acc);
                if (cc == 0) ll_stf(gx + (int64_t)l * DIN + vh * HV + row0 + rg, sq * scale, tg);
            }
        }
        // the head's first workgroup reads the head's 128 outputs of every lane back
        const bool last = row0 == 0;
        float x0, x1, z0, z1;
        {
            const int wl = w < NL ? w : 0;
            const uint64_t *o = gx + (int64_t)wl * DIN + vh * HV;
            const uint64_t *z = pin + (int64_t)wl * DN_ROWS + DN_Z + vh * HV;
            const bool on = last && w < nl;
            uint32_t u[4];
            ok = ll_gather<4, 0, true>(
                [&](int i) {
                    const int off = lane + 64 * (i & 1);
                    return i < 2 ? LLW{o + off, tg, on} : LLW{z + off, tp, on};
                },
                u, c.err, nullptr);
            x0 = u2f(u[0]); x1 = u2f(u[1]); z0 = u2f(u[2]); z1 = u2f(u[3]);
        }
        if (last) tr_mark(c, 124);
        if (dlt) {
#pragma unroll
            for (int l = 0; l < NL; l++) {
                if (l >= nl) break;
                float *dst = ssm + (int64_t)((cur + l + 1) % OXE_NSLOTS) * ssm_slot + ((int64_t)vh * HV + row0 + rg) * HV;
#pragma unroll
                for (int q = 0; q < 8; q++) dst[cc + 16 * q] = stl[l][q];
            }
        }
        tr_mark(c, 123);
        // gated norm (oxe_ops.cpp:19-49 rms + ssm_norm * silu(z)) and Q8_0 quantization of the head
        if (last && w < nl) {
            const int l = w;
            s.o[l][lane] = x0;
            s.o[l][lane + 64] = x1;
            const float mean = wave_mean_sq_128(x0, x1, s.o[l]);
            const float sc = 1.0f / sqrtf(mean + a.m.eps);
            const float o0 = ((x0 * sc) * nw0) * v_silu(z0);
            const float o1 = ((x1 * sc) * nw1) * v_silu(z1);
            float d0, d1;
            const uint32_t p0 = quant32_lanes(o0, &d0), p1 = quant32_lanes(o1, &d1);
            uint64_t *q = a.xc.o + ((size_t)c.par() * NL + l) * (DIN / 4) + (vh * HV) / 4;
            if ((lane & 3) == 0) {
                ll_st(q + lane / 4, p0, tg);
                ll_st(q + (lane + 64) / 4, p1, tg);
            }
            uint64_t *d = a.xc.od + ((size_t)c.par() * NL + l) * (DIN / 32) + vh * (HV / 32);
            if (lane == 0) { ll_st(d + 0, f2h(d0), tg); ll_st(d + 2, f2h(d1), tg); }
            if (lane == 32) { ll_st(d + 1, f2h(d0), tg); ll_st(d + 3, f2h(d1), tg); }
        }
        if (last) tr_mark(c, 125);
        if (!all_ok(ok, &c.ps->fail)) return false;
    }
    tr_end(c, TP_DN);
    return true;
}

// out: rows [8 b, 8 b + 8) of ssm_out / attn_output over the quantised mixer output, + the residual
// (x of the layer, tag xtag); the sums go to x1
template <int NL>
FZ_PHASE bool phase_out(const RunCtl *ctl, const FusedArgs *ap, int il, int k, uint32_t xtag) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, k);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    const FZ_CAS LayerDev &L = layer_of(c, il);
    auto &s = c.sm->out;
    const int t = threadIdx.x;
    const int r0 = 8 * c.b;
    WSlice<MIX_W, 4> ws;
    wload<MIX_W, 4>(ws, L.out.q, L.out.d, 8, [&](int rl) { return (int64_t)(r0 + rl); });
    const uint64_t *xin = a.xc.x + (size_t)c.par() * NL * E;
    const uint32_t tm = c.tag(k, L.att ? PH_PV : PH_MIX);
    bool ok;
    float xres;
    const int l = t >> 8, tt = t & 255;
    const bool act = l < NL && l < c.nl;
    const int l1 = l < NL ? l : 0;
    const bool xon = t < NL * 8 && t / 8 < c.nl;
    const uint64_t *xr = xin + (int64_t)((t / 8) % NL) * E + r0 + t % 8;
    const XR xrs = make_xr(a.xbase, a.xbytes);
    if (L.att) {
        // the attention's gated outputs (f32), read coalesced (word t + FT j) into LDS; then thread
        // (lane l, 16 elements at 16 tt), Q8_0 blocks of 32 over adjacent thread pairs
        // (quantize_row_q8_0 NEON: amax, d = amax / 127, id from the f32 d, round-half-even codes)
        static_assert(NL * MIX_W == 16 * FT, "16 words per thread");
        {
            // word 2 (t + FT m) + h is u[2 m + h]
            auto wi = [&](int j) { return 2 * (t + FT * (j / 2)) + (j & 1); };
            uint32_t u[17];
            const uint64_t *gi = a.xc.g + (size_t)c.par() * NL * MIX_W;
            ok = ll_gather<17, 8, true>(
                [&](int j) { return j < 16 ? LLW{gi + wi(j), tm, wi(j) / MIX_W < c.nl} : LLW{xr, xtag, xon}; }, u, c.err,
                &xrs);
#pragma unroll
            for (int j = 0; j < 16; j++) {
                const int i = wi(j);
                s.stg[i / MIX_W][i % MIX_W] = i / MIX_W < c.nl ? u2f(u[j]) : 0.0f;
            }
            xres = u2f(u[16]);
        }
        if (!all_ok(ok, &c.ps->fail)) return false;
        float v[16];
#pragma unroll
        for (int q = 0; q < 16; q += 4) {
            const float4 f = *(const float4 *)&s.stg[l1][16 * tt + q];
            v[q] = f.x; v[q + 1] = f.y; v[q + 2] = f.z; v[q + 3] = f.w;
        }
        float am = 0.0f;
#pragma unroll
        for (int q = 0; q < 16; q++) am = fmaxf(am, __builtin_fabsf(v[q]));
        am = fmaxf(am, dpp_f<DPP_XOR1>(am));
        const float dd = am / 127.0f;
        const float id = dd != 0.0f ? 1.0f / dd : 0.0f;
        uint32_t w[4];
#pragma unroll
        for (int q = 0; q < 4; q++) {
            uint32_t u = 0;
#pragma unroll
            for (int bb = 0; bb < 4; bb++) u |= ((uint32_t)((int32_t)__builtin_rintf(v[4 * q + bb] * id) & 0xff)) << (8 * bb);
            w[q] = u;
        }
        if (l < NL) {
            *(uint4 *)&s.xq[l][16 * tt] = make_uint4(w[0], w[1], w[2], w[3]);
            if ((tt & 1) == 0) s.xd[l][tt / 2] = f2h(dd);
        }
        __syncthreads();
    } else {
        // the quantised delta-net output (4 codes per word), read coalesced: word t + FT j by thread
        // t; scale word t by threads t < NL * MIX_W / 32
        static_assert(NL * MIX_W / 4 == 4 * FT, "4 words per thread");
        const int ll = (t / (MIX_W / 32)) % NL, bb = t % (MIX_W / 32);
        const bool don = t < NL * (MIX_W / 32) && t / (MIX_W / 32) < c.nl;
        const uint64_t *oi = a.xc.o + (size_t)c.par() * NL * (MIX_W / 4);
        const uint64_t *di = a.xc.od + ((size_t)c.par() * NL + ll) * (MIX_W / 32) + bb;
        // word 2 (t + FT m) + h is u[2 m + h]
        auto wi = [&](int j) { return 2 * (t + FT * (j / 2)) + (j & 1); };
        uint32_t u[6];
        ok = ll_gather<6, 2, true>(
            [&](int j) {
                return j < 4 ? LLW{oi + wi(j), tm, wi(j) / (MIX_W / 4) < c.nl}
                             : (j == 4 ? LLW{di, tm, don} : LLW{xr, xtag, xon});
            },
            u, c.err, &xrs);
#pragma unroll
        for (int j = 0; j < 4; j++) {
            const int i = wi(j), li = i / (MIX_W / 4);
            ((uint32_t *)&s.xq[li][0])[i % (MIX_W / 4)] = li < c.nl ? u[j] : 0u;
        }
        if (t < NL * (MIX_W / 32)) s.xd[ll][bb] = don ? (uint16_t)u[4] : (uint16_t)0;
        xres = u2f(u[5]);
        if (!all_ok(ok, &c.ps->fail)) return false;
    }
    tr_pass(c);
    wdot<MIX_W, 4, NL>(ws, 8, &s.xq[0][0], MIX_W, &s.xd[0][0], MIX_W / 32, s.g, [&] { tr_mark(c, 171); });
    tr_mark(c, 172);
    if (t < NL * 8) {
        const int ll = t / 8, rl = t % 8;
        if (ll < c.nl)
            ll_stf(a.xc.x1 + ((size_t)c.par() * NL + ll) * E + r0 + rl, s.g.out[ll][rl] + xres, c.tag(k, PH_OUT));
    }
    tr_end(c, TP_OUT);
    return true;
}

// router: post_attention_norm + quantise (kept in this workgroup's persistent LDS for the experts),
// router row b (f32, ggml_vec_dot_f32 order), the shared gate (last WG), shared gate/up half tiles
// (WGs < 128: gate rows 16 tile + 4 half + i and the matching up rows) + swiglu
template <int NL>
FZ_PHASE bool phase_router(const RunCtl *ctl, const FusedArgs *ap, int il, int k) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, k);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    const FZ_CAS LayerDev &L = layer_of(c, il);
    auto &s = c.sm->router;
    const int t = threadIdx.x;
    const int b = c.b;
    const bool shg = b == c.G - 1;
    const bool gu = b < 2 * FFSH / 8;   // 128 half tiles
    const int tile = b >> 1, hf = b & 1;
    const float4 wrow = gldn((const float4 *)(L.router + (int64_t)b * E + 4 * t));
    float4 wsg = make_float4(0, 0, 0, 0);
    if (shg) wsg = gldn((const float4 *)(L.shexp_gate + 4 * t));
    WSlice<E, 2> ws;
    auto rowof = [&](int rl) { return (int64_t)(tile * 16 + (rl < 4 ? hf * 4 + rl : 8 + hf * 4 + (rl - 4))); };
    wload<E, 2>(ws, L.shexp_gu.q, L.shexp_gu.d, gu ? 8 : 0, rowof);
    const W8 nw = wload8(L.post_norm);
    {
        // element e = 4 t + q goes to chain e % 16, step e / 16
        const float wr[4] = {wrow.x, wrow.y, wrow.z, wrow.w}, gr[4] = {wsg.x, wsg.y, wsg.z, wsg.w};
#pragma unroll
        for (int q = 0; q < 4; q++) {
            const int e = 4 * t + q;
            s.w[e % 16][e / 16] = wr[q];
            if (shg) s.sg[e % 16][e / 16] = gr[q];
        }
    }
    const XR xr = make_xr(a.xbase, a.xbytes);
    if (!prologue<NL, true>(c.nl, c.ctl, nullptr, nullptr, a.xc.x1 + (size_t)c.par() * NL * E, c.tag(k, PH_OUT), c.err, nw,
                      a.m.eps, s.xf, &s.xq[0][0], E, &s.xd[0][0], E / 32, s.ns, s.xn, &c.ps->fail, &xr, [&] { tr_pass(c); }))
        return false;
    tr_mark(c, 131);
    {
        const int l = t >> 8, tt = t & 255;
        if (l < NL) {
            *(uint2 *)&c.ps->xq[l][8 * tt] = *(const uint2 *)&s.xq[l][8 * tt];
            if ((tt & 3) == 0) c.ps->xd[l][(8 * tt) / 32] = s.xd[l][(8 * tt) / 32];
        }
    }
    // f32 dots: lane c of a 16-lane group runs chain c (elements c + 16 q); xor 8, 4, 1, 2 is the
    // NEON reduction tree (vec.cpp:104-125)
    {
        // the normalised lanes, chain-major as well
        const int l = t >> 8, tt = t & 255;
        if (l < NL) {
#pragma unroll
            for (int q = 0; q < 8; q++) {
                const int e = 8 * tt + q;
                s.xc[l][e % 16][e / 16] = s.xn[l][e];
            }
        }
    }
    // f32 dots on wave 0 (measured: on a wave of their own beside the shared gate/up GEMV's chains,
    // the phase is no faster)
    auto f32_dots = [&]() {
        if (t < 64) {
            const int tw = t, l = (tw >> 4) & 1, cc = tw & 15;
            const bool sgd = tw >= 32;
            const float *wv = sgd ? s.sg[cc] : s.w[cc];
            const float *xv = s.xc[l][cc];
            float acc = 0.0f;
            if (!sgd || shg) acc = chain_fma<E / 16>(wv, xv);
            const float v = dot16_tree_f(acc);
            if (cc == 0 && l < c.nl) {
                if (!sgd) ll_stf(a.xc.lg + ((size_t)c.par() * NL + l) * NEXP + b, v, c.tag(k, PH_ROUTER));
                else if (shg) ll_stf(a.xc.sg + (size_t)c.par() * NL + l, sigmoid_t(v, exp_tab()), c.tag(k, PH_ROUTER));
            }
        }
    };
    __syncthreads();
    f32_dots();
    tr_mark(c, 132);
    if (gu) {
        wdot<E, 2, NL>(ws, 8, &s.xq[0][0], E, &s.xd[0][0], E / 32, s.g);
        if (t < NL * 4) {
            const int l = t / 4, i = t % 4;
            if (l < c.nl)
                ll_stf(a.xc.hsh + ((size_t)c.par() * NL + l) * FFSH + tile * 8 + hf * 4 + i,
                       v_silu(s.g.out[l][i]) * s.g.out[l][4 + i], c.tag(k, PH_ROUTER));
        }
    }
    tr_end(c, TP_ROUTER);
    return true;
}

// routing of every lane (each workgroup, from the published logits), then the routed experts'
// gate/up (group b = (union slot u = b / 16, 64-row group b % 16): 4 tiles = 32 h values per lane,
// one Q8_0 block), then the down projection + combine of rows [8 b, 8 b + 8), written to x of the
// next run layer
// il_next >= 0: once the down phase's inputs are in, the projection slice of layer il_next goes
// to pp
template <int NL>
FZ_PHASE bool phase_moe(const RunCtl *ctl, const FusedArgs *ap, int il, int k, int il_next, ProjPre &pp) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, k);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    const FZ_CAS LayerDev &L = layer_of(c, il);
    auto &se = c.sm->exp;
    auto &ps = *c.ps;
    const int t = threadIdx.x, b = c.b, nl = c.nl;
    const uint32_t trt = c.tag(k, PH_ROUTER), tet = c.tag(k, PH_EXP);
    // 1. routing (engine.rs:3414-3475) of the published logits; the post-norm quantised lanes are
    // this workgroup's own (router phase, persistent LDS)
    bool ok = true;
    if (t < NL * NEXP) {
        const int l = t / NEXP, i = t % NEXP;
        uint32_t u[1];
        ok = ll_gather<1, 0, false>([&](int) { return LLW{a.xc.lg + ((size_t)c.par() * NL + l) * NEXP + i, trt, l < nl}; }, u, c.err, nullptr);
        se.lg[l][i] = l < nl ? u2f(u[0]) : 0.0f;
    }
    if (t == 0) ps.ro.tie = 0;
    if (!all_ok(ok, &ps.fail)) return false;
    tr_pass(c);
    tr_mark(c, 105);
    // the next layer's projection slice is loaded in parts between the down phase's steps
    const bool pf = il_next >= 0;
    const FZ_CAS LayerDev &Ln = layer_of(c, pf ? il_next : il);
    const int pre_rows = proj_rows(Ln);
    if ((t >> 6) < nl) route_wave(se.lg[t >> 6], t >> 6, ps.ro);
    __syncthreads();
    tr_mark(c, 106);
    if (t < 64) {
        // union in first-use order (lane-major, engine.rs:3458-3475): entry t (lane t / 8, rank
        // t % 8) is new when no earlier entry names its expert; its union slot is the number of
        // new entries before its first occurrence
        const int e = t < nl * KUSED ? ps.ro.ids[t / KUSED][t % KUSED] : -1;
        int first = t;
#pragma unroll
        for (int u = NL * KUSED - 1; u >= 0; u--) {
            const int o = __builtin_amdgcn_readlane(e, u);
            first = (o == e && u < first) ? u : first;
        }
        const bool isnew = e >= 0 && first == t;
        const unsigned long long mask = __ballot(isnew);
        const int n = __popcll(mask);
        if (isnew) ps.uni[__popcll(mask & ((1ull << t) - 1))] = e;
        if (t < NL * KUSED) ps.slot[t / KUSED][t % KUSED] = e >= 0 ? __popcll(mask & ((1ull << first) - 1)) : 0;
        if (t == 0) ps.nu = n;
        if (b == 0 && t == 0) {
            if (ps.ro.tie) atomicAdd(a.b.counters + CNT_ERR_TIE, 1u);
            atomicAdd(a.b.counters + CNT_UNI_SUM, (uint32_t)n);
            atomicAdd(a.b.counters + CNT_EXP_CALLS, 1u);
        }
    }
    __syncthreads();
    const int nu = ps.nu < 0 ? 0 : (ps.nu > OXE_MAX_UNION ? OXE_MAX_UNION : ps.nu);
    tr_mark(c, 101);
    // 2. weight loads: this group's gate/up rows, and the down rows of every union expert + shared
    const bool gw = b < nu * 16;
    const int u_g = b >> 4, gq = b & 15;
    int e_g = gw ? ps.uni[u_g] : 0;
    e_g = e_g < 0 ? 0 : (e_g >= NEXP ? NEXP - 1 : e_g);
    WSlice<E, 16> ew;
    wload<E, 16>(ew, L.exp_gu.q + (int64_t)e_g * 2 * FF * E, L.exp_gu.d + (int64_t)e_g * 2 * FF * (E / 32), gw ? 64 : 0,
                 [&](int rl) { return (int64_t)(gq * 64 + rl); });
    // the down rows of every union expert and the shared expert (rows [8 b, 8 b + 8) of each unit):
    // the first DW_EARLY units per thread right behind the gate/up rows, the rest in the down phase
    // (measured: any issued here slow the gate/up stream more than they save). The weight loads are
    // unconditional (a load skipped on some path makes the compiler's wait for an earlier one
    // conservative, i.e. a wait for all): units past the union re-read the shared expert's rows.
    const int r0 = 8 * b;
    const int uh = t >> 8, rr = (t >> 5) & 7, ck = t & 31;
    auto unit_q = [&](int u) -> const int8_t * {
        int e = ps.uni[u < OXE_MAX_UNION ? u : 0];
        e = e < 0 ? 0 : (e >= NEXP ? NEXP - 1 : e);
        return u < nu && u < OXE_MAX_UNION ? L.exp_down.q + (int64_t)e * E * FF : L.shexp_down.q;
    };
    uint4 dw[9];
    auto dload = [&](int q) {
        dw[q] = gldn((const uint4 *)(unit_q(2 * q + uh) + (int64_t)(r0 + rr) * FF + 16 * ck));
    };
    const int su = t / 16 < DW_UNITS ? t / 16 : OXE_MAX_UNION, srr = (t % 16) / 2, shf = t % 2;
    uint4 dsc;
    auto sload = [&]() {
        int e = ps.uni[su < OXE_MAX_UNION ? su : 0];
        e = e < 0 ? 0 : (e >= NEXP ? NEXP - 1 : e);
        const uint16_t *base = su < nu && su < OXE_MAX_UNION ? L.exp_down.d + (int64_t)e * E * (FF / 32) : L.shexp_down.d;
        dsc = gldn((const uint4 *)(base + (int64_t)(r0 + srr) * (FF / 32) + shf * 8));
    };
    // measured best: none behind the gate / up rows, five of the nine before the inputs are polled
    constexpr int DW_EARLY = 0, DW_PRE = 5;
#pragma unroll
    for (int q = 0; q < DW_EARLY; q++) dload(q);
    if (DW_EARLY > 0) sload();
    tr_mark(c, 102);
    // 3. gate/up + swiglu + Q8_0 of the group's 32 h values per lane
    if (gw) {
        tr_mark(c, 103);
        wdot<E, 16, NL>(ew, 64, &ps.xq[0][0], E, &ps.xd[0][0], E / 32, se.g);
        tr_mark(c, 104);
        if (t < 64) {
            // swiglu of the group's 32 h values of lane l = t / 32 (half wave), then Q8_0
            static_assert(NL * 32 <= 64, "one wave");
            const int l = t / 32, i = t % 32, tl = i >> 3, r = i & 7;
            const float hv = l < NL ? v_silu(se.g.out[l < NL ? l : 0][tl * 16 + r]) * se.g.out[l < NL ? l : 0][tl * 16 + 8 + r] : 0.0f;
            float dd;
            const uint32_t word = quant32_lanes(hv, &dd);
            const size_t hi = ((size_t)c.par() * NL + (l < NL ? l : 0)) * OXE_MAX_UNION + u_g;
            if (l < nl && (i & 3) == 0) ll_st(a.xc.hq + hi * (FF / 4) + (gq * 32 + i) / 4, word, tet);
            if (l < nl && i == 0) ll_st(a.xc.hd + hi * (FF / 32) + gq, f2h(dd), tet);
        }
    }
    tr_end(c, TP_EXPERTS);
    tr_start(c);
    __syncthreads();   // the down phase's LDS aliases the experts'
    // down units [DW_EARLY, DW_PRE) issued before the phase's inputs are polled, the rest behind them
    // (a poll waits behind every load the thread has outstanding)
#pragma unroll
    for (int q = DW_EARLY; q < DW_PRE; q++) dload(q);
    if (DW_EARLY == 0) sload();
    // 4. down + combine (engine.rs:3542-3624). Inputs in the order they are published: the shared
    // expert's h (quantised here), the residual rows and the shared gate (router / out phases), then
    // the routed experts' quantised h of the union's live slots.
    auto &sd = c.sm->down;
    const size_t pl = (size_t)c.par() * NL;
    // this thread's inputs, latest producers first: the routed experts' h (4 codes per word; word
    // t + FT m of [lane][union slot][FF / 4], read coalesced) and its scale word t, then the shared
    // expert's h (element t of each lane), the residual row and the shared gate (t < NL * 8)
    constexpr int NHW = NL * OXE_MAX_UNION * (FF / 4) / FT;   // h words per thread
    static_assert(NL * OXE_MAX_UNION * (FF / 4) == NHW * FT && NL * OXE_MAX_UNION * (FF / 32) == FT, "word split");
    const int ld_ = t / (OXE_MAX_UNION * (FF / 32)), ud = (t / (FF / 32)) % OXE_MAX_UNION;
    const int tx = t < NL * 8 ? t : NL * 8 - 1;
    const bool xon = t < NL * 8 && tx / 8 < nl;
    // h word 2 (t + FT m) + h of [lane][union slot][FF / 4] is u[2 m + h]
    auto hwi = [&](int j) { return 2 * (t + FT * (j / 2)) + (j & 1); };
    auto hq_on = [&](int j) {
        const int i = hwi(j), q = i / (OXE_MAX_UNION * (FF / 4)), u = (i / (FF / 4)) % OXE_MAX_UNION;
        return q < nl && u < nu;
    };
    constexpr int NW = NHW + 1 + NL + 2;
    const XR xr = make_xr(a.xbase, a.xbytes);
    uint32_t u[NW];
    ok = ll_gather<NW, NHW / 2, true>(
        [&](int i) {
            if (i < NHW) return LLW{a.xc.hq + pl * OXE_MAX_UNION * (FF / 4) + hwi(i), tet, hq_on(i)};
            if (i == NHW) return LLW{a.xc.hd + (pl * OXE_MAX_UNION) * (FF / 32) + t, tet, ld_ < nl && ud < nu};
            if (i < NHW + 1 + NL) {
                const int l = i - NHW - 1;
                return LLW{a.xc.hsh + (pl + l) * FFSH + t, trt, l < nl};
            }
            if (i == NHW + 1 + NL) return LLW{a.xc.x1 + (pl + tx / 8) * E + r0 + tx % 8, c.tag(k, PH_OUT), xon};
            return LLW{a.xc.sg + pl + tx / 8, trt, xon};
        },
        u, c.err, &xr);
    const uint32_t hdv = u[NHW];
    float hsv[NL];
#pragma unroll
    for (int l = 0; l < NL; l++) hsv[l] = l < nl ? u2f(u[NHW + 1 + l]) : 0.0f;
    const float x1v = u2f(u[NHW + 1 + NL]), sgv = u2f(u[NHW + 2 + NL]);
#pragma unroll
    for (int q = DW_PRE; q < 9; q++) dload(q);
    if (pf) proj_load_part<0>(Ln, b, c.G, 0, pre_rows, pp);
    // Q8_0 of the shared expert's h: element t of lane l in thread t, a block per half wave
    static_assert(FFSH == FT, "one shared-expert element per thread and lane");
#pragma unroll
    for (int l = 0; l < NL; l++) {
        float dd;
        const uint32_t word = quant32_lanes(hsv[l], &dd);
        if ((t & 3) == 0) *(uint32_t *)&sd.hq[l][OXE_MAX_UNION][t] = word;
        if ((t & 31) == 0) sd.hd[l][OXE_MAX_UNION][t / 32] = f2h(dd);
    }
#pragma unroll
    for (int m = 0; m < NHW; m++) {
        const int i = hwi(m), q = i / (OXE_MAX_UNION * (FF / 4)), uu = (i / (FF / 4)) % OXE_MAX_UNION;
        ((uint32_t *)&sd.hq[q][uu][0])[i % (FF / 4)] = hq_on(m) ? u[m] : 0u;
    }
    sd.hd[ld_][ud][t % (FF / 32)] = (uint16_t)hdv;
    if (!all_ok(ok, &ps.fail)) return false;
    tr_pass(c);
    if (pf) proj_load_part<1>(Ln, b, c.G, 0, pre_rows, pp);
    tr_mark(c, 161);
    if (t < DW_UNITS * 16) {
        // scale products of (unit su, row srr, blocks [8 shf, 8 shf + 8)) for every lane
        const uint32_t sw[4] = {dsc.x, dsc.y, dsc.z, dsc.w};
#pragma unroll
        for (int l = 0; l < NL; l++) {
            float dv[8];
#pragma unroll
            for (int q = 0; q < 8; q++)
                dv[q] = h2f(sd.hd[l][su][8 * shf + q]) * h2f((uint16_t)(sw[q / 2] >> (16 * (q & 1))));
            *(float4 *)&sd.d[su][l][srr][8 * shf] = make_float4(dv[0], dv[1], dv[2], dv[3]);
            *(float4 *)&sd.d[su][l][srr][8 * shf + 4] = make_float4(dv[4], dv[5], dv[6], dv[7]);
        }
    }
    // branch-free but for the one unit slot past DW_UNITS (uniform per wave), so the dots interleave:
    // units past the union dot zeros with the shared expert's rows (never read); both lanes of a pair
    // hold the block's sum and store it to the same word
#pragma unroll
    for (int q = 0; q < 9; q++) {
        const int u = 2 * q + uh;
        if (2 * q + 1 < DW_UNITS || u < DW_UNITS) {
#pragma unroll
            for (int l = 0; l < NL; l++) {
                const uint4 xa = *(const uint4 *)&sd.hq[l][u][16 * ck];
                int32_t v = dot16(dw[q], xa, 0);
                v += dpp_i<DPP_XOR1>(v);
                sd.f[u][l][rr][ck >> 1] = (float)v;
            }
        }
    }
    __syncthreads();
    if (pf) proj_load_part<2>(Ln, b, c.G, 0, pre_rows, pp);
    tr_mark(c, 162);
    if (t < DW_UNITS * NL * 8) {
        const int u = t / (NL * 8), l = (t / 8) % NL, r = t % 8;
        if (u == OXE_MAX_UNION || u < nu) {
            const float *fr = &sd.f[u][l][r][0], *dr = &sd.d[u][l][r][0];
            float acc = 0.0f;
#pragma unroll
            for (int bb = 0; bb < FF / 32; bb += 4) {
                const float4 f4 = *(const float4 *)(fr + bb), d4 = *(const float4 *)(dr + bb);
                acc = __builtin_fmaf(f4.x, d4.x, acc);
                acc = __builtin_fmaf(f4.y, d4.y, acc);
                acc = __builtin_fmaf(f4.z, d4.z, acc);
                acc = __builtin_fmaf(f4.w, d4.w, acc);
            }
            sd.dn[u][l][r] = acc;
        }
    }
    __syncthreads();
    if (pf) proj_load_part<3>(Ln, b, c.G, 0, pre_rows, pp);
    tr_mark(c, 163);
    if (t < NL * 8) {
        const int l = t / 8, r = t % 8;
        if (l < nl) {
            float m = sd.dn[ps.slot[l][0]][l][r] * ps.ro.w[l][0];
            for (int j = 1; j < KUSED; j++) {
                const float p = sd.dn[ps.slot[l][j]][l][r] * ps.ro.w[l][j];
                m = m + p;
            }
            const float sh = sd.dn[OXE_MAX_UNION][l][r] * sgv;
            const float f = m + sh;
            ll_stf(a.xc.x + ((size_t)((k + 1) & 1) * NL + l) * E + r0 + r, f + x1v, c.tag(k, PH_DOWN));
        }
    }
    tr_end(c, TP_DOWN);
    return true;
}

// attention scores (workgroup = kv head x 128 positions) with the query prologue (q_norm, RoPE,
// f16) and the run's own K rows computed in place (k_norm, RoPE); the workgroup whose range holds
// a new position writes its K cache row
OXE_DEV uint16_t *kcache_layer(const FZ_CAS FusedArgs &a, const FZ_CAS LayerDev &L) {
    return a.m.kcache + (int64_t)L.index * NKV * a.m.n_ctx * HD;
}

typedef _Float16 h2t __attribute__((ext_vector_type(2)));
OXE_DEV h2t u2h2f(uint32_t u) { return __builtin_bit_cast(h2t, u); }
OXE_DEV uint32_t h22uf(h2t v) { return __builtin_bit_cast(uint32_t, v); }
OXE_DEV float f16x8_reduce_q(h2t acc[4]) {
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = acc[i] + u2h2f((uint32_t)dpp_i<DPP_XOR2>((int)h22uf(acc[i])));
#pragma unroll
    for (int i = 0; i < 4; i++) acc[i] = acc[i] + u2h2f((uint32_t)dpp_i<DPP_XOR1>((int)h22uf(acc[i])));
    const float t0 = (float)acc[0].x + (float)acc[2].x;
    const float t1 = (float)acc[0].y + (float)acc[2].y;
    const float t2 = (float)acc[1].x + (float)acc[3].x;
    const float t3 = (float)acc[1].y + (float)acc[3].y;
    return (t0 + t1) + (t2 + t3);
}


template <int NL>
FZ_PHASE bool phase_scores(const RunCtl *ctl, const FusedArgs *ap, int il, int k, bool seed_only) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, k);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    const FZ_CAS LayerDev &L = layer_of(c, il);
    auto &s = c.sm->sc;
    const int t = threadIdx.x, w = t >> 6, lane = t & 63, nl = c.nl;
    const int pos0 = c.ctl->pos0, pmax = pos0 + nl - 1;
    // workgroup (kvh, chunk0) takes position chunks chunk0, chunk0 + G / 2, ... (16 positions each)
    const int kvh = c.b % NKV, cstride = c.G / NKV, chunk0 = c.b / NKV;
    const bool act = chunk0 * SC_P <= pmax;
    // the first chunk's cached K rows (positions < pos0): thread = (position t / 32, 16-byte part)
    const uint16_t *kcl = kcache_layer(a, L) + (int64_t)kvh * a.m.n_ctx * HD;
    const int kp = t >> 5, kpart = t & 31;
    uint4 kpre = make_uint4(0, 0, 0, 0);
    if (act && !seed_only && chunk0 * SC_P + kp < pos0) kpre = gldn((const uint4 *)(kcl + (int64_t)(chunk0 * SC_P + kp) * HD + 8 * kpart));
    // per wave, its vectors' norm weights and RoPE rows (read-only), before the barrier
    const int kjob = w;                          // waves 0..NL-1: K row of lane w
    const int pk = pos0 + kjob;
    const int pkc = pk / SC_P;                   // the chunk holding position pk
    const bool kdo = act && kjob < nl && pkc >= chunk0 && (pkc - chunk0) % cstride == 0;
    const bool qdo = act && !seed_only;
    float kw[4], qw[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        kw[i] = kdo ? L.k_norm[lane + 64 * i] : 0.0f;
        qw[i] = qdo ? L.q_norm[lane + 64 * i] : 0.0f;
    }
    const int rl = lane & (NROT / 2 - 1);
    float kcs[2] = {0.0f, 0.0f}, qcs[(NL * GQA + 7) / 8][2];
    if (kdo) { kcs[0] = a.m.rope[(int64_t)pk * NROT + 2 * rl]; kcs[1] = a.m.rope[(int64_t)pk * NROT + 2 * rl + 1]; }
#pragma unroll
    for (int q = 0; q < (NL * GQA + 7) / 8; q++) {
        const int l = (w + 8 * q) / GQA;
        const bool on = qdo && w + 8 * q < NL * GQA && l < nl;
        qcs[q][0] = on ? a.m.rope[(int64_t)(pos0 + l) * NROT + 2 * rl] : 0.0f;
        qcs[q][1] = on ? a.m.rope[(int64_t)(pos0 + l) * NROT + 2 * rl + 1] : 0.0f;
    }
    // each wave takes its vectors (the K row of lane w on waves w < NL in range; queries job
    // w + 8 q = (lane job / 8, head job % 8)) through raw -> rms norm * weight -> RoPE -> f16 on
    // its own: lane c holds elements c + 64 i; RoPE pairs (c, c + 32) for c < 32 (slot 0)
    const uint64_t *pin = a.xc.p + (size_t)c.par() * NL * DN_ROWS;
    const uint32_t tp = c.tag(k, PH_PROJ);
    constexpr int NQJ = (NL * GQA + 7) / 8;
    float kv4[4], qv4[NQJ][4];
    {
        // the query rows of this wave's jobs and the K row, 4 words each (elements lane + 64 i)
        uint32_t u[4 * NQJ + 4];
        const bool ok = ll_gather<4 * NQJ + 4, 0, true>(
            [&](int i) {
                const int q = i / 4, e = lane + 64 * (i % 4);
                if (q < NQJ) {
                    const int job = w + 8 * q, l = (job / GQA) % NL, h = kvh * GQA + job % GQA;
                    return LLW{pin + (int64_t)l * DN_ROWS + h * 2 * HD + e, tp, qdo && job < NL * GQA && job / GQA < nl};
                }
                return LLW{pin + (int64_t)(kjob % NL) * DN_ROWS + AT_K + kvh * HD + e, tp, kdo};
            },
            u, c.err, nullptr);
#pragma unroll
        for (int q = 0; q < NQJ; q++)
#pragma unroll
            for (int i = 0; i < 4; i++) qv4[q][i] = u2f(u[4 * q + i]);
#pragma unroll
        for (int i = 0; i < 4; i++) kv4[i] = u2f(u[4 * NQJ + i]);
        if (!all_ok(ok, &c.ps->fail)) return false;
    }
    tr_pass(c);
    auto finish = [&](float v[4], const float wt[4], const float cs[2], float *replay, uint16_t *dst) {
#pragma unroll
        for (int i = 0; i < 4; i++) replay[lane + 64 * i] = v[i];
        const float mean = wave_mean_sq_256(v, replay);
        const float scale = 1.0f / sqrtf(mean + a.m.eps);
#pragma unroll
        for (int i = 0; i < 4; i++) v[i] = (v[i] * scale) * wt[i];
        const float o = __shfl_xor(v[0], NROT / 2, 64);
        if (lane < NROT / 2) v[0] = __builtin_fmaf(v[0], cs[0], -(o * cs[1]));
        else if (lane < NROT) v[0] = __builtin_fmaf(o, cs[1], v[0] * cs[0]);
#pragma unroll
        for (int i = 0; i < 4; i++) dst[lane + 64 * i] = f2h(v[i]);
    };
    if (kdo) {
        finish(kv4, kw, kcs, s.ktmp[kjob], s.knew[kjob]);
        uint16_t *kc = kcache_layer(a, L);
#pragma unroll
        for (int i = 0; i < 4; i++) kc[((int64_t)kvh * a.m.n_ctx + pk) * HD + lane + 64 * i] = s.knew[kjob][lane + 64 * i];
    }
#pragma unroll
    for (int q = 0; q < (NL * GQA + 7) / 8; q++) {
        const int job = w + 8 * q, l = job / GQA;
        if (qdo && job < NL * GQA) {
            if (l < nl) finish(qv4[q], qw, qcs[q], s.tmp[job], s.q[job]);
            else
#pragma unroll
                for (int i = 0; i < 4; i++) s.q[job][lane + 64 * i] = 0;
        }
    }
    __syncthreads();
    tr_mark(c, 151);
    if (act && !seed_only) {
        // thread = (lane l, head pair hq, position pp of the chunk, chain quad j). Positions of a
        // chunk past the lane's own (masked in the softmax) get the tag with value 0, so the
        // softmax polls whole groups of 4.
        const int l = t >> 8, hq = (t >> 6) & 3, pp = (t >> 2) & (SC_P - 1), j = t & 3;
        uint64_t *scx = a.xc.sc + ((size_t)c.par() * NL + (l < NL ? l : 0)) * NH * a.m.n_ctx;
        const uint32_t ts = c.tag(k, PH_MIX);
        for (int chunk = chunk0; chunk * SC_P <= pmax; chunk += cstride) {
            const int cb = chunk * SC_P;
            if (chunk == chunk0) {
                if (cb + kp < pos0) *(uint4 *)&s.krows[kp][8 * kpart] = kpre;
            } else if (cb + kp < pos0) {
                *(uint4 *)&s.krows[kp][8 * kpart] = gldn((const uint4 *)(kcl + (int64_t)(cb + kp) * HD + 8 * kpart));
            }
            __syncthreads();
            const int p = cb + pp;
            if (l < nl && p <= pos0 + l) {
                const uint16_t *krow = p < pos0 ? s.krows[pp] : s.knew[p - pos0];
                h2t acc[2][4];
#pragma unroll
                for (int q = 0; q < 2; q++)
#pragma unroll
                    for (int i = 0; i < 4; i++) acc[q][i] = h2t{(_Float16)0.0f, (_Float16)0.0f};
#pragma unroll
                for (int sx = 0; sx < HD / 32; sx++) {
                    const uint4 kv = *(const uint4 *)(krow + 32 * sx + 8 * j);
                    const h2t k0 = u2h2f(kv.x), k1 = u2h2f(kv.y), k2 = u2h2f(kv.z), k3 = u2h2f(kv.w);
#pragma unroll
                    for (int q = 0; q < 2; q++) {
                        const uint4 qv = *(const uint4 *)(&s.q[l * GQA + 2 * hq + q][32 * sx + 8 * j]);
                        acc[q][0] = __builtin_elementwise_fma(k0, u2h2f(qv.x), acc[q][0]);
                        acc[q][1] = __builtin_elementwise_fma(k1, u2h2f(qv.y), acc[q][1]);
                        acc[q][2] = __builtin_elementwise_fma(k2, u2h2f(qv.z), acc[q][2]);
                        acc[q][3] = __builtin_elementwise_fma(k3, u2h2f(qv.w), acc[q][3]);
                    }
                }
#pragma unroll
                for (int q = 0; q < 2; q++) {
                    const float sc = f16x8_reduce_q(acc[q]);
                    if (j == 0) ll_stf(scx + (int64_t)(kvh * GQA + 2 * hq + q) * a.m.n_ctx + p, sc, ts);
                }
            } else if (l < nl && j == 0 && p < a.m.n_ctx) {
#pragma unroll
                for (int q = 0; q < 2; q++) ll_stf(scx + (int64_t)(kvh * GQA + 2 * hq + q) * a.m.n_ctx + p, 0.0f, ts);
            }
            __syncthreads();
        }
    }
    tr_end(c, TP_SCORES);
    return true;
}

// Attention output (k_attn.hip pv_kernel's arithmetic): workgroup (kv head kvh, lane l, 16-dim
// chunk, head pair hp) for heads 2 hp, 2 hp + 1 of the GQA group; 256 workgroups. Head q of the
// pair is handled by waves 4 q .. 4 q + 3: its softmax (oxe_soft_max_f32, oxe_ops.cpp:101-115)
// in one pass over its scores held in registers (up to PV_SMK groups of 4 positions per thread;
// longer rows take three passes), max and group-sum total combined over the four waves. The
// chunk's V^T rows (16 dims x n_kv) are staged in LDS: 16-byte chunks holding only positions of
// earlier launches are loaded before the barrier, the rest after it, device-coherently. Thread
// (q = t / 256, dim d = (t / 16) % 16, cp = t % 16) runs chain pair cp of ggml_vec_dot_f16
// (positions 32 s + 2 cp and +1: accumulator cp / 4, halves 2 (cp % 4) and +1) for dim d and head
// q; the F16x8 reduce is done by lane moves inside the 16-lane row. The V^T entries of this run's
// own positions are taken from the projection outputs (f16 of the f32 V rows, the value the
// projection phase writes to V^T for later runs); every other entry is the cache's. The gated
// outputs (f32) go to the mixer-output buffer; the output projection quantizes them.
constexpr int PV_SMK = 2;    // softmax groups per thread in registers (n_kv <= 2048)
constexpr int PVD = 16;      // dims per workgroup
constexpr int PV_HP = GQA / 2;  // head pairs per kv head
constexpr int PV_VK = 4;     // V^T 16-byte chunks per thread staged from registers (n_kv <= 1024)
constexpr int PV_VMAX = 2048;   // positions of the V^T tile held in LDS (longer rows: the rest from memory)

template <int NL>
FZ_PHASE bool phase_pv(const RunCtl *ctl, const FusedArgs *ap, int il, int k) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, k);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    const FZ_CAS LayerDev &L = layer_of(c, il);
    const int t = threadIdx.x, nl = c.nl;
    constexpr int NCH = HD / PVD;
    const int hp = c.b % PV_HP;
    const int dchunk = (c.b / PV_HP) % NCH;
    const int l = (c.b / (PV_HP * NCH)) % NL;
    const int kvh = c.b / (PV_HP * NCH * NL);
    const bool act = kvh < NKV && l < nl;
    const int n_ctx = a.m.n_ctx;
    const int pos0 = c.ctl->pos0, pos = pos0 + l;
    int n_kv = (pos + 1 + 255) / 256 * 256;
    if (n_kv < 256) n_kv = 256;
    if (n_kv > n_ctx) n_kv = n_ctx;
    const int ns = n_kv / 32;
    const int nst = n_kv < PV_VMAX ? n_kv : PV_VMAX;   // positions staged in LDS
    const int nvc = nst / 8;                            // staged 16-byte chunks per V^T row
    const int vs = nst + 32;                            // LDS row stride in halves
    const uint16_t *vt = a.m.vcache + (int64_t)L.index * NKV * HD * n_ctx + (int64_t)(kvh * HD + dchunk * PVD) * n_ctx;
    // staged chunk i = t + FT q: row i / nvc, chunk i % nvc (this run's positions are patched in
    // LDS afterwards)
    uint4 vpre[PV_VK];
#pragma unroll
    for (int q = 0; q < PV_VK; q++) {
        const int i = t + FT * q, r = i / nvc, ch = i % nvc;
        vpre[q] = (act && i < PVD * nvc) ? gldn((const uint4 *)(vt + (int64_t)r * n_ctx + 8 * ch)) : make_uint4(0, 0, 0, 0);
    }
    const uint64_t *pin = a.xc.p + (size_t)c.par() * NL * DN_ROWS;
    const uint32_t tp = c.tag(k, PH_PROJ), ts = c.tag(k, PH_MIX);
    if (act) {
        // byte offsets from the LDS base (pointer arithmetic only: an integer round trip would lose
        // the LDS address space, and generic accesses wait for every memory operation in flight)
        const size_t o_v = (size_t)n_ctx * 4, o_mx = o_v + (size_t)PVD * vs * 2;
        const size_t o_ps = (o_mx + 8 * sizeof(float) + 7) & ~(size_t)7, o_f = o_ps + 8 * sizeof(double);
        uint32_t *s_pp = (uint32_t *)c.dyn;                                  // [n_kv / 2][2] f16 pairs
        uint16_t *s_v = (uint16_t *)(c.dyn + o_v);                          // [PVD][vs] V^T rows
        float *s_mx = (float *)(c.dyn + o_mx);                              // [2][4] wave maxima
        double *s_ps = (double *)(c.dyn + o_ps);                            // [2][4] wave sums
        float *s_f = (float *)(c.dyn + o_f);                                // [2] 1 / sum
        uint16_t *s_vn = (uint16_t *)(c.dyn + o_f + 2 * sizeof(float));     // [NL][PVD] this run's V
        const int q = t >> 8, tq = t & 255, wq = (t >> 6) & 3;
        const int cp = t & 15, d = (t >> 4) & (PVD - 1);
        const int h = kvh * GQA + 2 * hp + q;
        // the scores of head q: groups of 4 positions up to the one holding pos (the scores phase
        // tags every position of its chunks); later groups are masked and not read
        const uint64_t *sc = a.xc.sc + ((size_t)c.par() * NL + l) * NH * n_ctx + (int64_t)h * n_ctx;
        auto sget = [&](int g, uint32_t (&u)[4]) -> bool {
            return ll_gather<4, 0, false>([&](int i) { return LLW{sc + 4 * g + i, ts, 4 * g <= pos}; }, u, c.err, nullptr);
        };
        const int ng = n_kv / 4;
        const bool shortrow = ng <= 256 * PV_SMK;
        // this thread's scores of head q (short rows: positions tq + 256 j, read coalesced and staged
        // in LDS, where the V^T tile goes later), this run's V entries of the chunk's 16 dims
        // (t < NL * PVD) and this thread's gate, in one gather
        constexpr int NSC = 4 * PV_SMK;
        float *s_raw = (float *)s_v;                                        // [2][n_kv] staged scores
        const int vl = (t / PVD) % NL, vd = t % PVD;
        // position 2 (tq + 256 m) + h is u0[2 m + h]; a pair is wanted when its first position is
        auto pi = [&](int i) { return 2 * (tq + 256 * (i / 2)) + (i & 1); };
        const XR xr = make_xr(a.xbase, a.xbytes);
        uint32_t u0[NSC + 2];
        bool ok = ll_gather<NSC + 2, NSC / 2, true>(
            [&](int i) {
                if (i < NSC) {
                    const int p0 = pi(i & ~1);
                    return LLW{sc + pi(i), ts, shortrow && p0 < n_kv && p0 <= pos};
                }
                if (i == NSC)
                    return LLW{pin + (int64_t)vl * DN_ROWS + AT_V + kvh * HD + dchunk * PVD + vd, tp, t < NL * PVD && vl < nl};
                return LLW{pin + (int64_t)l * DN_ROWS + h * 2 * HD + HD + dchunk * PVD + d, tp, cp == 0};
            },
            u0, c.err, &xr);
        if (shortrow)
#pragma unroll
            for (int i = 0; i < NSC; i++) {
                const int p = pi(i);
                if (p < n_kv) s_raw[q * n_kv + p] = u2f(u0[i]);
            }
        if (t < NL * PVD) s_vn[vl * PVD + vd] = f2h(vl < nl ? u2f(u0[NSC]) : 0.0f);
        float sg = cp == 0 ? u2f(u0[NSC + 1]) : 0.0f;
        const float scale = 1.0f / sqrtf((float)HD);
        {
            // softmax of head q: wp = s * scale (masked: -inf), max, e = v_expf(wp - max) with group
            // sums (e0 + e1) + (e2 + e3) added in double, p = f16(e * f32(1 / sum))
            auto wval = [&](uint32_t u, int p) { return p <= pos ? __builtin_bit_cast(float, u) * scale : -__builtin_inff(); };
            auto group = [&](int g, float mx) {
                uint32_t u[4];
                (void)sget(g, u);   // polled before (the same groups, first pass)
                const uint4 v = make_uint4(u[0], u[1], u[2], u[3]);
                const float e0 = v_expf(wval(v.x, 4 * g) - mx), e1 = v_expf(wval(v.y, 4 * g + 1) - mx);
                const float e2 = v_expf(wval(v.z, 4 * g + 2) - mx), e3 = v_expf(wval(v.w, 4 * g + 3) - mx);
                return (e0 + e1) + (e2 + e3);
            };
            // max over the head's four waves (LDS), then the group-sum total
            auto head_max = [&](float m) {
                m = wave_max_any(m);
                if ((t & 63) == 0) s_mx[q * 4 + wq] = m;
                __syncthreads();
                const float m01 = s_mx[q * 4] > s_mx[q * 4 + 1] ? s_mx[q * 4] : s_mx[q * 4 + 1];
                const float m23 = s_mx[q * 4 + 2] > s_mx[q * 4 + 3] ? s_mx[q * 4 + 2] : s_mx[q * 4 + 3];
                return m01 > m23 ? m01 : m23;
            };
            auto head_recip = [&](double part, float mx) {
                part = wave_sum_d_any(part);
                if ((t & 63) == 0) s_ps[q * 4 + wq] = part;
                __syncthreads();
                const double P = (s_ps[q * 4] + s_ps[q * 4 + 1]) + (s_ps[q * 4 + 2] + s_ps[q * 4 + 3]);
                float f;
                const bool ok = bracket_ok_recip(P, P, ng, &f);
                if (!ok && tq == 0) {
                    // the reference's sequential double sum of the group sums (rare: the parallel
                    // sum's bracket straddles a rounding edge), recomputed from the scores
                    double sum = 0.0;
                    for (int g = 0; g < ng; g++) sum += (double)group(g, mx);
                    s_f[q] = (float)(1.0 / sum);
                }
                __syncthreads();   // every wave of the workgroup (both heads) reaches it
                if (!ok) f = s_f[q];
                return f;
            };
            float mx = -__builtin_inff();
            double part = 0.0;
            if (shortrow) {
                if (!all_ok(ok, &c.ps->fail)) return false;
                tr_pass(c);
                float e[PV_SMK][4];
#pragma unroll
                for (int k2 = 0; k2 < PV_SMK; k2++) {
                    const int g = tq + 256 * k2;
                    float4 f = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                    if (g < ng) f = *(const float4 *)&s_raw[q * n_kv + 4 * g];
                    const float fr[4] = {f.x, f.y, f.z, f.w};
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        e[k2][i] = g < ng ? wval(__builtin_bit_cast(uint32_t, fr[i]), 4 * g + i) : -__builtin_inff();
                        mx = (mx > e[k2][i]) ? mx : e[k2][i];
                    }
                }
                mx = head_max(mx);
                tr_mark(c, 143);
#pragma unroll
                for (int k2 = 0; k2 < PV_SMK; k2++) {
                    const int g = tq + 256 * k2;
                    if (g < ng) {
#pragma unroll
                        for (int i = 0; i < 4; i++) e[k2][i] = v_expf(e[k2][i] - mx);
                        part += (double)((e[k2][0] + e[k2][1]) + (e[k2][2] + e[k2][3]));
                    }
                }
                const float f = head_recip(part, mx);
#pragma unroll
                for (int k2 = 0; k2 < PV_SMK; k2++) {
                    const int g = tq + 256 * k2;
                    if (g < ng) {
                        s_pp[(2 * g) * 2 + q] = (uint32_t)f2h(e[k2][0] * f) | ((uint32_t)f2h(e[k2][1] * f) << 16);
                        s_pp[(2 * g + 1) * 2 + q] = (uint32_t)f2h(e[k2][2] * f) | ((uint32_t)f2h(e[k2][3] * f) << 16);
                    }
                }
            } else {
                // long rows: max, sums and probabilities in three passes over the scores
                for (int g = tq; g < ng; g += 256) {
                    uint32_t u[4];
                    ok = sget(g, u) && ok;
#pragma unroll
                    for (int i = 0; i < 4; i++) {
                        const float wv = wval(u[i], 4 * g + i);
                        mx = (mx > wv) ? mx : wv;
                    }
                }
                if (!all_ok(ok, &c.ps->fail)) return false;
                tr_pass(c);
                mx = head_max(mx);
                for (int g = tq; g < ng; g += 256) part += (double)group(g, mx);
                const float f = head_recip(part, mx);
                for (int g = tq; g < ng; g += 256) {
                    uint32_t u[4];
                    (void)sget(g, u);
                    uint16_t pq[4];
#pragma unroll
                    for (int i = 0; i < 4; i++) pq[i] = f2h(v_expf(wval(u[i], 4 * g + i) - mx) * f);
                    s_pp[(2 * g) * 2 + q] = (uint32_t)pq[0] | ((uint32_t)pq[1] << 16);
                    s_pp[(2 * g + 1) * 2 + q] = (uint32_t)pq[2] | ((uint32_t)pq[3] << 16);
                }
            }
        }
        tr_mark(c, 144);
        // the V^T tile into LDS, then this run's positions patched in
#pragma unroll
        for (int q2 = 0; q2 < PV_VK; q2++) {
            const int i = t + FT * q2, r = i / nvc, ch = i % nvc;
            if (i < PVD * nvc) *(uint4 *)(s_v + r * vs + 8 * ch) = vpre[q2];
        }
        for (int i = t + FT * PV_VK; i < PVD * nvc; i += FT) {
            const int r = i / nvc, ch = i % nvc;
            *(uint4 *)(s_v + r * vs + 8 * ch) = gldn((const uint4 *)(vt + (int64_t)r * n_ctx + 8 * ch));
        }
        if (cp == 0) sg = sigmoid_t(sg, exp_tab());
        __syncthreads();
        if (t < NL * PVD) {
            const int vl = t / PVD, vd = t % PVD;
            if (vl < nl && pos0 + vl < nst) s_v[vd * vs + pos0 + vl] = s_vn[vl * PVD + vd];
        }
        __syncthreads();
        tr_mark(c, 141);
        // V^T . p for dim d, chain pair cp, head q
        h2t acc = h2t{(_Float16)0.0f, (_Float16)0.0f};
        const uint16_t *vrow = s_v + d * vs + 2 * cp;
        const uint32_t *prow = s_pp + cp * 2 + q;
        const int nss = nst / 32;
#pragma unroll 8
        for (int s = 0; s < nss; s++)
            acc = __builtin_elementwise_fma(u2h2f(*(const uint32_t *)(vrow + 32 * s)), u2h2f(prow[32 * s]), acc);
        for (int s = nss; s < ns; s++) {
            const int p0 = 32 * s + 2 * cp;
            uint32_t vw = gldn((const uint32_t *)(vt + (int64_t)d * n_ctx + p0));
            // this run's positions from the projection outputs
            if (p0 >= pos0 && p0 < pos0 + nl) vw = (vw & 0xffff0000u) | s_vn[(p0 - pos0) * PVD + d];
            if (p0 + 1 >= pos0 && p0 + 1 < pos0 + nl) vw = (vw & 0xffffu) | ((uint32_t)s_vn[(p0 + 1 - pos0) * PVD + d] << 16);
            acc = __builtin_elementwise_fma(u2h2f(vw), u2h2f(prow[32 * s]), acc);
        }
        // GGML_F16x8_REDUCE: accumulator j += j ^ 2 (cp ^ 8), j += j ^ 1 (cp ^ 4); widen halves
        // (h0 + h4, h1 + h5 | h2 + h6, h3 + h7) and vaddvq ((t0 + t1) + (t2 + t3))
        h2t x = acc;
        x = x + u2h2f((uint32_t)dpp_i<DPP_ROR8>((int)h22uf(x)));
        x = x + u2h2f((uint32_t)dpp_i<DPP_ROR4>((int)h22uf(x)));
        const float lo = (float)x.x, hi = (float)x.y;
        const float tlo = lo + dpp_f<DPP_XOR2>(lo), thi = hi + dpp_f<DPP_XOR2>(hi);
        const float s2 = tlo + thi;
        const float out = s2 + dpp_f<DPP_XOR1>(s2);
        tr_mark(c, 142);
        if (cp == 0) ll_stf(a.xc.g + ((size_t)c.par() * NL + l) * MIX_W + h * HD + dchunk * PVD + d, out * sg, c.tag(k, PH_PV));
    }
    tr_end(c, TP_PV);
    return true;
}

// MTP entry: eh_proj . [enorm(embd(tok)); hnorm(h)], rows [8 b, 8 b + 8), written as the "down"
// output of run layer 0 (the input x of the MTP layer, run layer 1)
template <int NL>
FZ_PHASE bool phase_entry(const RunCtl *ctl, const FusedArgs *ap, int il) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, 0);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    const FZ_CAS LayerDev &L = layer_of(c, il);
    auto &s = c.sm->entry;
    const int t = threadIdx.x, r0 = 8 * c.b;
    WSlice<2 * E, 4> ws;
    wload<2 * E, 4>(ws, L.eh_proj.q, L.eh_proj.d, 8, [&](int rl) { return (int64_t)(r0 + rl); });
    const W8 nwe = wload8(L.enorm), nwh = wload8(L.hnorm);
    // the entry's inputs come from earlier launches (nothing to poll)
    (void)prologue<NL>(c.nl, c.ctl, a.m.tok_embd.q, a.m.tok_embd.d, nullptr, 0u, c.err, nwe, a.m.eps, s.xf, &s.xq[0][0], 2 * E,
                       &s.xd[0][0], 2 * E / 32, s.ns, nullptr, &c.ps->fail);
    {
        // h of each lane: hid[hin_sel[l]]
        const int l = t >> 8, tt = t & 255;
        float v[8];
        if (l < NL && l < c.nl) get8(a.b.hid + (int64_t)lane_pick<NL>(c.ctl->hin_sel, l) * E + 8 * tt, v);
        else
            for (int i = 0; i < 8; i++) v[i] = 0.0f;
        if (l < NL) put8(&s.xf[l][8 * tt], v);
        __syncthreads();
        norm8(v, s.xf[l < NL ? l : 0], nwh.v, a.m.eps, s.ns);
        if (l < NL) {
            if (l < c.nl) quant8(v, &s.xq[l][E + 8 * tt], &s.xd[l][(E + 8 * tt) / 32]);
            else {
                *(uint2 *)&s.xq[l][E + 8 * tt] = make_uint2(0, 0);
                if ((tt & 3) == 0) s.xd[l][(E + 8 * tt) / 32] = 0;
            }
        }
        __syncthreads();
    }
    wdot<2 * E, 4, NL>(ws, 8, &s.xq[0][0], 2 * E, &s.xd[0][0], 2 * E / 32, s.g);
    if (t < NL * 8) {
        const int l = t / 8, rl = t % 8;
        if (l < c.nl) ll_stf(a.xc.x + ((size_t)1 * NL + l) * E + r0 + rl, s.g.out[l][rl], c.tag(0, PH_DOWN));
    }
    tr_end(c, TP_ENTRY);
    return true;
}

// output norm + LM head + per-workgroup argmax keys (first strict maximum, NaN never wins)
OXE_DEV uint32_t ordered_bits_f(float f) {
    const uint32_t u = __builtin_bit_cast(uint32_t, f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// k: the run layer after the last (its input x is the head's input)
template <int NL>
FZ_PHASE bool phase_head(const RunCtl *ctl, const FusedArgs *ap, const float *norm_w, int k) {
    Ctx<NL> c = make_ctx<NL>(ctl, ap, k);
    tr_start(c);
    const FZ_CAS FusedArgs &a = *c.a;
    auto &s = c.sm->head;
    const int t = threadIdx.x, nl = c.nl, mask = c.ctl->head_mask;
    const int64_t V = a.head_w.rows;
    constexpr int TR = HEAD_TR;                              // rows per tile
    const int64_t ntiles = (V + TR - 1) / TR;
    // Tiles: `per` (even) in a contiguous range per workgroup, then pairs of the remaining tiles
    // claimed from a counter, so the workgroups that stream faster take more of the tail (the HBM
    // gives some XCDs' CUs less than others). Fewer than 4 tiles per workgroup: a static split only.
    constexpr int64_t STATIC_PCT = 90;   // share of the tiles split statically (measured best)
    const int64_t per = 2 * ((ntiles * STATIC_PCT / 100) / (2 * c.G));
    const bool dyn = per >= 4;
    const int64_t t0 = dyn ? per * c.b : ntiles * c.b / c.G, t1 = dyn ? t0 + per : ntiles * (c.b + 1) / c.G;
    WSlice<E, HEAD_P> A, B;
    auto rows_of = [&](int64_t tile) { const int64_t r = V - tile * TR; return (int)(r < TR ? r : TR); };
    if (t0 < t1) wload<E, HEAD_P>(A, a.head_w.q, a.head_w.d, rows_of(t0), [&](int rl) { return t0 * TR + rl; });
    const W8 nw = wload8(norm_w);
    wait_vm<5>();   // about half of the 11 loads above
    const XR xr = make_xr(a.xbase, a.xbytes);
    if (!prologue<NL>(nl, c.ctl, nullptr, nullptr, a.xc.x + (size_t)c.par() * NL * E, c.tag(k - 1, PH_DOWN), c.err, nw, a.m.eps,
                      s.xf, &s.xq[0][0], E, &s.xd[0][0], E / 32, s.ns, s.xn, &c.ps->fail, &xr))
        return false;
    tr_pass(c);
    if (c.b == 0) {
        // h_nextn of each lane (Engine::hidden): the normalised x2
        const int l = t >> 8, tt = t & 255;
        if (l < nl) put8(a.b.hid + (int64_t)l * E + 8 * tt, &s.xn[l][8 * tt]);
    }
    if (mask == 0) return true;
    float best = -__builtin_inff();
    int64_t bi = -1;
    const int rl = t % TR, l = t / TR;
    // two register buffers; both reload every iteration, past the range the last tile again (read from
    // cache), so no load sits behind a branch and the compiler's waits stay counts of loads in flight
    auto dot_tile = [&](WSlice<E, HEAD_P> &W, int64_t tile) {
        const int nr = rows_of(tile);
        wdot<E, HEAD_P, NL>(W, nr, &s.xq[0][0], E, &s.xd[0][0], E / 32, s.g);
        if (l < NL && l < nl && rl < nr) {
            const float v = s.g.out[l][rl];
            const int64_t row = tile * TR + rl;
            if (a.keep_logits) a.b.logits[l * V + row] = v;
            if (v > best) { best = v; bi = row; }
        }
    };
    if (!dyn) {
        for (int64_t tile = t0; tile < t1; tile += 2) {
            const int64_t tb = tile + 1 < t1 ? tile + 1 : t1 - 1, ta = tile + 2 < t1 ? tile + 2 : t1 - 1;
            wload<E, HEAD_P, true>(B, a.head_w.q, a.head_w.d, rows_of(tb), [&](int r) { return tb * TR + r; });
            dot_tile(A, tile);
            wload<E, HEAD_P, true>(A, a.head_w.q, a.head_w.d, rows_of(ta), [&](int r) { return ta * TR + r; });
            if (tile + 1 < t1) dot_tile(B, tile + 1);
        }
    } else {
        // the i-th tile of this workgroup: i < per its own, then pair k = (i - per) / 2 of its claims
        // (tiles ns + d, ns + d + 1 for the counter's value d), -1 past the last tile. Claim k is
        // issued by thread 0 two iterations before pair k is reached (at i = per + 2 k - 4), its value
        // written to LDS mid-iteration and published by the next barrier; every claim issued is read
        // before the workgroup leaves, so no atomic is in flight at the launch's end (when the last
        // workgroup out clears the counter). Tiles are visited in increasing order (claims increase).
        const int64_t ns = per * c.G;
        uint32_t *hq = a.sync + FZ_W_HEADQ;
        auto seq = [&](int64_t i) -> int64_t {
            if (i < per) return t0 + i;
            const int64_t f = s.claim[((i - per) >> 1) & 3] + ((i - per) & 1);
            return f < ntiles ? f : -1;
        };
        uint32_t rv = 0;
        for (int64_t i = 0;; i += 2) {
            const int64_t tc = seq(i);
            if (tc < 0) break;
            const bool claim = i >= per - 4;
            if (claim && t == 0) rv = __hip_atomic_fetch_add(hq, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const int64_t sb = seq(i + 1), sa = seq(i + 2);
            const int64_t tb = sb < 0 ? tc : sb, ta = sa < 0 ? tb : sa;   // past the end: a reload
            wload<E, HEAD_P, true>(B, a.head_w.q, a.head_w.d, rows_of(tb), [&](int r) { return tb * TR + r; });
            dot_tile(A, tc);
            if (claim && t == 0) s.claim[((i - per + 4) >> 1) & 3] = ns + (int64_t)rv;
            wload<E, HEAD_P, true>(A, a.head_w.q, a.head_w.d, rows_of(ta), [&](int r) { return ta * TR + r; });
            if (sb >= 0) dot_tile(B, tb);
        }
    }
    // per-lane key of this workgroup: the largest value, then the smallest row
    unsigned long long key = 0ull;
    if (l < NL && l < nl && ((mask >> l) & 1) && bi >= 0) {
        // a restricted draft head's rows are ascending token ids: the first maximum by row is the
        // first by id
        const uint32_t id = a.head_ids ? a.head_ids[bi] : (uint32_t)bi;
        key = ((unsigned long long)ordered_bits_f(best) << 32) | (0xffffffffu - id);
    }
    if (t < NL * TR) {
        for (int m = TR / 2; m >= 1; m >>= 1) {
            const unsigned long long o = __shfl_xor(key, m, 64);
            key = key > o ? key : o;
        }
        if (rl == 0 && l < NL) {
            a.keys[(int64_t)l * c.G + c.b] = key;
            // and as two tagged halves, for the launch's last stage (the device-driven MTP step)
            uint64_t *kx = a.xc.kx + ((size_t)l * c.G + c.b) * 2;
            ll_st(kx, (uint32_t)key, c.tag(k, PH_HEAD));
            ll_st(kx + 1, (uint32_t)(key >> 32), c.tag(k, PH_HEAD));
        }
    }
    tr_end(c, TP_HEAD);
    return true;
}

// One call per layer boundary: the MoE tail (experts, down) of layer ilp as run layer kp (ilp >= 0),
// then the projection, mixer, output and router phases of layer il as run layer k (il >= 0; embed:
// its input is the token embedding). The call boundary sits between the router and experts phases,
// so the down phase can load the next layer's projection slice into registers.
template <int NL>
__device__ __attribute__((noinline)) bool run_step(const RunCtl *ctl, const FusedArgs *ap, int ilp, int kp, int il, int k,
                                                   bool embed, uint32_t base) {
    ProjPre pre;
    if (ilp >= 0 && !phase_moe<NL>(ctl, ap, ilp, kp, il, pre)) return false;
    if (il < 0) return true;
    const LayerDev &L = ap->layers[il];
    const int att = L.att;
    // the residual: the embedding (written by the projection phase) or the previous layer's output
    const uint32_t xtag = base + 1u + (embed ? 8u * (uint32_t)k + PH_PROJ : 8u * (uint32_t)(k - 1) + PH_DOWN);
    DnPre dp;
    if (!phase_proj<NL>(ctl, ap, il, k, embed, 0, att ? AT_ROWS : DN_ROWS, pre, ilp >= 0, dp)) return false;
    if (!att) {
        if (!phase_dn<NL>(ctl, ap, il, k, dp)) return false;
    } else {
        if (!phase_scores<NL>(ctl, ap, il, k, false)) return false;
        if (!phase_pv<NL>(ctl, ap, il, k)) return false;
    }
    if (!phase_out<NL>(ctl, ap, il, k, xtag)) return false;
    if (!phase_router<NL>(ctl, ap, il, k)) return false;
    return true;
}

template <int NL>
OXE_DEV void run_all(const RunCtl *ctl, const FusedArgs *ap, uint32_t base) {
    const int mode = ap->mode, nlay = ap->n_layer;
    if (mode == FM_VERIFY) {
        for (int il = 0; il <= nlay; il++)
            if (!run_step<NL>(ctl, ap, il - 1, il - 1, il < nlay ? il : -1, il, il == 0, base)) return;
        (void)phase_head<NL>(ctl, ap, ap->m.out_norm, nlay);
    } else if (mode == FM_DRAFT) {
        const int il = nlay;
        if (!phase_entry<NL>(ctl, ap, il)) return;
        // the MTP layer (attention) as run layer 1, its input the entry output
        if (!run_step<NL>(ctl, ap, -1, 0, il, 1, false, base)) return;
        if (!run_step<NL>(ctl, ap, il, 1, -1, 2, false, base)) return;
        (void)phase_head<NL>(ctl, ap, ap->layers[il].head_norm, 2);
    } else {
        const int il = nlay;
        if (!phase_entry<NL>(ctl, ap, il)) return;
        ProjPre pre;
        DnPre dp;   // the MTP layer is an attention layer: not loaded
        if (!phase_proj<NL>(ctl, ap, il, 1, false, AT_K, AT_ROWS, pre, false, dp)) return;
        (void)phase_scores<NL>(ctl, ap, il, 1, true);
    }
}

}  // namespace fz

// The device-driven MTP step's decision at the end of its fused draft (stage 1) or verify (stage 2)
// run, by workgroup 0 once every other workgroup has left (done: the run's phases ran; false for an
// inactive run, whose step still decides to stop). The LM head's per-workgroup keys are read as
// tagged words (their stores may still be in flight); hid rows are workgroup 0's own writes.
template <int NL>
OXE_DEV void mtp_stage(const RunCtl *ctl, const FusedArgs *ap, uint32_t base, bool done) {
    using namespace fz;
    const FZ_CAS FusedArgs &a = *uni(ap);
    const MtpHooks &h = *a.mh;
    const int stage = uni(ctl)->stage, t = threadIdx.x, G = gridDim.x;
    struct StageSm {
        unsigned long long k[FT / 64];
        CommitSm cs;
        int aborted;
    };
    StageSm &sm = *(StageSm *)fz_dyn;
    if (t == 0) sm.aborted = done && cld32(a.sync + FZ_W_ERR) != 0;
    __syncthreads();
    const bool ran = done && !sm.aborted;
    unsigned long long key = 0ull;
    if (ran) {
        static_assert(NL * 256 == FT, "a key per thread: lane t / 256, workgroup t % 256");
        const int l = t / 256, bb = t % 256;
        const int kh = a.mode == FM_VERIFY ? a.n_layer : 2;   // the head's run layer (run_all)
        const uint32_t tag = base + 1u + 8u * (uint32_t)kh + (uint32_t)PH_HEAD;
        uint32_t u[2];
        const bool ok = ll_gather<2, 0, false>(
            [&](int i) { return LLW{a.xc.kx + ((size_t)l * G + bb) * 2 + i, tag, bb < G}; }, u, a.sync + FZ_W_ERR,
            nullptr);
        key = ok && bb < G ? ((unsigned long long)u[1] << 32) | u[0] : 0ull;
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) {
            const unsigned long long o = __shfl_xor(key, m, 64);
            key = o > key ? o : key;
        }
        if ((t & 63) == 0) sm.k[t >> 6] = key;
        (void)ok;   // a failed gather leaves the sticky error word set (checked below)
    }
    __syncthreads();
    if (t == 0 && ran && cld32(a.sync + FZ_W_ERR) != 0) sm.aborted = 1;
    __syncthreads();
    auto lane_max = [&](int l) {
        unsigned long long m = 0ull;
        for (int w = 4 * l; w < 4 * l + 4; w++) m = sm.k[w] > m ? sm.k[w] : m;
        return m;
    };
    const bool good = ran && !sm.aborted;
    if (stage == 1) {
        if (t == 0) {
            if (done && !good) h.ms->err |= 4;   // the draft run aborted: the steps stop
            const int dl = uni(ctl)->nl - 1;     // the draft is the run's last lane
            *h.ctl_verify = mtp_after_draft(h.ms, good ? lane_max(dl < NL ? dl : NL - 1) : 0ull, h.force, h.force_n, h.n_ctx);
        }
    } else if (stage == 2) {
        if (t == 0 && done && !good) h.ms->err |= 4;   // the verify run aborted: the steps stop
        const uint32_t g0 = decode_key(good ? lane_max(0) : 0ull), g1 = decode_key(good ? lane_max(1) : 0ull);
        mtp_commit(h.ms, good, g0, g1, a.b.hid, h.n_ctx, h.out_tok, h.out_cap, h.ctl_draft, sm.cs);
    }
}

template <int NL>
__global__ __launch_bounds__(fz::FT, 1) void fused_kernel(const RunCtl *__restrict__ ctl, const FusedArgs *__restrict__ ap) {
    using namespace fz;
    if (!ctl->active) {
        if (ctl->stage != 0 && blockIdx.x == 0) mtp_stage<NL>(ctl, ap, 0u, false);
        return;
    }
    if (threadIdx.x == 0) {
        fz_ps.base = cld32(&ap->sync[FZ_W_FLAG]);
        fz_ps.fail = 0;
        fz_ps.tev = 0;
        fz_ps.dyn_off = (uint32_t)(uintptr_t)(FZ_LDS unsigned char *)fz_dyn;
    }
    if (threadIdx.x < 32) fz_ps.exp2tab[threadIdx.x] = oxe_libm::kExp2fTab[threadIdx.x];
    __syncthreads();
    const uint32_t base = (uint32_t)__builtin_amdgcn_readfirstlane((int)fz_ps.base);
    run_all<NL>(ctl, ap, base);
    // every workgroup counts itself out, aborted or not; the last one moves the tag base past this
    // launch's tags and re-arms the counter (the next launch on the stream starts after this one ends)
    __syncthreads();
    if (ctl->stage != 0 && blockIdx.x == 0) {
        // a run of the device-driven MTP step: workgroup 0 leaves last, after the step's decision
        uint32_t *sync = ap->sync;
        if (threadIdx.x == 0) {
            uint32_t spins = 0;
            while (cld32(sync + FZ_W_DONE) != gridDim.x - 1 && ++spins < 4u * SPIN_MAX) __builtin_amdgcn_s_sleep(2);
            if (spins >= 4u * SPIN_MAX) cst32(sync + FZ_W_ERR, 1u);
        }
        __syncthreads();
        mtp_stage<NL>(ctl, ap, base, true);
        __syncthreads();
        if (threadIdx.x == 0) {
            cst32(sync + FZ_W_DONE, 0u);
            cst32(sync + FZ_W_HEADQ, 0u);
            cst32(sync + FZ_W_FLAG, base + FZ_TAG_STRIDE);
        }
        return;
    }
    if (threadIdx.x == 0) {
        uint32_t *sync = ap->sync;
        const uint32_t old = __hip_atomic_fetch_add(sync + FZ_W_DONE, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (old == gridDim.x - 1) {
            cst32(sync + FZ_W_DONE, 0u);
            cst32(sync + FZ_W_HEADQ, 0u);
            cst32(sync + FZ_W_FLAG, base + FZ_TAG_STRIDE);
        }
    }
}

size_t fused_lds_bytes(int n_ctx) {
    const size_t base = sizeof(fz::PhaseSm<OXE_NL>);
    // the attention-output phase: f16 probability pairs [n_ctx / 2][2], the V^T tile
    // [PVD][min(n_ctx, PV_VMAX) + 32], and the softmax's cross-wave maxima and sums
    const size_t vmax = (size_t)(n_ctx < fz::PV_VMAX ? n_ctx : fz::PV_VMAX);
    const size_t pv = (size_t)n_ctx * 4 + (size_t)fz::PVD * (vmax + 32) * 2 + 256;
    return (base > pv ? base : pv + 16) / 16 * 16 + 16;
}

int fused_blocks_per_cu(size_t lds) {
    static size_t configured = 0;
    if (lds > configured) {
        if (hipFuncSetAttribute((const void *)fused_kernel<OXE_NL>, hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds) !=
            hipSuccess)
            return 0;
        configured = lds;
    }
    int n = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fused_kernel<OXE_NL>, fz::FT, lds) != hipSuccess) return 0;
    return n;
}

void launch_fused(const RunCtl *ctl, const FusedArgs *dev_args, int grid, size_t lds, hipStream_t st) {
    hipLaunchKernelGGL(fused_kernel<OXE_NL>, dim3((unsigned)grid), dim3(fz::FT), lds, st, ctl, dev_args);
}

// after an aborted run: the error word and the finished counter cleared, the tag base moved past
// every tag the aborted launch may have written
__global__ void fused_sync_reset_kernel(uint32_t *w) {
    const uint32_t base = w[FZ_W_FLAG];
    __syncthreads();
    for (int i = threadIdx.x; i < FZ_SYNC_WORDS; i += blockDim.x) w[i] = i == FZ_W_FLAG ? base + FZ_TAG_STRIDE : 0u;
}
void launch_fused_sync_reset(uint32_t *sync, hipStream_t st) {
    hipLaunchKernelGGL(fused_sync_reset_kernel, dim3(1), dim3(256), 0, st, sync);
}

// every exchange word back to tag 0 (never a live tag) and the tag base to 0
__global__ void fused_xch_clear_kernel(uint64_t *x, size_t n, uint32_t *sync) {
    for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) x[i] = 0ull;
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < FZ_SYNC_WORDS; i += blockDim.x) sync[i] = 0u;
}
void launch_fused_xch_clear(uint64_t *xch, size_t words, uint32_t *sync, hipStream_t st) {
    hipLaunchKernelGGL(fused_xch_clear_kernel, dim3(256), dim3(256), 0, st, xch, words, sync);
}

}  // namespace oxe
