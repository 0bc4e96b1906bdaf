"""TEST INFRASTRUCTURE ONLY: ctypes binding of the CPU oracle (liboxo.so).

The oracle restates the reference's CPU arithmetic (n0rpan/snapdragon-engine, crates/kernels-sys
and crates/model) in its float order. Only tests/, __graft_entry__.smoke() and bench.py's
cpu_baseline leg may load it, and only as the checker.
"""
import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboxo.so")


class ModelDesc(C.Structure):
    _fields_ = [
        ("n_layer", C.c_int32), ("n_embd", C.c_int32), ("n_vocab", C.c_int32),
        ("n_head", C.c_int32), ("n_head_kv", C.c_int32), ("head_dim", C.c_int32),
        ("n_expert", C.c_int32), ("n_expert_used", C.c_int32), ("ff_exp", C.c_int32), ("ff_shexp", C.c_int32),
        ("ssm_conv_kernel", C.c_int32), ("ssm_d_state", C.c_int32), ("ssm_n_kheads", C.c_int32),
        ("ssm_n_vheads", C.c_int32), ("ssm_d_inner", C.c_int32),
        ("full_attention_interval", C.c_int32), ("n_rot", C.c_int32), ("rope_sections", C.c_int32 * 4),
        ("rms_eps", C.c_float), ("rope_freq_base", C.c_float), ("n_ctx_train", C.c_int32), ("has_mtp", C.c_int32),
    ]


def desc_35b_a3b(**over):
    """The BASELINE 35B-A3B shape (reference tests/fixtures/ornith.json, vocab 151936)."""
    d = ModelDesc(n_layer=40, n_embd=2048, n_vocab=151936, n_head=16, n_head_kv=2, head_dim=256,
                  n_expert=256, n_expert_used=8, ff_exp=512, ff_shexp=512, ssm_conv_kernel=4,
                  ssm_d_state=128, ssm_n_kheads=16, ssm_n_vheads=32, ssm_d_inner=4096,
                  full_attention_interval=4, n_rot=64, rms_eps=np.float32(9.999999974752427e-07),
                  rope_freq_base=1e7, n_ctx_train=262144, has_mtp=1)
    d.rope_sections[:] = [11, 11, 10, 0]
    for k, v in over.items():
        setattr(d, k, v)
    return d


def desc_small(**over):
    """A reduced model with the same per-layer shapes: 4 layers (3 delta-net + 1 attention) + MTP,
    vocab 4096; the shape of the reference's mini-model tests (model/src/testkit.rs)."""
    over.setdefault("n_layer", 4)
    over.setdefault("n_vocab", 4096)
    return desc_35b_a3b(**over)


def build():
    subprocess.check_call(["make", "-s", "-C", HERE, "liboxo.so"])


_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        P = C.POINTER
        f32p, u16p, i8p, i32p, u32p = P(C.c_float), P(C.c_uint16), P(C.c_int8), P(C.c_int32), P(C.c_uint32)
        sig = {
            "oxo_f16_to_f32": (C.c_float, [C.c_uint16]),
            "oxo_f32_to_f16": (C.c_uint16, [C.c_float]),
            "oxo_f16_fma": (C.c_uint16, [C.c_uint16, C.c_uint16, C.c_uint16]),
            "oxo_f16_add": (C.c_uint16, [C.c_uint16, C.c_uint16]),
            "oxo_quantize_row_q8_0": (None, [f32p, C.c_int64, i8p, u16p]),
            "oxo_dequantize_row_q8_0": (None, [i8p, u16p, C.c_int64, f32p]),
            "oxo_gemv_q8_0": (None, [C.c_int64, C.c_int64, C.c_int, i8p, u16p, i8p, u16p, f32p, i32p]),
            "oxo_vec_dot_f32": (C.c_float, [C.c_int, f32p, f32p]),
            "oxo_vec_dot_f16": (C.c_float, [C.c_int, u16p, u16p]),
            "oxo_v_expf": (C.c_float, [C.c_float]),
            "oxo_v_silu": (C.c_float, [C.c_float]),
            "oxo_silu_f32": (None, [C.c_int, f32p, f32p]),
            "oxo_swiglu_f32": (None, [C.c_int, f32p, f32p, f32p]),
            "oxo_vec_soft_max_f32": (C.c_double, [C.c_int, f32p, f32p, C.c_float]),
            "oxo_vec_sum_f32": (C.c_float, [C.c_int, f32p]),
            "oxo_vec_max_f32": (C.c_float, [C.c_int, f32p]),
            "oxo_rms_norm_f32": (None, [f32p, f32p, C.c_int64, C.c_float]),
            "oxo_rms_norm_mul_f32": (None, [f32p, f32p, f32p, C.c_int64, C.c_float]),
            "oxo_gdn_l2_norm_f32": (None, [f32p, C.c_int64, C.c_float]),
            "oxo_sigmoid_f32": (None, [C.c_int64, f32p, f32p]),
            "oxo_softplus_f32": (None, [C.c_int64, f32p, f32p]),
            "oxo_soft_max_f32": (None, [C.c_int, f32p, f32p, C.c_float, f32p, f32p]),
            "oxo_argsort_top_k_f32": (None, [f32p, C.c_int, C.c_int, i32p, i32p, P(C.c_int)]),
            "oxo_ssm_conv_step_f32": (None, [f32p, f32p, f32p, C.c_int, C.c_int, f32p]),
            "oxo_gated_delta_net_step_f32_from": (None, [f32p, f32p, f32p, f32p, f32p, C.c_float, C.c_float, C.c_int64, f32p]),
            "oxo_mrope_cache_init": (None, [C.c_int64, i32p, C.c_int, C.c_int, C.c_int64, C.c_float, C.c_float,
                                            C.c_float, C.c_float, C.c_float, C.c_float, C.c_int, C.c_int, f32p]),
            "oxo_rope_neox_inplace": (None, [f32p, C.c_int, f32p]),
            "oxo_attn_head_f16": (None, [f32p, u16p, C.c_int64, u16p, u16p, C.c_int64, C.c_int, C.c_int, C.c_int,
                                         C.c_float, f32p]),
            "oxo_eval_unary": (None, [C.c_int, C.c_uint32, C.c_int64, C.c_int64, f32p]),
            "oxo_engine_new": (C.c_void_p, [P(ModelDesc), C.c_uint64, C.c_int64]),
            "oxo_engine_free": (None, [C.c_void_p]),
            "oxo_engine_new_lanes": (C.c_void_p, [P(ModelDesc), C.c_uint64, C.c_int64, C.c_int]),
            "oxo_engine_new_typed": (C.c_void_p, [P(ModelDesc), C.c_uint64, C.c_int64, C.c_int, i32p]),
            "oxo_engine_reset": (None, [C.c_void_p]),
            "oxo_verify": (C.c_int, [C.c_void_p, u32p, C.c_int, u32p]),
            "oxo_commit": (C.c_int, [C.c_void_p, C.c_int]),
            "oxo_step": (C.c_uint32, [C.c_void_p, C.c_uint32]),
            "oxo_mtp_run": (C.c_uint32, [C.c_void_p, u32p, C.c_int, C.c_int64, f32p, C.c_int]),
            "oxo_mtp_seed": (None, [C.c_void_p, u32p, C.c_int, C.c_int64, f32p]),
            "oxo_pos": (C.c_int64, [C.c_void_p]),
            "oxo_cur_slot": (C.c_int, [C.c_void_p]),
            "oxo_tie_count": (C.c_int, [C.c_void_p]),
            "oxo_hidden": (f32p, [C.c_void_p, C.c_int]),
            "oxo_logits": (f32p, [C.c_void_p, C.c_int]),
            "oxo_n_ctx": (C.c_int64, [C.c_void_p]),
            "oxo_set_keep_logits": (None, [C.c_void_p, C.c_int]),
            "oxo_gen_seconds": (C.c_double, [C.c_void_p]),
            "oxo_set_plan": (C.c_int, [C.c_void_p, C.c_int]),
            "oxo_set_draft_vocab": (C.c_int, [C.c_void_p, u32p, C.c_int]),
            "oxo_plan_barriers": (C.c_int64, [C.c_void_p]),
            "oxo_pin_team": (C.c_int, [C.c_int]),
            "oxo_kcache": (u16p, [C.c_void_p]),
            "oxo_vcache": (u16p, [C.c_void_p]),
            "oxo_conv_state": (f32p, [C.c_void_p]),
            "oxo_ssm_state": (f32p, [C.c_void_p]),
            "oxo_kcache_mut": (u16p, [C.c_void_p]),
            "oxo_vcache_mut": (u16p, [C.c_void_p]),
            "oxo_set_pos": (None, [C.c_void_p, C.c_int64]),
            "oxo_mixer": (None, [C.c_void_p, C.c_int, C.c_int, C.c_int64, f32p, f32p]),
            "oxo_moe": (None, [C.c_void_p, C.c_int, C.c_int, f32p, f32p]),
            "oxo_mtp_entry": (None, [C.c_void_p, u32p, C.c_int, f32p, f32p]),
            "oxo_engine_set_router": (None, [C.c_void_p, C.c_int, C.c_int, C.c_int, f32p]),
            "oxo_synth_q8": (None, [C.c_uint64, C.c_int, C.c_int, C.c_int64, C.c_int64, C.c_int64, i8p, u16p]),
            "oxo_dequantize_row_kq": (C.c_int, [C.c_int, C.c_void_p, f32p, C.c_int64]),
            "oxo_synth_kq": (C.c_int64, [C.c_uint64, C.c_int, C.c_int, C.c_int, C.c_int64, C.c_int64, C.c_int64,
                                         C.POINTER(C.c_uint8)]),
            "oxo_synth_f32": (None, [C.c_uint64, C.c_int, C.c_int, C.c_int64, f32p]),
            "oxo_synth_normal": (None, [C.c_uint64, C.c_uint64, C.c_int64, C.c_float, C.c_float, f32p]),
            "oxo_driver_new": (C.c_void_p, [C.c_void_p, C.c_int]),
            "oxo_driver_free": (None, [C.c_void_p]),
            "oxo_driver_import": (None, [C.c_void_p, C.c_int64, f32p]),
            "oxo_engine_read_state": (C.c_int, [C.c_void_p, C.c_void_p, C.c_int64, C.c_int64]),
            "oxo_driver_prefill": (C.c_uint32, [C.c_void_p, u32p, C.c_int]),
            "oxo_driver_step": (C.c_int, [C.c_void_p, C.c_uint32, u32p, C.c_int64]),
            "oxo_driver_step_plain": (C.c_uint32, [C.c_void_p, C.c_uint32]),
            "oxo_driver_step_force": (C.c_int, [C.c_void_p, C.c_uint32, u32p, P(C.c_int64), C.c_int]),
            "oxo_driver_rewind": (C.c_int, [C.c_void_p, C.c_int]),
            "oxo_driver_stats": (None, [C.c_void_p, P(C.c_int64)]),
            "oxo_quantize_row_q8_K": (None, [f32p, C.c_void_p, C.c_int64]),
            "oxo_vl_gemv": (C.c_int, [C.c_int, C.c_int64, C.c_int64, C.c_int, C.c_void_p, C.c_void_p, f32p]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def ptr(a, ct):
    return a.ctypes.data_as(C.POINTER(ct))


# ---- kernel-level helpers (numpy in, numpy out)

def quantize_q8_0(x):
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    rows = x.reshape(-1, k)
    q = np.empty(rows.shape, np.int8)
    d = np.empty((rows.shape[0], k // 32), np.uint16)
    for i in range(rows.shape[0]):
        lib().oxo_quantize_row_q8_0(ptr(rows[i], C.c_float), k, ptr(q[i], C.c_int8), ptr(d[i], C.c_uint16))
    return q.reshape(x.shape), d.reshape(x.shape[:-1] + (k // 32,))


# ggml block_q8_K (ggml-common.h:371-375) and the K-quant block sizes (315-368)
Q8K = np.dtype([("d", "<f4"), ("qs", "i1", (256,)), ("bsums", "<i2", (16,))])
KQ_BYTES = {3: 110, 4: 144, 5: 176, 6: 210}


def quantize_q8_K(x):
    """quantize_row_q8_K_ref per row: float rows [..., k] -> uint8 [..., k/256 * 292]"""
    x = np.ascontiguousarray(x, dtype=np.float32)
    k = x.shape[-1]
    rows = x.reshape(-1, k)
    y = np.zeros((rows.shape[0], k // 256 * 292), np.uint8)
    for i in range(rows.shape[0]):
        lib().oxo_quantize_row_q8_K(ptr(rows[i], C.c_float), y[i].ctypes.data_as(C.c_void_p), k)
    return y.reshape(x.shape[:-1] + (k // 256 * 292,))


def vl_gemv(ty, w, k, y):
    """oxe_vl_gemv per lane: w uint8 [nr][k/256 * block bytes] (ggml blocks), y uint8 [nl][k/256 * 292]
    -> f32 [nl][nr]"""
    w = np.ascontiguousarray(w, np.uint8)
    y = np.ascontiguousarray(y, np.uint8)
    nr, nl = w.shape[0], y.shape[0]
    s = np.empty((nl, nr), np.float32)
    rc = lib().oxo_vl_gemv(ty, k, nr, nl, w.ctypes.data_as(C.c_void_p), y.ctypes.data_as(C.c_void_p), ptr(s, C.c_float))
    if rc != 1:
        raise ValueError(f"vl_gemv: type {ty} not handled")
    return s


def gemv_q8_0(wq, wd, xq, xd, want_isum=False):
    nr, k = wq.shape
    nl = xq.shape[0]
    y = np.empty((nl, nr), np.float32)
    isum = np.empty((nl, nr, k // 32), np.int32) if want_isum else None
    lib().oxo_gemv_q8_0(k, nr, nl, ptr(np.ascontiguousarray(wq), C.c_int8), ptr(np.ascontiguousarray(wd), C.c_uint16),
                        ptr(np.ascontiguousarray(xq), C.c_int8), ptr(np.ascontiguousarray(xd), C.c_uint16),
                        ptr(y, C.c_float), ptr(isum, C.c_int32) if want_isum else None)
    return (y, isum) if want_isum else y


def synth_q8(seed, layer, kind, rows, k, expert=0):
    q = np.empty((rows, k), np.int8)
    d = np.empty((rows, k // 32), np.uint16)
    lib().oxo_synth_q8(seed, layer, kind, expert, rows, k, ptr(q, C.c_int8), ptr(d, C.c_uint16))
    return q, d


KQ_BLOCK = {11: 110, 12: 144, 13: 176, 14: 210}   # ggml type id -> bytes per 256 weights


def synth_kq(seed, layer, kind, ty, rows, k, expert=0):
    """synthetic K-quant tensor (ggml type 11..14): rows x k/256 blocks as uint8 [rows][row bytes]"""
    out = np.empty((rows, k // 256 * KQ_BLOCK[ty]), np.uint8)
    n = lib().oxo_synth_kq(seed, layer, kind, ty, expert, rows, k, ptr(out, C.c_uint8))
    assert n == out.size
    return out


def dequantize_row_kq(ty, raw, k):
    """dequantize_row_q*_K (ggml type 11..14) of one row of k / 256 blocks -> f32 [k]"""
    b = np.ascontiguousarray(raw, np.uint8)
    y = np.empty(k, np.float32)
    assert lib().oxo_dequantize_row_kq(ty, b.ctypes.data_as(C.c_void_p), ptr(y, C.c_float), k) == 1
    return y


def synth_f32(seed, layer, kind, n):
    v = np.empty(n, np.float32)
    lib().oxo_synth_f32(seed, layer, kind, n, ptr(v, C.c_float))
    return v


def synth_normal(seed, uid, n, mu=0.0, sigma=1.0):
    v = np.empty(n, np.float32)
    lib().oxo_synth_normal(seed, uid, n, mu, sigma, ptr(v, C.c_float))
    return v


# tensor kinds (include/oxe_model.h)
T = dict(ATTN_NORM=0, POST_NORM=1, DN_QKV=2, DN_Z=3, DN_BETA=4, DN_ALPHA=5, DN_CONV=6, DN_A=7, DN_DT=8,
         DN_NORM=9, DN_OUT=10, ATT_Q=11, ATT_K=12, ATT_V=13, ATT_QNORM=14, ATT_KNORM=15, ATT_OUT=16,
         ROUTER=17, SHEXP_GATE=18, GATE_EXPS=19, UP_EXPS=20, DOWN_EXPS=21, GATE_SHEXP=22, UP_SHEXP=23,
         DOWN_SHEXP=24, EH_PROJ=25, ENORM=26, HNORM=27, HEAD_NORM=28, TOK_EMBD=29, OUT_NORM=30, OUTPUT=31)
GLOBAL_LAYER = 63


def config1_inputs(seed=0):
    """W [4096 x 2048] Q8_0 (codes U[-127,127], fp16 scales U(0.001, 0.02)),
    x = 2 lanes x 2048 N(0,1) (Irwin-Hall), quantized per 32-block. Tensor uid: layer 62."""
    wq, wd = synth_q8(seed, 62, T["OUTPUT"], 4096, 2048)
    x = synth_normal(seed, 62 * 64 + 40, 2 * 2048).reshape(2, 2048)
    xq, xd = quantize_q8_0(x)
    return wq, wd, x, xq, xd


class Engine:
    """Oracle engine (engine.rs semantics) on the synthetic model."""

    def __init__(self, desc, seed=0, n_ctx=1024, lanes=2, types=None):
        """types: {(layer, kind): ggml type id} for matrices that are not Q8_0 (layer GLOBAL_LAYER
        for the LM head)"""
        self.desc = desc
        if types:
            tt = np.full(64 * 64, 8, np.int32)
            for (layer, kind), ty in types.items():
                tt[layer * 64 + kind] = ty
            self.h = lib().oxo_engine_new_typed(C.byref(desc), seed, n_ctx, lanes, ptr(tt, C.c_int32))
            if not self.h:
                raise ValueError("a matrix type this model cannot take there")
        else:
            self.h = (lib().oxo_engine_new(C.byref(desc), seed, n_ctx) if lanes == 2 else
                      lib().oxo_engine_new_lanes(C.byref(desc), seed, n_ctx, lanes))
        self.n_ctx = lib().oxo_n_ctx(self.h)

    def close(self):
        if self.h:
            lib().oxo_engine_free(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def verify(self, toks):
        t = np.asarray(toks, np.uint32)
        out = np.zeros(8, np.uint32)
        rc = lib().oxo_verify(self.h, ptr(t, C.c_uint32), len(t), ptr(out, C.c_uint32))
        assert rc == 0, "verify failed"
        return out[: len(t)].copy()

    def commit(self, m):
        assert lib().oxo_commit(self.h, m) == 0

    def set_draft_vocab(self, ids):
        v = np.ascontiguousarray(ids, np.uint32)
        n = lib().oxo_set_draft_vocab(self.h, ptr(v, C.c_uint32), len(v))
        if n < 0:
            raise ValueError("empty draft vocabulary")
        return n

    def set_plan(self, nthreads):
        """run through the reference's static plan on a pinned team of nthreads (0: the default
        path); returns the team size"""
        return int(lib().oxo_set_plan(self.h, nthreads))

    def plan_barriers(self):
        return int(lib().oxo_plan_barriers(self.h))

    def step(self, tok):
        return int(lib().oxo_step(self.h, tok))

    def mtp_run(self, toks, pos0, hs, head_last=True):
        t = np.asarray(toks, np.uint32)
        h = np.ascontiguousarray(hs, np.float32)
        return int(lib().oxo_mtp_run(self.h, ptr(t, C.c_uint32), len(t), pos0, ptr(h, C.c_float), int(head_last)))

    def mtp_seed(self, toks, pos0, hs):
        t = np.asarray(toks, np.uint32)
        h = np.ascontiguousarray(hs, np.float32)
        lib().oxo_mtp_seed(self.h, ptr(t, C.c_uint32), len(t), pos0, ptr(h, C.c_float))

    @property
    def pos(self):
        return int(lib().oxo_pos(self.h))

    def read_state(self, buf, n_pos):
        """Engine::read_state (engine.rs:1819-1871) of write_state bytes"""
        b = np.ascontiguousarray(buf, np.uint8)
        assert lib().oxo_engine_read_state(self.h, b.ctypes.data_as(C.c_void_p), b.nbytes, n_pos) == 0, "read_state"

    def set_router(self, layer, row0, rows):
        r = np.ascontiguousarray(rows, np.float32)
        lib().oxo_engine_set_router(self.h, layer, row0, r.shape[0], ptr(r, C.c_float))

    def hidden(self, lane):
        return np.ctypeslib.as_array(lib().oxo_hidden(self.h, lane), (self.desc.n_embd,)).copy()

    def logits(self, lane):
        return np.ctypeslib.as_array(lib().oxo_logits(self.h, lane), (self.desc.n_vocab,)).copy()


class Driver:
    """MtpDriver (crates/model/src/mtp.rs:314-608) over an oracle Engine."""

    def __init__(self, eng, depth=1):
        self.eng = eng
        self.h = lib().oxo_driver_new(eng.h, depth)

    def prefill(self, toks):
        t = np.asarray(toks, np.uint32)
        return int(lib().oxo_driver_prefill(self.h, ptr(t, C.c_uint32), len(t)))

    def step(self, x, override_d1=-1, force=None):
        """one speculative step; override_d1 / force[i] >= 0 replace draft 1 / draft i + 1"""
        out = np.zeros(8, np.uint32)
        if force is not None:
            f = np.asarray(force, np.int64)
            n = lib().oxo_driver_step_force(self.h, x, ptr(out, C.c_uint32), ptr(f, C.c_int64), len(f))
        else:
            n = lib().oxo_driver_step(self.h, x, ptr(out, C.c_uint32), override_d1)
        return [int(v) for v in out[:n]]

    def import_state(self, q, hl):
        h = np.ascontiguousarray(hl, np.float32)
        lib().oxo_driver_import(self.h, q, ptr(h, C.c_float))

    def step_plain(self, x):
        return int(lib().oxo_driver_step_plain(self.h, x))

    def rewind(self, m):
        return int(lib().oxo_driver_rewind(self.h, m))

    def stats(self):
        s = np.zeros(4, np.int64)
        lib().oxo_driver_stats(self.h, ptr(s, C.c_int64))
        return dict(steps=int(s[0]), drafted=int(s[1]), accepted=int(s[2]), tokens_out=int(s[3]))


def bench_prompt(n):
    """oxe bench's prompt ids (crates/oxe-cli/src/bin/oxe.rs:428-435): (i*2654435761 mod 2^32) % 150000 + 1000."""
    i = np.arange(n, dtype=np.uint64)
    return (((i * 2654435761) & 0xFFFFFFFF) % 150000 + 1000).astype(np.uint32)
