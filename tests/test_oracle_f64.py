"""The oracle engine's layer composition against an independent float64 statement of it (no GPU).

tests/f64_model.py restates the decode layers from the reference's engine (crates/model/src/
engine.rs: delta-net mixer 2394-2609, gated attention 2614-2827 and 3327-3368, MoE 3372-3624, MTP
entry 2362-2390, head 3630-3715) in float64 NumPy, calling no oracle arithmetic. Each test feeds the
oracle (oracle/model.cpp) and the float64 model the same state and inputs and compares the outputs
within north_star's floating-point bar: every element within 1e-3 of the largest magnitude of the
float64 result. `test_planted_mistakes_fail_the_bar` shows that each plausible wiring error
(key-head mapping, q / gate halves, entry concatenation order, shared-expert gate placement, decay,
gated-norm order) moves the result far past that bar, so the comparison pins the wiring.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O
from f64_model import F64Model, Mistake, f16

SEED = 23
TOL = 1e-3


def rel_err(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.abs(got - want).max() / np.abs(want).max())


@pytest.fixture(scope="module")
def desc():
    return O.desc_small()


@pytest.fixture(scope="module")
def f64(desc):
    return F64Model(desc, SEED)


def eng_arrays(e, d, n_ctx):
    """numpy views of the oracle engine's state: conv [slot][rec][nch][3], S [slot][rec][nv][hv][hv],
    K [att][kvh][n_ctx][hd] (f16 bits), V^T [att][kvh*hd][n_ctx] (f16 bits)."""
    L = O.lib()
    nch = d.ssm_d_inner + 2 * d.ssm_n_kheads * d.ssm_d_state
    hv = d.ssm_d_inner // d.ssm_n_vheads
    n_rec = d.n_layer - d.n_layer // d.full_attention_interval
    n_att = d.n_layer // d.full_attention_interval + (1 if d.has_mtp else 0)
    conv = np.ctypeslib.as_array(L.oxo_conv_state(e.h), (2, n_rec, nch, d.ssm_conv_kernel - 1))
    S = np.ctypeslib.as_array(L.oxo_ssm_state(e.h), (2, n_rec, d.ssm_n_vheads, hv, hv))
    K = np.ctypeslib.as_array(L.oxo_kcache_mut(e.h), (n_att, d.n_head_kv, n_ctx, d.head_dim))
    VT = np.ctypeslib.as_array(L.oxo_vcache_mut(e.h), (n_att, d.n_head_kv * d.head_dim, n_ctx))
    return conv, S, K, VT


def oracle_mixer(e, l, x, pos0):
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty_like(x)
    O.lib().oxo_mixer(e.h, l, x.shape[0], pos0, O.ptr(x, C.c_float), O.ptr(out, C.c_float))
    return out


def oracle_moe(e, l, x1):
    x1 = np.ascontiguousarray(x1, np.float32)
    out = np.empty_like(x1)
    O.lib().oxo_moe(e.h, l, x1.shape[0], O.ptr(x1, C.c_float), O.ptr(out, C.c_float))
    return out


def lanes_input(n, uid):
    return O.synth_normal(SEED, uid, n * 2048).reshape(n, 2048)


# ---- delta-net layer: two lanes, the second continuing from the first's state -----------------
def dn_case(desc, f64, mistakes=None):
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    conv, S, _, _ = eng_arrays(e, desc, e.n_ctx)
    rng = np.random.default_rng(5)
    conv[0, 0] = rng.standard_normal(conv[0, 0].shape).astype(np.float32)
    S[0, 0] = (0.1 * rng.standard_normal(S[0, 0].shape)).astype(np.float32)
    conv0, S0 = conv[0, 0].astype(np.float64), S[0, 0].astype(np.float64)
    x = lanes_input(2, 9001)
    got = oracle_mixer(e, 0, x, 0)
    m = f64 if mistakes is None else F64Model(desc, SEED, mistakes)
    m._w = f64._w
    cv, st = conv0.copy(), S0.copy()
    want, states = [], []
    for ln in range(2):
        want.append(m.dn_mixer(0, x[ln].astype(np.float64), cv, st))
        states.append((cv.copy(), st.copy()))
    res = dict(x1=(got, np.array(want)),
               conv=[(conv[ln, 0].copy(), states[ln][0]) for ln in range(2)],
               S=[(S[ln, 0].copy(), states[ln][1]) for ln in range(2)])
    e.close()
    return res


def test_delta_net_layer(desc, f64):
    r = dn_case(desc, f64)
    got, want = r["x1"]
    for ln in range(2):
        assert rel_err(got[ln], want[ln]) < TOL, ln
        # lane 0 writes slot cur (in place), lane 1 slot cur + 1 from lane 0's state (engine.rs:2491-2505)
        assert rel_err(*r["S"][ln]) < TOL, ln
        assert rel_err(*r["conv"][ln]) < TOL, ln


# ---- gated attention layer over 300 cached positions ------------------------------------------
def att_case(desc, f64, pos0=300, n_ctx=512, mistakes=None):
    e = O.Engine(desc, seed=SEED, n_ctx=n_ctx)
    _, _, K, VT = eng_arrays(e, desc, e.n_ctx)
    rng = np.random.default_rng(6)
    K[0, :, :pos0] = rng.standard_normal(K[0, :, :pos0].shape).astype(np.float16).view(np.uint16)
    VT[0, :, :pos0] = rng.standard_normal(VT[0, :, :pos0].shape).astype(np.float16).view(np.uint16)
    Kf = K[0].view(np.float16).astype(np.float64)
    Vf = VT[0].view(np.float16).astype(np.float64)
    x = lanes_input(2, 9002)
    l = desc.full_attention_interval - 1          # the first attention layer (att index 0)
    got = oracle_mixer(e, l, x, pos0)
    m = f64 if mistakes is None else F64Model(desc, SEED, mistakes)
    m._w = f64._w
    want = np.array([m.att_mixer(l, x[ln].astype(np.float64), pos0 + ln, Kf, Vf) for ln in range(2)])
    res = dict(x1=(got, want),
               K=(K[0, :, pos0:pos0 + 2].view(np.float16).copy(), Kf[:, pos0:pos0 + 2]),
               V=(VT[0, :, pos0:pos0 + 2].view(np.float16).copy(), Vf[:, pos0:pos0 + 2]))
    e.close()
    return res


def test_attention_layer(desc, f64):
    r = att_case(desc, f64)
    got, want = r["x1"]
    for ln in range(2):
        assert rel_err(got[ln], want[ln]) < TOL, ln
    # the new K rows (k_norm, RoPE at pos0 + lane) and V^T columns, both fp16
    for name in ("K", "V"):
        g, w = r[name]
        assert rel_err(g.astype(np.float64), w) < TOL, name


# ---- MoE layer: router, top-8, shared expert, combine ------------------------------------------
def moe_case(desc, f64, mistakes=None):
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    x1 = lanes_input(2, 9003)
    got = oracle_moe(e, 1, x1)
    m = f64 if mistakes is None else F64Model(desc, SEED, mistakes)
    m._w = f64._w
    want, routes = [], []
    for ln in range(2):
        x2, rt = m.moe(1, x1[ln].astype(np.float64), want_route=True)
        want.append(x2)
        routes.append(rt)
    e.close()
    return got, np.array(want), routes


def test_moe_layer(desc, f64):
    got, want, routes = moe_case(desc, f64)
    for ln in range(2):
        # the 8th and 9th probabilities are well apart, so float64 and the reference choose alike
        assert routes[ln]["margin"] > 1e-3
        assert rel_err(got[ln], want[ln]) < TOL, ln


# ---- whole decode steps, layer by layer, then the MTP head ------------------------------------
# Q8_0 activations make the model piecewise constant in its inputs: a 1e-7 difference upstream flips
# a few codes of the next quantised vector and moves that GEMV by ~3e-3. A float64 run chained on
# its own outputs therefore cannot meet 1e-3 after a few layers, whatever the wiring. Each piece is
# checked from the oracle's own input and state instead (teacher forcing): engine B is driven phase
# by phase through oxo_mixer / oxo_moe / oxo_mtp_entry, its final x2 feeds the float64 head, and
# engine A's plain steps (verify + commit) must return the same logits and hidden rows.
def oracle_entry(e, tok, h):
    t = np.array([tok], np.uint32)
    h = np.ascontiguousarray(h, np.float32).reshape(1, -1)
    x = np.empty_like(h)
    O.lib().oxo_mtp_entry(e.h, O.ptr(t, C.c_uint32), 1, O.ptr(h, C.c_float), O.ptr(x, C.c_float))
    return x


def test_decode_steps_and_mtp_head(desc, f64):
    toks = [101, 2047, 3333]
    A = O.Engine(desc, seed=SEED, n_ctx=256)
    B = O.Engine(desc, seed=SEED, n_ctx=256)
    conv, S, K, VT = eng_arrays(B, desc, B.n_ctx)

    def layer(l, x, pos):
        """oracle B's mixer + MoE of layer l at pos, each checked against float64 from the same
        input and state; returns B's x2"""
        xo = np.asarray(x, np.float32)[None, :]
        att = l == desc.n_layer or (l + 1) % desc.full_attention_interval == 0
        if att:
            ai = l // desc.full_attention_interval if l < desc.n_layer else K.shape[0] - 1
            Kf = K[ai].view(np.float16).astype(np.float64)
            Vf = VT[ai].view(np.float16).astype(np.float64)
            want1 = f64.att_mixer(l, xo[0].astype(np.float64), pos, Kf, Vf)
        else:
            ri = l - (l + 1) // desc.full_attention_interval
            cv, st = conv[0, ri].astype(np.float64), S[0, ri].astype(np.float64)
            want1 = f64.dn_mixer(l, xo[0].astype(np.float64), cv, st)
        x1 = oracle_mixer(B, l, xo, pos)
        assert rel_err(x1[0], want1) < TOL, (l, pos, "mixer")
        x2 = oracle_moe(B, l, x1)
        assert rel_err(x2[0], f64.moe(l, x1[0].astype(np.float64))) < TOL, (l, pos, "moe")
        return x2[0]

    for pos, t in enumerate(toks):
        g = A.step(t)
        x = f64.embed(t)                     # dequantisation is exact in f32: the oracle's own input
        for l in range(desc.n_layer):
            x = layer(l, x, pos)
        hout, logits = f64.head(x.astype(np.float64), O.GLOBAL_LAYER, O.T["OUT_NORM"])
        assert rel_err(A.hidden(0), hout) < TOL, pos
        assert rel_err(A.logits(0), logits) < TOL, pos
        top2 = np.sort(logits)[-2:]
        if top2[1] - top2[0] > 1e-2 * np.abs(logits).max():
            assert g == int(np.argmax(logits)), pos
    # MTP head at the next position: entry(token, h), the MTP attention layer (own KV) + its MoE,
    # the shared head behind head_norm
    h = A.hidden(0)
    t, pos, l = 77, len(toks), desc.n_layer
    d = A.mtp_run([t], pos, h[None, :])
    x = oracle_entry(B, t, h)[0]
    assert rel_err(x, f64.entry(t, h.astype(np.float64))) < TOL
    x = layer(l, x, pos)
    hout, logits = f64.head(x.astype(np.float64), l, O.T["HEAD_NORM"])
    assert rel_err(A.hidden(0), hout) < TOL
    assert rel_err(A.logits(0), logits) < TOL
    top2 = np.sort(logits)[-2:]
    if top2[1] - top2[0] > 1e-2 * np.abs(logits).max():
        assert d == int(np.argmax(logits))
    A.close()
    B.close()


# ---- each planted wiring mistake fails the bar ------------------------------------------------
def test_planted_mistakes_fail_the_bar(desc, f64):
    def worst(r):
        got, want = r["x1"]
        return max(rel_err(got[ln], want[ln]) for ln in range(2))

    for m in (Mistake.KEY_HEAD_DIV, Mistake.NO_DECAY, Mistake.ZNORM_ORDER):
        assert worst(dn_case(desc, f64, Mistake(m))) > 20 * TOL, m
    assert worst(att_case(desc, f64, mistakes=Mistake(Mistake.QGATE_SWAP))) > 20 * TOL
    got, want, _ = moe_case(desc, f64, Mistake(Mistake.SHGATE_ON_SUM))
    assert max(rel_err(got[ln], want[ln]) for ln in range(2)) > 20 * TOL
    # the MTP entry's concatenation order
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    h = O.synth_normal(SEED, 9004, 2048)
    x = oracle_entry(e, 5, h)[0]
    bad = F64Model(desc, SEED, Mistake(Mistake.ENTRY_SWAP))
    bad._w = f64._w
    assert rel_err(x, f64.entry(5, h.astype(np.float64))) < TOL
    assert rel_err(x, bad.entry(5, h.astype(np.float64))) > 20 * TOL
    e.close()


def test_f16_helper_rounds_like_the_cache():
    # the float64 model's fp16 rounding is numpy's IEEE conversion (round to nearest even)
    assert f16(1 + 2 ** -11) == 1.0 and f16(1 + 3 * 2 ** -11) == 1 + 2 ** -9
