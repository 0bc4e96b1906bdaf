"""Routing with exactly tied probabilities on the GPU, bit for bit against the oracle.

The reference takes top-8 by std::sort of all 256 indices with x[a] > x[b] whenever the 9 largest
probabilities are not strictly distinct (crates/kernels-sys/csrc/oxe_ops.cpp:157-164); std::sort is
not stable, so tied experts come out in libstdc++'s order (the oracle calls the host's std::sort; the
device restates the algorithm, oxe_stdsort.h, itself checked against std::sort in test_stdsort.py).
  * kernel level (oxe_hip_route_f32): rows of logits with duplicated values — all equal, pairs, a
    repeated 9th value, few distinct levels — ids and weights against the oracle's softmax, top-k
    and renormalisation;
  * engine level, both run modes: every layer's router rows duplicated in pairs (row 2i + 1 = row
    2i, so every probability appears twice and each routing takes the sort path) or in threes (the
    8th and 9th probabilities are then always equal: the sort decides which experts run, not only
    their order); the MTP prefill and device-driven steps return the oracle's tokens, logits and
    hidden rows bit for bit.
"""
import ctypes as C

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

SEED = 17


def oracle_route(lg):
    L = O.lib()
    n = 256
    x = np.ascontiguousarray(lg, np.float32)
    p = np.empty(n, np.float32)
    wp = np.empty(n, np.float32)
    L.oxo_soft_max_f32(n, O.ptr(p, C.c_float), O.ptr(x, C.c_float), np.float32(1.0), None, O.ptr(wp, C.c_float))
    ids = np.empty(8, np.int32)
    scr = np.empty(n, np.int32)
    tie = C.c_int(0)
    L.oxo_argsort_top_k_f32(O.ptr(p, C.c_float), n, 8, O.ptr(ids, C.c_int32), O.ptr(scr, C.c_int32), C.byref(tie))
    w = p[ids].copy()
    s = np.float32(L.oxo_vec_sum_f32(8, O.ptr(w, C.c_float)))
    s = max(min(s, np.float32(np.inf)), np.float32(6.103515625e-5))
    return ids, (w / s).astype(np.float32), tie.value


def tie_rows():
    rng = np.random.default_rng(3)
    rows = [np.zeros(256, np.float32)]                                     # 256-way tie
    r = rng.standard_normal(128).astype(np.float32)
    rows.append(np.repeat(r, 2))                                           # every value twice, adjacent
    rows.append(np.concatenate([r, r[::-1]]))                              # pairs far apart
    r = rng.standard_normal(256).astype(np.float32)
    top = np.argsort(-r)
    r[top[8]] = r[top[7]]                                                  # the 9th equals the 8th
    rows.append(r)
    r = rng.standard_normal(256).astype(np.float32)
    top = np.argsort(-r)
    r[top[20]] = r[top[3]]                                                 # a value ranked 4th repeats lower down
    rows.append(r)
    for levels in (2, 3, 7, 40):
        rows.append((rng.integers(0, levels, 256) * 0.37).astype(np.float32))
    rows.append(rng.standard_normal(256).astype(np.float32))              # no tie (fast path)
    return np.stack(rows)


def test_route_kernel_ties_bitexact(dev):
    import torch
    import oxe_amd as A
    lg = tie_rows()
    tc = torch.zeros(1, dtype=torch.int32, device=dev)
    ids, w = A.route_f32(torch.from_numpy(lg).to(dev), tc)
    torch.cuda.synchronize()
    ids, w = ids.cpu().numpy(), w.cpu().numpy()
    ties = 0
    for i, row in enumerate(lg):
        oi, ow, tie = oracle_route(row)
        ties += tie
        assert list(ids[i]) == list(oi), (i, list(ids[i]), list(oi))
        assert np.array_equal(w[i].view(np.uint32), ow.view(np.uint32)), i
    assert ties == len(lg) - 1 and int(tc.item()) == ties


def copied_router(d, layer, copies):
    r = O.synth_f32(SEED, layer, O.T["ROUTER"], 256 * d.n_embd).reshape(256, d.n_embd)
    for j in range(1, copies):
        r[j::copies] = r[0::copies][: len(r[j::copies])]
    return r


@pytest.mark.parametrize("copies", [2, 3])
@pytest.mark.parametrize("mode", ["fused", "per_phase"])
def test_engine_with_tied_routers_bitexact(dev, mode, copies):
    import oxe_amd as A
    d = O.desc_small()
    g = A.Engine(d, seed=SEED, n_ctx=256)
    if mode == "per_phase":
        g.set_fused(False)
    elif not g.fused:
        pytest.skip("the fused run kernel needs a 256-CU device")
    o = O.Engine(d, seed=SEED, n_ctx=256)
    for layer in range(d.n_layer + 1):
        r = copied_router(d, layer, copies)
        g.set_router(layer, 0, r)
        o.set_router(layer, 0, r)
    prompt = O.bench_prompt(7) % d.n_vocab
    drv = O.Driver(o)
    xg, xo = g.mtp_prefill(prompt), drv.prefill(prompt)
    assert xg == xo
    cap = 32
    g.mtp_device_begin(xg, cap)
    g.mtp_device_steps(4, use_graph=True)
    toks_g, x_next = g.mtp_device_end(cap)
    toks_o, x = [], xo
    for _ in range(4):
        out = drv.step(x)
        toks_o += list(out)
        x = out[-1]
    assert list(toks_g) == toks_o and x_next == x
    assert np.array_equal(np.asarray(g.hidden(0), np.float32).view(np.uint32), o.hidden(0).view(np.uint32))
    assert g.counter(64) > 0          # the sort path ran
    assert O.lib().oxo_tie_count(o.h) > 0
    # a plain verify of two lanes: logits of both lanes
    pos = g.pos
    assert o.pos == pos
    vg, vo = g.verify([11, 4000]), o.verify([11, 4000])
    assert list(vg) == list(vo)
    for ln in range(2):
        assert np.array_equal(np.asarray(g.logits(ln), np.float32).view(np.uint32), o.logits(ln).view(np.uint32)), ln
    g.close()
    o.close()
