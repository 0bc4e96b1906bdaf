"""Batched prefill on the GPU (Engine::prefill_ext, crates/model/src/engine/prefill.rs:763;
MtpDriver::prefill_batched, mtp.rs:468-500) against token-by-token decoding.

The reference gates its batched prefill on bit-identity with llama.cpp's batched prefill, which for
all-Q8_0 weights equals decoding token by token (docs/lab-notes/M3-PREFILL.md:55-75: Q8_0 GEMM ==
GEMV, conv / delta rule / attention per token in decode order). Bar here: the KV cache, the conv
and delta-net state, every position's h_nextn, the last token's logits and the argmax bit-exact
against (a) the CPU oracle stepping token by token and (b) this engine's own decode path (itself
pinned to the oracle by test_engine_gpu.py), at lengths that cross the 256-position softmax pads,
the 64-token GEMM tiles and the 2048-token prefill chunk, from position 0 and from the middle of
a context, and with decoding continued afterwards."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

SEED = 7
HD, NKV, NCH, NVH, HV = 256, 2, 8192, 32, 128


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def engine(d, n_ctx, fused=True):
    import oxe_amd as A
    g = A.Engine(d, seed=SEED, n_ctx=n_ctx)
    if not fused:
        g.set_fused(False)
    return g


def prompt(d, n, salt=0):
    return [int(v) % d.n_vocab for v in O.bench_prompt(n + salt)[salt:]]


def state(g, d, main_only=False):
    """(K cache, V^T cache, conv state, delta-net state) of the current slot, as arrays; main_only:
    the K / V^T of the main attention layers only (not the MTP layer's)"""
    n_att = sum(1 for i in range(d.n_layer) if (i + 1) % d.full_attention_interval == 0) + 1
    n_rec = d.n_layer - (n_att - 1)
    n_ctx = g.n_ctx
    kv = (n_att - (1 if main_only else 0)) * NKV * n_ctx * HD * 2
    return (g.state(0, kv, dtype=np.uint16), g.state(1, kv, dtype=np.uint16),
            g.state(2, n_rec * NCH * 3 * 4, dtype=np.uint32), g.state(3, n_rec * NVH * HV * HV * 4, dtype=np.uint32))


def assert_same_state(ga, gb, d, what, main_only=False):
    for name, a, b in zip(("K", "V^T", "conv", "ssm"), state(ga, d, main_only), state(gb, d, main_only)):
        assert np.array_equal(a, b), f"{what}: {name} differs at {np.flatnonzero(a != b)[:8]}"


def decode(g, toks):
    """token-by-token steps; returns the last argmax and every step's h_nextn"""
    hs, x = [], None
    for t in toks:
        x = g.step(t)
        hs.append(g.hidden(0))
    return x, np.stack(hs)


@pytest.mark.parametrize("n", [1, 2, 3, 37, 300])
def test_prefill_equals_decode(n):
    d = O.desc_small()
    toks = prompt(d, n)
    a, b = engine(d, 512), engine(d, 512)
    print(f"prefill n={n}", flush=True)
    nx, h = a.prefill(toks, hidden=True)
    x, hs = decode(b, toks)
    assert nx == x
    assert a.pos == b.pos == n
    assert np.array_equal(bits(h), bits(hs)), f"h_nextn rows differ: {sorted(set(np.nonzero(bits(h) != bits(hs))[0]))[:8]}"
    assert np.array_equal(bits(a.hidden(0)), bits(b.hidden(0)))
    assert np.array_equal(bits(a.logits(0)), bits(b.logits(0)))
    assert_same_state(a, b, d, f"n={n}")
    # decoding continues from the prefilled state exactly
    for _ in range(3):
        nx, x = a.step(nx), b.step(x)
        assert nx == x
        assert np.array_equal(bits(a.logits(0)), bits(b.logits(0)))
    a.close()
    b.close()


def test_prefill_equals_oracle():
    d = O.desc_small()
    toks = prompt(d, 29, salt=3)
    g, o = engine(d, 256), O.Engine(d, seed=SEED, n_ctx=256)
    print("prefill vs oracle n=29", flush=True)
    nx, h = g.prefill(toks, hidden=True)
    x = None
    for i, t in enumerate(toks):
        x = o.step(t)
        assert np.array_equal(bits(h[i]), bits(o.hidden(0))), f"h_nextn of position {i}"
    assert nx == x
    assert np.array_equal(bits(g.logits(0)), bits(o.logits(0)))
    n_ctx = g.n_ctx
    kg = g.state(0, 2 * NKV * n_ctx * HD * 2, dtype=np.uint16)
    ko = np.ctypeslib.as_array(O.lib().oxo_kcache(o.h), (2 * NKV * n_ctx * HD,))
    assert np.array_equal(kg, ko)
    vg = g.state(1, 2 * NKV * n_ctx * HD * 2, dtype=np.uint16)
    vo = np.ctypeslib.as_array(O.lib().oxo_vcache(o.h), (2 * NKV * n_ctx * HD,))
    assert np.array_equal(vg, vo)
    g.close()
    o.close()


@pytest.mark.parametrize("fused", [True, False])
def test_prefill_mid_context(fused):
    """prefill after decode steps and after another prefill (conv window and attention over the
    earlier positions), in both decode run modes"""
    d = O.desc_small()
    a, b = engine(d, 768, fused), engine(d, 768, fused)
    if fused and not a.fused:
        pytest.skip("the fused run kernel needs a 256-CU device")
    p1, p2, p3 = prompt(d, 20), prompt(d, 45, salt=20), prompt(d, 260, salt=65)
    print(f"mid-context prefill fused={fused}", flush=True)
    for t in p1:
        assert a.step(t) == b.step(t)
    nx = a.prefill(p2)
    x, _ = decode(b, p2)
    assert nx == x
    nx = a.prefill(p3)
    x, _ = decode(b, p3)
    assert nx == x
    assert a.pos == b.pos == 325
    assert np.array_equal(bits(a.logits(0)), bits(b.logits(0)))
    assert_same_state(a, b, d, "mid-context")
    for _ in range(2):
        nx, x = a.step(nx), b.step(x)
        assert nx == x
    a.close()
    b.close()


def test_prefill_across_chunks():
    """2100 tokens: two prefill chunks (2048 + 52), softmax rows up to 2304 positions"""
    d = O.desc_small()
    toks = prompt(d, 2100, salt=1)
    a, b = engine(d, 2304), engine(d, 2304)
    print("prefill n=2100", flush=True)
    nx = a.prefill(toks)
    x = None
    for i in range(0, 2100, 2):
        g = b.verify(toks[i:i + 2])
        b.commit(2)
        x = int(g[-1])
    assert nx == x
    assert np.array_equal(bits(a.logits(0)), bits(b.logits(1)))   # the last verify's second lane
    assert np.array_equal(bits(a.hidden(0)), bits(b.hidden(1)))
    assert_same_state(a, b, d, "2100 tokens")
    a.close()
    b.close()


def test_prefill_per_head_attention_path():
    """5000 tokens: the third chunk's score rows reach 5120 positions, beyond the kv-head-shared
    kernel's LDS (4800), so its attention runs on the per-head kernel; equal to 2-token verify
    decoding bit for bit (logits, hidden state, KV and recurrent state)"""
    d = O.desc_small()
    n = 5000
    toks = prompt(d, n, salt=3)
    a, b = engine(d, 5120), engine(d, 5120)
    print(f"prefill n={n}", flush=True)
    nx = a.prefill(toks)
    x = None
    for i in range(0, n, 2):
        g = b.verify(toks[i:i + 2])
        b.commit(2)
        x = int(g[-1])
    assert nx == x
    assert np.array_equal(bits(a.logits(0)), bits(b.logits(1)))
    assert np.array_equal(bits(a.hidden(0)), bits(b.hidden(1)))
    assert_same_state(a, b, d, f"{n} tokens")
    a.close()
    b.close()


def test_mtp_prefill_batched_equals_mtp_prefill():
    """MtpDriver::prefill_batched: the same target state, MTP KV and speculative steps as the
    2-token-verify prompt path"""
    d = O.desc_small()
    toks = prompt(d, 90, salt=5)
    a, b = engine(d, 512), engine(d, 512)
    print("mtp prefill batched n=90", flush=True)
    xa, xb = a.mtp_prefill_batched(toks), b.mtp_prefill(toks)
    assert xa == xb
    # the MTP KV may differ by the pairs still pending (seeded in batches vs in pairs) until the
    # next step seeds all of them
    assert_same_state(a, b, d, "after the MTP prefill", main_only=True)
    for _ in range(6):
        oa, ob = a.mtp_step(xa), b.mtp_step(xb)
        assert oa == ob
        xa, xb = oa[-1], ob[-1]
    assert_same_state(a, b, d, "after MTP steps")
    a.close()
    b.close()


def test_prefill_rejects_bad_arguments():
    d = O.desc_small()
    g = engine(d, 256)
    for toks in ([], [d.n_vocab], list(range(257))):
        with pytest.raises(RuntimeError):
            g.prefill(toks)
    assert g.pos == 0
    g.close()


def oracle_state_bytes(o, d):
    """Engine::write_state (engine.rs:1682-1722) assembled from the oracle's arrays: per attention
    layer the K rows of positions < pos per KV head, then the V^T rows; then the current slot's conv
    state and S."""
    n, n_ctx = o.pos, int(o.n_ctx)
    n_att = sum(1 for i in range(d.n_layer) if (i + 1) % d.full_attention_interval == 0) + 1
    n_rec = d.n_layer - (n_att - 1)
    kc = np.ctypeslib.as_array(O.lib().oxo_kcache(o.h), (n_att * NKV * n_ctx * HD,)).reshape(n_att, NKV, n_ctx, HD)
    vc = np.ctypeslib.as_array(O.lib().oxo_vcache(o.h), (n_att * NKV * HD * n_ctx,)).reshape(n_att, NKV * HD, n_ctx)
    conv_len, ssm_len = n_rec * NCH * 3, n_rec * NVH * HV * HV
    cur = O.lib().oxo_cur_slot(o.h)
    conv = np.ctypeslib.as_array(O.lib().oxo_conv_state(o.h), (2 * conv_len,))[cur * conv_len:(cur + 1) * conv_len]
    ssm = np.ctypeslib.as_array(O.lib().oxo_ssm_state(o.h), (2 * ssm_len,))[cur * ssm_len:(cur + 1) * ssm_len]
    parts = []
    for ai in range(n_att):
        for h in range(NKV):
            parts.append(kc[ai, h, :n].tobytes())
        parts.append(np.ascontiguousarray(vc[ai, :, :n]).tobytes())
    parts += [conv.tobytes(), ssm.tobytes()]
    return np.frombuffer(b"".join(parts), np.uint8)


def test_write_state_reference_order():
    """write_state after a batched prefill = the oracle's state after token-by-token steps, in the
    reference's byte order; state_bytes is the reference's formula"""
    d = O.desc_small()
    toks = prompt(d, 23, salt=9)
    g, o = engine(d, 256), O.Engine(d, seed=SEED, n_ctx=256)
    print("write_state n=23", flush=True)
    g.prefill(toks)
    for t in toks:
        o.step(t)
    got, want = g.write_state(), oracle_state_bytes(o, d)
    assert got.size == want.size == 2 * NKV * 4 * HD * 23 + 4 * 3 * (NCH * 3 + NVH * HV * HV)
    assert np.array_equal(got, want), f"first differing byte {np.flatnonzero(got != want)[:4]}"
    g.close()
    o.close()


def test_read_state_handoff_continues_exactly():
    """prefill on one engine, hand the state to another (read_state), decode on both: identical
    tokens and logits; a shorter state read into an engine that held a longer sequence zeroes the
    tail of V^T and decodes like a fresh engine"""
    d = O.desc_small()
    toks = prompt(d, 140, salt=2)
    a, b, c = engine(d, 512), engine(d, 512), engine(d, 512)
    print("read_state hand-off n=140", flush=True)
    nx = a.prefill(toks)
    blob = a.write_state()
    b.read_state(blob, len(toks))
    assert b.pos == a.pos == 140
    x = nx
    for _ in range(4):
        x1, x2 = a.step(x), b.step(x)
        assert x1 == x2
        assert np.array_equal(bits(a.logits(0)), bits(b.logits(0)))
        x = x1
    # c runs a longer sequence first, then takes the 140-token state: same continuation as a fresh read
    c.prefill(prompt(d, 300, salt=7))
    c.read_state(blob, len(toks))
    fresh = engine(d, 512)
    fresh.read_state(blob, len(toks))
    # the state of positions < 140 and every V^T column (the tail back to +0) match a fresh read;
    # K rows past the position are never read and are not cleared (as in the reference)
    assert np.array_equal(c.write_state(), fresh.write_state())
    assert np.array_equal(state(c, d)[1], state(fresh, d)[1])
    assert c.step(nx) == fresh.step(nx)
    assert np.array_equal(bits(c.logits(0)), bits(fresh.logits(0)))
    with pytest.raises(RuntimeError):
        c.read_state(blob[:-1], len(toks))
    for g in (a, b, c, fresh):
        g.close()
