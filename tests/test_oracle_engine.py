"""The oracle engine against the invariants the reference's own tests hold (no GPU).

  verify(n) == n single steps, bit for bit (crates/model/src/tests.rs:868-926)
  a rejected lane leaves no trace: verify([a, b]), commit(1) == step(a) (same file, random tails)
  MTP depth-1 greedy == plain greedy, with forced drafts hitting accept and reject
  (crates/model/src/tests.rs:1033-1117, draft_override hook mtp.rs:328-330)
on the 4-layer model with the 35B-A3B per-layer shapes (3 delta-net + 1 attention layer + MTP).
"""
import numpy as np
import pytest

import oracle as O

SEED = 11


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


@pytest.fixture(scope="module")
def desc():
    return O.desc_small()


def test_verify_equals_steps(desc):
    a = O.Engine(desc, seed=SEED, n_ctx=256)
    b = O.Engine(desc, seed=SEED, n_ctx=256)
    for toks in ([17, 3001], [5, 6], [4095, 0]):
        g = a.verify(toks)
        la = [a.logits(i) for i in range(2)]
        ha = [a.hidden(i) for i in range(2)]
        a.commit(2)
        for i, t in enumerate(toks):
            assert b.step(t) == g[i]
            assert np.array_equal(bits(b.logits(0)), bits(la[i]))
            assert np.array_equal(bits(b.hidden(0)), bits(ha[i]))
    assert a.pos == b.pos == 6


def test_rejected_lane_leaves_no_trace(desc):
    a = O.Engine(desc, seed=SEED, n_ctx=256)
    b = O.Engine(desc, seed=SEED, n_ctx=256)
    for x, rej, nxt in ((100, 2000, 7), (8, 9, 10), (77, 1234, 4000)):
        a.verify([x, rej])
        a.commit(1)
        ga = a.step(nxt)
        b.step(x)
        gb = b.step(nxt)
        assert ga == gb
        assert np.array_equal(bits(a.logits(0)), bits(b.logits(0)))
        assert np.array_equal(bits(a.hidden(0)), bits(b.hidden(0)))


def plain_greedy(desc, prompt, n):
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    x = None
    for t in prompt:
        x = e.step(int(t))
    out = []
    for _ in range(n):
        out.append(x)
        x = e.step(x)
    return out, x


def test_mtp_greedy_equals_plain_with_forced_drafts(desc):
    prompt = (O.bench_prompt(5) % desc.n_vocab).tolist()
    n = 14
    ref, _ = plain_greedy(desc, prompt, n + 2)
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    drv = O.Driver(e)
    x = drv.prefill(prompt)
    assert x == ref[0]
    got = [x]
    pattern = [1, 0, 1, 1, 0, 0, 1, 0, 1]   # 1: force the correct draft (accept), 0: a wrong one
    i = 0
    while len(got) < n:
        k = len(got)
        d1 = ref[k] if pattern[i % len(pattern)] else (ref[k] + 1) % desc.n_vocab
        out = drv.step(x, override_d1=d1)
        assert len(out) == (2 if pattern[i % len(pattern)] else 1)
        got += out
        x = out[-1]
        i += 1
    assert got[:n] == ref[:n]
    st = drv.stats()
    assert st["accepted"] == sum(pattern[j % len(pattern)] for j in range(i))


def test_rewind_and_step_plain_equal_plain_greedy(desc):
    """MtpDriver::rewind (mtp.rs:596-608): after an accepted step, keeping only x and continuing
    from the first greedy token is plain greedy again; step_plain (mtp.rs:504-515) interleaves."""
    prompt = (O.bench_prompt(5) % desc.n_vocab).tolist()
    ref, _ = plain_greedy(desc, prompt, 12)
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    drv = O.Driver(e)
    x = drv.prefill(prompt)
    got = [x]
    out = drv.step(x, override_d1=ref[1])        # accepted: commits x and d1
    assert out == ref[1:3]
    assert drv.rewind(3) == -1                   # more than the step committed
    assert drv.rewind(1) == 0                    # keep x only: the next token is ref[1] again
    x = out[0]
    got.append(x)
    x = drv.step_plain(x)
    got.append(x)
    out = drv.step(x, override_d1=(ref[4] + 1) % desc.n_vocab)   # rejected draft
    got += out
    x = out[-1]
    out = drv.step(x, override_d1=ref[5])
    got += out
    assert got == ref[: len(got)]


def test_four_lane_verify_equals_steps(desc):
    """the reference's verify width for MTP depth 3 (4 recurrent slots): verify(n) == n steps for
    n = 3, 4, and a partial commit leaves the state of the committed prefix"""
    a = O.Engine(desc, seed=SEED, n_ctx=256, lanes=4)
    b = O.Engine(desc, seed=SEED, n_ctx=256)
    for toks, m in (([17, 3001, 9], 3), ([5, 6, 7, 8], 4), ([40, 41, 42, 43], 2)):
        g = a.verify(toks)
        la = [a.logits(i) for i in range(m)]
        a.commit(m)
        for i, t in enumerate(toks[:m]):
            assert b.step(t) == g[i]
            assert np.array_equal(bits(b.logits(0)), bits(la[i]))
    assert a.pos == b.pos
    assert a.step(100) == b.step(100)
    assert np.array_equal(bits(a.logits(0)), bits(b.logits(0)))


@pytest.mark.parametrize("depth", [2, 3])
def test_mtp_depth_k_greedy_equals_plain(desc, depth):
    """MtpDriver at depth k (mtp.rs:522-592) with forced drafts through every acceptance count
    equals plain greedy decoding (crates/model/src/tests.rs:1033-1117)"""
    prompt = [int(v) % desc.n_vocab for v in O.bench_prompt(9)]
    ref, _ = plain_greedy(desc, prompt, 30)
    e = O.Engine(desc, seed=SEED, n_ctx=256, lanes=depth + 1)
    drv = O.Driver(e, depth)
    x = drv.prefill(prompt)
    out, k = [x], 0
    for a in [depth, 0, 1, depth, depth - 1, 0]:
        f = [ref[k + 1 + i] for i in range(a)] + ([(ref[k + 1 + a] + 1) % desc.n_vocab] if a < depth else [])
        r = drv.step(x, force=f + [-1] * (depth - len(f)))
        assert len(r) == a + 1
        out += r
        k += a + 1
        x = r[-1]
    assert out == ref[:len(out)]
    st = drv.stats()
    assert st["drafted"] == 6 * depth and st["accepted"] == sum([depth, 0, 1, depth, depth - 1, 0])


def test_tied_router_rows_take_the_sort_path(desc):
    # router rows duplicated in pairs: every probability appears twice, so every routing sorts; the
    # engine invariants still hold on that path
    a = O.Engine(desc, seed=SEED, n_ctx=256)
    b = O.Engine(desc, seed=SEED, n_ctx=256)
    for layer in range(desc.n_layer + 1):
        r = O.synth_f32(SEED, layer, O.T["ROUTER"], 256 * desc.n_embd).reshape(256, desc.n_embd)
        r[1::2] = r[0::2]
        a.set_router(layer, 0, r)
        b.set_router(layer, 0, r)
    g = a.verify([17, 3001])
    la = a.logits(1)
    a.commit(2)
    assert b.step(17) == g[0]
    assert b.step(3001) == g[1]
    assert np.array_equal(bits(b.logits(0)), bits(la))
    assert O.lib().oxo_tie_count(a.h) >= desc.n_layer * 2


def test_read_state_handoff(desc):
    # Engine::read_state of write_state-ordered bytes continues exactly like the original engine
    import ctypes as C
    L = O.lib()
    a = O.Engine(desc, seed=SEED, n_ctx=256)
    for t in (5, 900, 31, 4000, 12):
        a.step(t)
    n, nc, hd, nkv = a.pos, int(a.n_ctx), desc.head_dim, desc.n_head_kv
    n_att = desc.n_layer // desc.full_attention_interval + 1
    n_rec = desc.n_layer - (n_att - 1)
    kc = np.ctypeslib.as_array(L.oxo_kcache(a.h), (n_att * nkv * nc * hd,)).reshape(n_att, nkv, nc, hd)
    vc = np.ctypeslib.as_array(L.oxo_vcache(a.h), (n_att * nkv * hd * nc,)).reshape(n_att, nkv * hd, nc)
    conv_len, ssm_len = n_rec * 8192 * 3, n_rec * 32 * 128 * 128
    cur = L.oxo_cur_slot(a.h)
    conv = np.ctypeslib.as_array(L.oxo_conv_state(a.h), (2 * conv_len,))[cur * conv_len:(cur + 1) * conv_len]
    ssm = np.ctypeslib.as_array(L.oxo_ssm_state(a.h), (2 * ssm_len,))[cur * ssm_len:(cur + 1) * ssm_len]
    parts = []
    for ai in range(n_att):
        for h in range(nkv):
            parts.append(kc[ai, h, :n].tobytes())
        parts.append(np.ascontiguousarray(vc[ai, :, :n]).tobytes())
    blob = np.frombuffer(b"".join(parts) + conv.tobytes() + ssm.tobytes(), np.uint8)
    b = O.Engine(desc, seed=SEED, n_ctx=256)
    b.read_state(blob, n)
    assert b.pos == n
    assert L.oxo_engine_read_state(b.h, blob.ctypes.data_as(C.c_void_p), blob.nbytes - 1, n) == -1
    for t in (77, 3):
        assert a.step(t) == b.step(t)
        assert np.array_equal(bits(a.logits(0)), bits(b.logits(0)))


def test_pinned_team_same_bits_and_restores_mask(desc):
    # oxo_pin_team pins team thread i to the i-th CPU of the caller's mask (the reference's pool,
    # crates/sched/src/lib.rs:1-11) and restores the caller's mask; placement never changes a value
    import os
    L = O.lib()
    before = os.sched_getaffinity(0)
    a = O.Engine(desc, seed=SEED, n_ctx=64)
    b = O.Engine(desc, seed=SEED, n_ctx=64)
    want = [a.step(t) for t in (5, 900, 31)]
    try:
        team = L.oxo_pin_team(1)
        assert team >= 1
        if len(before) > 1:
            assert os.sched_getaffinity(0) == {sorted(before)[0]}
        got = [b.step(t) for t in (5, 900, 31)]
    finally:
        assert L.oxo_pin_team(0) == 0
    assert os.sched_getaffinity(0) == before
    assert got == want
    assert np.array_equal(bits(a.logits(0)), bits(b.logits(0)))
    assert np.array_equal(bits(a.hidden(0)), bits(b.hidden(0)))
