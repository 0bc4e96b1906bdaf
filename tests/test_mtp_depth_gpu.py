"""MTP depth 2 and 3 (MtpDriver::step with depth k, crates/model/src/mtp.rs:522-592) on the GPU
against the oracle's driver at the same depth.

The draft chain runs the MTP head k times; the verify of [x, d_1..d_k] runs here in pieces of at
most two lanes, committed one after the other and stopped at the first rejected draft. Forced drafts
(the reference's draft_override hook, mtp.rs:554-558) walk the plain greedy sequence through every
acceptance count 0..k; tokens, driver state (the next steps) and counters must equal the oracle's,
and the greedy output must equal plain greedy decoding (crates/model/src/tests.rs:1033-1117)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

SEED = 5
N_CTX = 512


@pytest.fixture(scope="module")
def setup():
    d = O.desc_small()
    prompt = [int(v) % d.n_vocab for v in O.bench_prompt(13)]
    e = O.Engine(d, seed=SEED, n_ctx=N_CTX)
    x = None
    for t in prompt:
        x = e.step(t)
    plain = [x]
    for _ in range(60):
        x = e.step(x)
        plain.append(x)
    e.close()
    return d, prompt, plain


def forces_for(plain, k, a, depth, n_vocab):
    """drafts for a step from plain[k]: the first a correct, the (a+1)-th wrong, the rest the head's"""
    f = [plain[k + 1 + i] for i in range(a)]
    if a < depth:
        f.append((plain[k + 1 + a] + 1) % n_vocab)
    return f + [-1] * (depth - len(f))


@pytest.mark.parametrize("depth", [2, 3])
def test_forced_steps_match_oracle_and_plain_greedy(setup, depth):
    import oxe_amd as A
    d, prompt, plain = setup
    g = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    g.mtp_set_depth(depth)
    o = O.Engine(d, seed=SEED, n_ctx=N_CTX, lanes=depth + 1)   # the reference's (k+1)-lane verify
    od = O.Driver(o, depth)
    x = g.mtp_prefill(prompt)
    assert od.prefill(prompt) == x == plain[0]
    pattern = [depth, 0, 1, depth, depth - 1, 2, 0, depth] if depth == 3 else [2, 0, 1, 2, 1, 0, 2, 2]
    k = 0
    for a in pattern:
        f = forces_for(plain, k, a, depth, d.n_vocab)
        print(f"depth {depth} step at {k}: accept {a}", flush=True)
        rg, ro = g.mtp_step_force(x, f), od.step(x, force=f)
        assert rg == ro == plain[k + 1: k + 2 + a]
        k += a + 1
        x = rg[-1]
    # unforced steps: the head's own drafts (random weights: nearly always rejected)
    for _ in range(4):
        rg, ro = g.mtp_step_force(x, []), od.step(x, force=[])
        assert rg == ro == plain[k + 1: k + 1 + len(rg)]
        k += len(rg)
        x = rg[-1]
    st, so = g.mtp_stats(), od.stats()
    assert (st["steps"], st["drafted"], st["accepted"]) == (so["steps"], so["drafted"], so["accepted"])
    assert g.pos == o.pos
    g.close()
    o.close()


def test_depth3_rewind_matches_oracle(setup):
    """rewind after a depth-3 step that committed x and three drafts (keep 2), then continue"""
    import oxe_amd as A
    d, prompt, plain = setup
    g = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    g.mtp_set_depth(3)
    o = O.Engine(d, seed=SEED, n_ctx=N_CTX, lanes=4)
    od = O.Driver(o, 3)
    x = g.mtp_prefill(prompt)
    od.prefill(prompt)
    f = plain[1:4]
    assert g.mtp_step_force(x, f) == od.step(x, force=f) == plain[1:5]
    g.mtp_rewind(2)
    assert od.rewind(2) == 0
    assert g.pos == o.pos
    x, k = plain[2], 2                       # x and plain[1] kept: plain[2] is the next input
    for a in (3, 1, 0):
        f = forces_for(plain, k, a, 3, d.n_vocab)
        rg, ro = g.mtp_step_force(x, f), od.step(x, force=f)
        assert rg == ro == plain[k + 1: k + 2 + a]
        k += a + 1
        x = rg[-1]
    g.close()
    o.close()


def test_server_spec_depth(setup):
    """the server's decode_spec_argmax / decode_spec at depth 2 and 3 equal plain greedy decoding,
    rows bit for bit; the device-driven step refuses a depth above 1"""
    import oxe_amd as A
    d, prompt, plain = setup
    sp = A.ServerEngine(A.Engine(d, seed=SEED, n_ctx=N_CTX), mtp=False)
    sp.prefill(prompt)
    for depth in (2, 3):
        s = A.ServerEngine(A.Engine(d, seed=SEED, n_ctx=N_CTX), mtp=True)
        assert s.spec_max_depth() == 3
        s.spec_set_depth(depth)
        x = int(np.argmax(s.prefill(prompt)))
        out = [x]
        while len(out) < 12:
            extra, gg = s.decode_spec_argmax(x)
            assert extra == gg[:-1] and 1 <= len(gg) <= depth + 1
            out += gg
            x = gg[-1]
        assert out == plain[:len(out)]
        drafted, _ = s.spec_counters()
        assert drafted % depth == 0 and drafted > 0
    # rows of a depth-3 step against plain decode rows (a fresh pair of engines)
    s = A.ServerEngine(A.Engine(d, seed=SEED, n_ctx=N_CTX), mtp=True)
    s.spec_set_depth(3)
    x = int(np.argmax(s.prefill(prompt)))
    for _ in range(3):
        extra, rows = s.decode_spec(x)
        for t, r in zip([x] + extra, rows):
            assert np.array_equal(sp.decode(t).view(np.uint32), r.view(np.uint32))
        x = int(np.argmax(rows[-1]))
    g = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    g.mtp_set_depth(3)   # the device-driven step runs depth 1 or 2
    with pytest.raises(RuntimeError):
        g.mtp_device_begin(plain[0], 8)


def depth2_engine(d, mode):
    import oxe_amd as A
    g = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    if mode == "per_phase":
        g.set_fused(False)
    elif not g.fused:
        g.close()
        pytest.skip("the fused run kernel needs a 256-CU device")
    g.mtp_set_depth(2)
    return g


@pytest.mark.parametrize("mode", ["fused", "per_phase"])
def test_device_depth2_forced_matches_oracle(setup, mode):
    """Device-driven depth-2 steps (two drafts, verify pieces (x, d1) then (d2), all decided on the
    GPU) with forced drafts through every acceptance count, against the oracle's depth-2 driver:
    tokens, counters and position; then host-driven steps continue from the handed-back state (its
    pending catch-up pairs) exactly as the oracle's driver does."""
    d, prompt, plain = setup
    g = depth2_engine(d, mode)
    o = O.Engine(d, seed=SEED, n_ctx=N_CTX, lanes=3)
    od = O.Driver(o, 2)
    x = g.mtp_prefill(prompt)
    assert od.prefill(prompt) == x == plain[0]
    pattern = [2, 0, 1, 2, 1, 0, 2, 2, 1, 1]
    forces, want, k, xo = [], [], 0, x
    for a in pattern:
        f = forces_for(plain, k, a, 2, d.n_vocab)
        forces += f
        ro = od.step(xo, force=f)
        assert ro == plain[k + 1: k + 2 + a]
        want += ro
        k += a + 1
        xo = ro[-1]
    g.mtp_set_force(forces)
    g.mtp_device_begin(x, 64)
    g.mtp_device_steps(len(pattern), use_graph=True)
    toks, nx = g.mtp_device_end(64)
    assert toks == want
    assert nx == xo
    st, so = g.mtp_stats(), od.stats()
    assert (st["steps"], st["drafted"], st["accepted"]) == (so["steps"], so["drafted"], so["accepted"])
    assert g.pos == o.pos
    g.mtp_set_force([])
    for _ in range(3):
        rg, ro = g.mtp_step_force(nx, []), od.step(xo, force=[])
        assert rg == ro == plain[k + 1: k + 1 + len(rg)]
        k += len(rg)
        nx, xo = rg[-1], ro[-1]
    assert np.array_equal(np.asarray(g.hidden(0), np.float32).view(np.uint32), o.hidden(0).view(np.uint32))
    g.close()
    o.close()


@pytest.mark.parametrize("mode", ["fused", "per_phase"])
def test_device_depth2_natural_drafts(setup, mode):
    """Unforced device-driven depth-2 steps (the head's own drafts): eager and graph launches agree,
    and both equal the oracle's depth-2 driver and plain greedy decoding."""
    d, prompt, plain = setup
    o = O.Engine(d, seed=SEED, n_ctx=N_CTX, lanes=3)
    od = O.Driver(o, 2)
    xo = od.prefill(prompt)
    want = []
    for _ in range(6):
        ro = od.step(xo, force=[])
        want += ro
        xo = ro[-1]
    o.close()
    for use_graph in (False, True):
        g = depth2_engine(d, mode)
        x = g.mtp_prefill(prompt)
        g.mtp_device_begin(x, 64)
        g.mtp_device_steps(6, use_graph=use_graph)
        toks, nx = g.mtp_device_end(64)
        assert toks == want == plain[1:1 + len(want)]
        assert nx == xo
        assert g.mtp_stats()["drafted"] == 12
        g.close()

