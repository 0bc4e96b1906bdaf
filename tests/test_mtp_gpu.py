"""MTP depth-1 speculative decoding on the GPU against the oracle's MtpDriver (mtp.rs:314-608).

Reference tests mirrored: MTP greedy == plain greedy with forced drafts hitting every acceptance
length (crates/model/src/tests.rs:1033-1117); the device-driven step (accept/rollback on the GPU)
equals the host-driven one."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

SEED = 5
N_CTX = 512


def plain_greedy(d, prompt, n):
    e = O.Engine(d, seed=SEED, n_ctx=N_CTX)
    x = None
    for t in prompt:
        x = e.step(int(t))
    out = [x]
    for _ in range(n):
        x = e.step(x)
        out.append(x)
    e.close()
    return out


def forced_drafts(plain, pattern):
    """Walk the plain greedy sequence: step s forces the correct draft when pattern[s] else a wrong one."""
    forces, k = [], 0
    for acc in pattern:
        correct = plain[k + 1]
        forces.append(correct if acc else (correct + 1) % 4096)
        k += 2 if acc else 1
    return forces


@pytest.fixture(params=["fused", "per_phase"])
def mode(request):
    return request.param


def engine(d, mode):
    """A device engine in the given run mode (fused: one persistent launch per run)."""
    import oxe_amd as A
    g = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    if mode == "per_phase":
        g.set_fused(False)
    elif not g.fused:
        pytest.skip("the fused run kernel needs a 256-CU device")
    return g


@pytest.fixture(scope="module")
def setup():
    d = O.desc_small()
    prompt = O.bench_prompt(11) % d.n_vocab
    pattern = [1, 0, 1, 1, 0, 0, 1, 0]
    plain = plain_greedy(d, prompt, 2 * len(pattern) + 2)
    return d, prompt, pattern, plain, forced_drafts(plain, pattern)


def test_host_driver_matches_oracle_and_plain_greedy(setup, mode):
    d, prompt, pattern, plain, forces = setup
    g = engine(d, mode)
    o = O.Engine(d, seed=SEED, n_ctx=N_CTX)
    od = O.Driver(o)
    xg, xo = g.mtp_prefill(prompt), od.prefill(prompt)
    assert xg == xo == plain[0]
    out = []
    for f in forces:
        rg, ro = g.mtp_step(xg, f), od.step(xo, f)
        assert rg == ro
        out += rg
        xg, xo = rg[-1], ro[-1]
    assert out == plain[1:1 + len(out)]
    assert g.mtp_stats()["accepted"] == sum(pattern)
    assert np.array_equal(g.hidden(0).view(np.uint32), o.hidden(0).view(np.uint32))
    assert g.pos == o.pos


def test_device_driver_matches_host_driver(setup, mode):
    d, prompt, pattern, plain, forces = setup
    g = engine(d, mode)
    x = g.mtp_prefill(prompt)
    g.mtp_set_force(forces)
    g.mtp_device_begin(x, 64)
    g.mtp_device_steps(len(forces), use_graph=True)
    toks, nx = g.mtp_device_end(64)
    assert toks == plain[1:1 + len(toks)]
    assert nx == toks[-1]
    assert len(toks) == len(forces) + sum(pattern)
    # continue host-driven from the device state: still plain greedy
    r = g.mtp_step(nx)
    assert r == plain[1 + len(toks): 1 + len(toks) + len(r)]


def test_device_driver_natural_drafts_equal_plain(setup, mode):
    """No forced drafts (random weights: drafts are nearly always rejected); eager and graph agree."""
    d, prompt, pattern, plain, forces = setup
    outs = []
    for use_graph in (False, True):
        g = engine(d, mode)
        x = g.mtp_prefill(prompt)
        g.mtp_device_begin(x, 64)
        g.mtp_device_steps(6, use_graph=use_graph)
        toks, nx = g.mtp_device_end(64)
        outs.append(toks)
        g.close()
    assert outs[0] == outs[1]
    assert outs[0] == plain[1:1 + len(outs[0])]


def test_rewind_and_step_plain_match_oracle(setup):
    """Host-driven rewind (mtp.rs:596-608) and step_plain (504-515) against the oracle's driver,
    tokens and h_nextn bit for bit."""
    import oxe_amd as A
    d, prompt, pattern, plain, forces = setup
    g = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    o = O.Engine(d, seed=SEED, n_ctx=N_CTX)
    od = O.Driver(o)
    x = g.mtp_prefill(prompt)
    assert od.prefill(prompt) == x
    k = 0                                   # x == plain[k]: the greedy sequence is followed throughout
    for acc in (1, 1, 0, 1):
        f = plain[k + 1] if acc else (plain[k + 1] + 7) % d.n_vocab
        rg, ro = g.mtp_step(x, f), od.step(x, f)
        assert rg == ro == plain[k + 1: k + 2 + acc]
        if acc:
            g.mtp_rewind(1)                 # keep x only: the next token is plain[k + 1] again
            assert od.rewind(1) == 0
        x, k = plain[k + 1], k + 1
        xg, xo = g.mtp_step_plain(x), od.step_plain(x)
        assert xg == xo == plain[k + 1]
        x, k = xg, k + 1
        assert np.array_equal(g.hidden(0).view(np.uint32), o.hidden(0).view(np.uint32))
    g.close()
    o.close()
