"""BASELINE config 4 shape (40 layers + MTP, vocab 151936, all Q8_0) end to end on the GPU against
the oracle: a short prompt and MTP-1 steps; bit-exact logits and identical greedy tokens."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu


def test_full_model_mtp_steps_bitexact():
    import oxe_amd as A
    d = O.desc_35b_a3b()
    prompt = O.bench_prompt(6)
    g = A.Engine(d, seed=0, n_ctx=256)
    o = O.Engine(d, seed=0, n_ctx=256)
    od = O.Driver(o)
    xg, xo = g.mtp_prefill(prompt), od.prefill(prompt)
    assert xg == xo
    assert np.array_equal(g.logits(1).view(np.uint32), o.logits(1).view(np.uint32))
    for _ in range(3):
        rg, ro = g.mtp_step(xg), od.step(xo)
        assert rg == ro
        xg, xo = rg[-1], ro[-1]
    for ln in range(2):
        lg, lo = g.logits(ln), o.logits(ln)
        assert np.array_equal(lg.view(np.uint32), lo.view(np.uint32)), f"lane {ln} max diff {np.abs(lg - lo).max()}"
    assert g.counter(64) == 0
