"""The oracle's plan mode: the reference's static per-phase plan (crates/model/src/plan.rs:171-249)
run on a pinned team with one barrier per phase (crates/sched/src/lib.rs:43-84; engine.rs:2137-2190).
Every row, head, routing unit and logit is computed by one thread with the arithmetic of the
default path, so a plan run must give the same bits whatever the team size (the reference's own
thread-count-invariance property, crates/model/src/tests.rs:288). The CPU baseline of bench.py times
this mode."""
import functools

import numpy as np
import pytest

import oracle as O


@functools.lru_cache(maxsize=None)
def _run(team, depth=1, lanes=2, n_steps=4, force=None):
    d = O.desc_small()
    e = O.Engine(d, seed=5, n_ctx=512, lanes=lanes)
    if team:
        assert e.set_plan(team) >= 1
    dr = O.Driver(e, depth)
    x = dr.prefill(O.bench_prompt(12) % d.n_vocab)
    ids = [x]
    for i in range(n_steps):
        out = dr.step(ids[-1], force=force) if force is not None else dr.step(ids[-1])
        ids.extend(out)
    st = dict(ids=ids, hidden=e.hidden(0), logits=e.logits(0), pos=e.pos, stats=dr.stats(),
              barriers=e.plan_barriers())
    L = O.lib()
    n_att = d.n_layer // d.full_attention_interval + 1
    kc = np.ctypeslib.as_array(L.oxo_kcache(e.h), (n_att * d.n_head_kv * e.n_ctx * d.head_dim,)).copy()
    vc = np.ctypeslib.as_array(L.oxo_vcache(e.h), (n_att * d.n_head_kv * d.head_dim * e.n_ctx,)).copy()
    n_rec = d.n_layer - (n_att - 1)
    ssm = np.ctypeslib.as_array(L.oxo_ssm_state(e.h), (lanes * n_rec * 32 * 128 * 128,)).copy()
    st.update(kc=kc, vc=vc, ssm=ssm)
    e.set_plan(0)
    e.close()
    return st


@pytest.mark.parametrize("team", [1, 5])
def test_plan_equals_default_path(team):
    ref = _run(0)
    got = _run(team)
    assert got["ids"] == ref["ids"]
    assert got["pos"] == ref["pos"]
    assert got["stats"] == ref["stats"]
    for k in ("hidden", "logits"):
        assert np.array_equal(got[k].view(np.uint32), ref[k].view(np.uint32)), k
    for k in ("kc", "vc"):
        assert np.array_equal(got[k], ref[k]), k
    assert np.array_equal(got["ssm"].view(np.uint32), ref["ssm"].view(np.uint32))
    assert ref["barriers"] == -1 and got["barriers"] > 0


def test_plan_depth2_three_lane_verify():
    """MTP depth 2: three-lane verify runs, where the routing units are the union of the lanes'
    experts split evenly over the team"""
    ref = _run(0, depth=2, lanes=3, n_steps=3)
    got = _run(5, depth=2, lanes=3, n_steps=3)
    assert got["ids"] == ref["ids"]
    assert np.array_equal(got["logits"].view(np.uint32), ref["logits"].view(np.uint32))
    assert np.array_equal(got["ssm"].view(np.uint32), ref["ssm"].view(np.uint32))


def test_plan_barriers_per_verify():
    """one barrier per phase: 5 per delta-net layer (RecMix, RecOut, MoeRouter, MoeGateUp, MoeDown),
    7 per attention layer (AttnQkv, the K-row writes, AttnCore, AttnOut and the three MoE phases),
    plus the join after the head"""
    d = O.desc_small()
    e = O.Engine(d, seed=5, n_ctx=256)
    assert e.set_plan(2) == 2
    b0 = e.plan_barriers()
    e.verify([7, 8])
    n_att = d.n_layer // d.full_attention_interval
    n_rec = d.n_layer - n_att
    assert e.plan_barriers() - b0 == 5 * n_rec + 7 * n_att + 1
    e.set_plan(0)
    e.close()
