"""K-quant mixer matrices and a K-quant token embedding inside the engine's runs, the types of the
reference's Ornith file (tests/golden/gguf_header_ornith.json): K-quant attn_qkv / attn_gate /
ssm_beta / ssm_alpha / ssm_out, attention q / k / v / output, token embedding, Q3_K experts beside
a Q6_K shared expert, a Q6_K LM head (the reference's mv / mv_lanes over every qtype,
crates/model/src/engine.rs:2270-2343; the token embedding 2251-2256).

A synthetic model with those types is written as a GGUF file (tests/gguf_writer.py, the oracle's
synthetic K-quant blocks); the engine created from the file must decode bit for bit like the
oracle's typed engine on the same weights (itself pinned against the float64 model in
test_oracle_kquant_proj.py): prefill, logits, hidden states, two-lane verify runs, host-driven MTP
steps with accepted and rejected drafts (the MTP entry over the K-quant embedding, the MTP layer's
K-quant projections in draft and seeding runs), and device-driven steps."""
import os

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

pytestmark = pytest.mark.gpu

SEED = 23
T = O.T
q3, q4, q5, q6, f32 = 11, 12, 13, 14, 0


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def model_types(d):
    assert d.n_layer == 4 and d.full_attention_interval == 4
    ty = {}
    for kind, t in (("DN_QKV", q4), ("DN_Z", q4), ("DN_BETA", q4), ("DN_ALPHA", q4), ("DN_OUT", q4)):
        ty[(0, T[kind])] = t                     # the Ornith delta-net layer
    for kind, t in (("DN_QKV", q5), ("DN_Z", q6), ("DN_BETA", f32), ("DN_ALPHA", f32), ("DN_OUT", q3)):
        ty[(1, T[kind])] = t                     # mixed K-quant types beside F32 gates
    ty[(2, T["DN_OUT"])] = q6                    # Q8_0 projections, a K-quant output projection
    for layer, (q, k, v, o) in ((3, (q4, q5, q6, q4)), (4, (q4, q4, q4, q5))):
        for kind, t in (("ATT_Q", q), ("ATT_K", k), ("ATT_V", v), ("ATT_OUT", o)):
            ty[(layer, T[kind])] = t             # the Ornith attention layer; the MTP layer
    for layer in (0, 3):                         # Q3_K experts beside a Q6_K shared expert
        for kind, t in (("GATE_EXPS", q3), ("UP_EXPS", q3), ("DOWN_EXPS", q3), ("GATE_SHEXP", q6),
                        ("UP_SHEXP", q6), ("DOWN_SHEXP", q6)):
            ty[(layer, T[kind])] = t
    ty[(O.GLOBAL_LAYER, T["TOK_EMBD"])] = q4
    ty[(O.GLOBAL_LAYER, T["OUTPUT"])] = q6
    return ty


def scratch_dir():
    return "/dev/shm" if os.path.isdir("/dev/shm") and os.access("/dev/shm", os.W_OK) else "/tmp"


@pytest.fixture(scope="module")
def typed_file():
    d = O.desc_small()
    ty = model_types(d)
    path = os.path.join(scratch_dir(), f"oxe_test_kqp_{os.getpid()}.gguf")
    print("writing the Ornith-typed model as GGUF", flush=True)
    W.write_synth_model(path, O, d, SEED, ty)
    yield d, ty, path
    if os.path.exists(path):
        os.remove(path)


def test_kquant_projections_prefill_and_verify_match_oracle(typed_file):
    import oxe_amd as A
    d, ty, path = typed_file
    g = A.Engine.from_gguf(path, n_ctx=512)
    assert not g.fused
    ref = O.Engine(d, seed=SEED, n_ctx=512, types=ty)
    toks = [int(v) % d.n_vocab for v in O.bench_prompt(9)]
    print("prefill 9 tokens (two positions per run)", flush=True)
    nx, h = g.prefill(toks, hidden=True)
    want = [ref.step(t) for t in toks]
    assert nx == want[-1]
    assert np.array_equal(bits(g.logits(0)), bits(ref.logits(0)))
    assert np.array_equal(bits(h[-1]), bits(ref.hidden(0)))
    print("two-lane verify", flush=True)
    out = g.verify([nx, 17])
    assert list(out) == list(ref.verify([nx, 17]))
    for lane in (0, 1):
        assert np.array_equal(bits(g.logits(lane)), bits(ref.logits(lane))), lane
        assert np.array_equal(bits(g.hidden(lane)), bits(ref.hidden(lane))), lane
    g.close()


def test_kquant_projections_mtp_steps_match_oracle_driver(typed_file):
    import oxe_amd as A
    d, ty, path = typed_file
    g = A.Engine.from_gguf(path, n_ctx=512)
    ref = O.Engine(d, seed=SEED, n_ctx=512, types=ty)
    drv = O.Driver(ref)
    toks = [int(v) % d.n_vocab for v in O.bench_prompt(12)]
    print("MTP prefill", flush=True)
    x = g.mtp_prefill_batched(toks)
    assert x == drv.prefill(toks)
    for i in range(6):
        print(f"host step {i}", flush=True)
        if i % 3 == 2:
            want = drv.step(x, force=[(x * 7 + i) % d.n_vocab])
            got = g.mtp_step_force(x, [(x * 7 + i) % d.n_vocab])
        else:
            want, got = drv.step(x), g.mtp_step(x)
        assert got == want, i
        x = want[-1]
    assert np.array_equal(bits(g.hidden(0)), bits(ref.hidden(0)))
    print("device-driven steps", flush=True)
    n = 6
    g.mtp_device_begin(x, 2 * n + 4)
    g.mtp_device_steps(n, use_graph=True)
    gen, nxt = g.mtp_device_end(2 * n + 4)
    want = []
    for _ in range(n):
        o = drv.step(x)
        want += o
        x = o[-1]
    assert [int(t) for t in gen] == want
    assert nxt == x
    g.close()


def test_typed_engine_synthesised_on_device_matches_oracle():
    """the same types without a file: oxe_engine_create_typed + the device's synthetic weights (the
    oracle's K-quant blocks and F32 values generated on the device) decode like the typed oracle"""
    import oxe_amd as A
    d = O.desc_small()
    ty = model_types(d)
    g = A.Engine(d, seed=SEED, n_ctx=512, types=ty)
    assert not g.fused
    ref = O.Engine(d, seed=SEED, n_ctx=512, types=ty)
    toks = [int(v) % d.n_vocab for v in O.bench_prompt(5)]
    print("prefill 5 tokens", flush=True)
    nx = g.prefill(toks)
    assert nx == [ref.step(t) for t in toks][-1]
    assert np.array_equal(bits(g.logits(0)), bits(ref.logits(0)))
    assert np.array_equal(bits(g.hidden(0)), bits(ref.hidden(0)))
    out = g.verify([nx, 17])
    assert list(out) == list(ref.verify([nx, 17]))
    for lane in (0, 1):
        assert np.array_equal(bits(g.logits(lane)), bits(ref.logits(lane))), lane
    g.close()
