"""K-quant and F32 matrices inside the engine's runs (the reference's mv / mv_lanes over every qtype,
crates/model/src/engine.rs:2270-2343), the types a Qwen3.6 GGUF file holds: K-quant experts (gate /
up Q4_K, down Q5_K or Q6_K), F32 ssm_beta / ssm_alpha, a Q6_K LM head, and the Ornith file's
K-quant shared experts and Q3_K experts.

A synthetic model with those types is written as a GGUF file (tests/gguf_writer.py, the oracle's
synthetic K-quant blocks); the engine created from the file must decode bit for bit like the
oracle's typed engine on the same weights: prefill, logits, hidden states, host-driven MTP steps
with accepted and rejected drafts, and device-driven steps. Such an engine runs per phase (the
fused run kernel reads Q8_0 matrices only) and prefills two positions per run."""
import os

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

pytestmark = pytest.mark.gpu

SEED = 11
T = O.T


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def model_types(d):
    """per-layer types covering every unit kind of the K-quant MoE and head paths"""
    ty = {}
    q4, q5, q6, q3, f32 = 12, 13, 14, 11, 0

    def moe(layer, gate, up, down, sh_gate, sh_up, sh_down):
        for kind, t in ((T["GATE_EXPS"], gate), (T["UP_EXPS"], up), (T["DOWN_EXPS"], down), (T["GATE_SHEXP"], sh_gate),
                        (T["UP_SHEXP"], sh_up), (T["DOWN_SHEXP"], sh_down)):
            if t != 8:
                ty[(layer, kind)] = t
    assert d.n_layer == 4 and d.full_attention_interval == 4
    moe(0, q4, q4, q5, 8, 8, 8)          # Qwen3.6: K-quant experts, Q8_0 shared expert
    moe(1, q3, q3, q6, q6, q6, q6)       # Ornith: Q3_K experts, Q6_K shared expert
    moe(2, q4, q5, q3, 8, 8, q6)         # mixed gate / up types; K-quant down beside a K-quant shared down
    moe(3, 8, 8, 8, q4, q4, 8)           # Q8_0 experts beside a K-quant shared gate / up
    moe(4, q4, q4, q6, 8, 8, 8)          # the MTP block
    for layer in (0, 1):                 # F32 ssm_beta / ssm_alpha (layer 2 keeps Q8_0)
        ty[(layer, T["DN_BETA"])] = f32
        ty[(layer, T["DN_ALPHA"])] = f32
    ty[(O.GLOBAL_LAYER, T["OUTPUT"])] = q6
    return ty


def scratch_dir():
    return "/dev/shm" if os.path.isdir("/dev/shm") and os.access("/dev/shm", os.W_OK) else "/tmp"


@pytest.fixture(scope="module")
def typed_file():
    d = O.desc_small()
    ty = model_types(d)
    path = os.path.join(scratch_dir(), f"oxe_test_kq_{os.getpid()}.gguf")
    print("writing the K-quant model as GGUF", flush=True)
    W.write_synth_model(path, O, d, SEED, ty)
    yield d, ty, path
    if os.path.exists(path):
        os.remove(path)


def test_typed_engine_runs_per_phase_and_prefill_matches_oracle(typed_file):
    import oxe_amd as A
    d, ty, path = typed_file
    g = A.Engine.from_gguf(path, n_ctx=512)
    assert not g.fused
    with pytest.raises(Exception):
        g.set_fused(True)   # the fused run kernel reads Q8_0 matrices only
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
    wv = ref.verify([nx, 17])
    assert list(out) == list(wv)
    for lane in (0, 1):
        assert np.array_equal(bits(g.logits(lane)), bits(ref.logits(lane))), lane
        assert np.array_equal(bits(g.hidden(lane)), bits(ref.hidden(lane))), lane
    g.close()


def test_typed_engine_mtp_steps_match_oracle_driver(typed_file):
    import oxe_amd as A
    d, ty, path = typed_file
    g = A.Engine.from_gguf(path, n_ctx=512)
    ref = O.Engine(d, seed=SEED, n_ctx=512, types=ty)
    drv = O.Driver(ref)
    toks = [int(v) % d.n_vocab for v in O.bench_prompt(12)]
    print("MTP prefill", flush=True)
    x = g.mtp_prefill_batched(toks)
    assert x == drv.prefill(toks)
    # host-driven steps: the drafts as drafted, then forced accepts and rejects
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
    # device-driven steps (per-phase runs, captured in a graph)
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


def test_typed_engine_restricted_draft_head_matches_oracle(typed_file):
    """the restricted draft head over a Q6_K LM head (rows gathered from the file's blocks)"""
    import oxe_amd as A
    d, ty, path = typed_file
    g = A.Engine.from_gguf(path, n_ctx=512)
    ref = O.Engine(d, seed=SEED, n_ctx=512, types=ty)
    vocab = [i for i in range(d.n_vocab) if i % 5 == 1]
    assert g.mtp_set_draft_vocab(vocab) == (len(vocab) + 15) // 16 * 16
    ref.set_draft_vocab(vocab)
    for t in (3, 17, 42):
        assert g.step(t) == ref.step(t)
    h = np.asarray(ref.hidden(0), np.float32).copy()
    for i, tok in enumerate((77, 1234, 9)):
        got = g.mtp_run([tok], 3 + i, h[None, :])
        want = ref.mtp_run([tok], 3 + i, h[None, :])
        assert got == want and got % 5 == 1, i
        h = np.asarray(ref.hidden(0), np.float32).copy()
    g.close()
