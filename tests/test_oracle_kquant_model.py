"""The oracle's typed engine (K-quant experts, shared expert and LM head; F32 ssm_beta / ssm_alpha) against
the independent float64 model (no GPU).

The K-quant row dots themselves are pinned in test_oracle_kquant.py (exact rational dots from an
independent block decoder). Here the composition is pinned: which vector is quantised to q8_K for
which matrix, that F32 rows take the normed f32 vector itself, and where each typed matrix sits in
the MoE, the delta-net projections and the LM head (crates/model/src/engine.rs:2270-2343 mv /
mv_lanes; 2432-2444 beta / alpha rows; 3437-3625 MoE; 3630-3715 head). The float64 model decodes
K-quant blocks with its own vectorised decoder (f64_model.kq_values), itself checked here against
the scalar block decoder of tests/kquant_blocks.py. Planted mistakes (the min term's sign, F32 rows
on the un-normed input) fail the bar.
"""
import numpy as np
import pytest

import kquant_blocks as KB
import oracle as O
from f64_model import F64Model, Mistake, kq_values
from test_oracle_f64 import TOL, eng_arrays, lanes_input, oracle_mixer, oracle_moe, rel_err

SEED = 31
T = O.T


def types_for(desc):
    ty = {}
    for kind, t in (("GATE_EXPS", 12), ("UP_EXPS", 12), ("DOWN_EXPS", 13), ("GATE_SHEXP", 14), ("UP_SHEXP", 14),
                    ("DOWN_SHEXP", 14)):
        ty[(1, T[kind])] = t
    for kind, t in (("GATE_EXPS", 11), ("UP_EXPS", 13), ("DOWN_EXPS", 14), ("GATE_SHEXP", 12), ("UP_SHEXP", 12),
                    ("DOWN_SHEXP", 11)):
        ty[(2, T[kind])] = t
    ty[(0, T["DN_BETA"])] = 0
    ty[(0, T["DN_ALPHA"])] = 0
    ty[(O.GLOBAL_LAYER, T["OUTPUT"])] = 14
    return ty


@pytest.fixture(scope="module")
def desc():
    return O.desc_small()


@pytest.fixture(scope="module")
def f64(desc):
    return F64Model(desc, SEED, types=types_for(desc))


@pytest.mark.parametrize("ty", [3, 4, 5, 6])
def test_vectorised_decoder_matches_the_block_decoder(ty):
    raw = KB.random_blocks(ty, 3, 512, seed=40 + ty)
    got = kq_values(ty, raw)
    bb = KB.BYTES[ty]
    for r in range(3):
        for b in range(2):
            d, dmin, q, sc, m = KB.decode_block(ty, raw[r, b * bb:(b + 1) * bb])
            want = d * sc * q - dmin * m
            assert np.array_equal(got[r, 256 * b:256 * (b + 1)], want), (ty, r, b)


def moe_case(desc, f64, layer, mistakes=None):
    e = O.Engine(desc, seed=SEED, n_ctx=256, types=types_for(desc))
    x1 = lanes_input(2, 9100 + layer)
    got = oracle_moe(e, layer, x1)
    m = f64 if mistakes is None else F64Model(desc, SEED, mistakes, types=types_for(desc))
    want = []
    for ln in range(2):
        x2, rt = m.moe(layer, x1[ln].astype(np.float64), want_route=True)
        assert rt["margin"] > 1e-3
        want.append(x2)
    e.close()
    return got, np.array(want)


@pytest.mark.parametrize("layer", [1, 2])
def test_typed_moe_layer(desc, f64, layer):
    got, want = moe_case(desc, f64, layer)
    for ln in range(2):
        assert rel_err(got[ln], want[ln]) < TOL, ln


def dn_case(desc, f64, mistakes=None):
    e = O.Engine(desc, seed=SEED, n_ctx=256, types=types_for(desc))
    conv, S, _, _ = eng_arrays(e, desc, e.n_ctx)
    rng = np.random.default_rng(7)
    conv[0, 0] = rng.standard_normal(conv[0, 0].shape).astype(np.float32)
    S[0, 0] = (0.1 * rng.standard_normal(S[0, 0].shape)).astype(np.float32)
    cv, st = conv[0, 0].astype(np.float64), S[0, 0].astype(np.float64)
    # an input of rms 5: its norm differs from it by that factor (planted F32-row mistake below)
    x = (5.0 * lanes_input(2, 9110)).astype(np.float32)
    got = oracle_mixer(e, 0, x, 0)
    m = f64 if mistakes is None else F64Model(desc, SEED, mistakes, types=types_for(desc))
    want = np.array([m.dn_mixer(0, x[ln].astype(np.float64), cv, st) for ln in range(2)])
    e.close()
    return got, want, x.astype(np.float64)


def test_delta_net_layer_with_f32_beta_alpha(desc, f64):
    got, want, x = dn_case(desc, f64)
    for ln in range(2):
        assert rel_err(got[ln], want[ln]) < TOL, ln
        assert rel_err(got[ln] - x[ln], want[ln] - x[ln]) < TOL, ln   # the mixer's own output


def test_q6k_lm_head(desc, f64):
    """a step of the typed engine: its logits against the float64 head (Q6_K output matrix) on the
    oracle's own final hidden state, taken layer by layer from a second typed engine"""
    A = O.Engine(desc, seed=SEED, n_ctx=256, types=types_for(desc))
    B = O.Engine(desc, seed=SEED, n_ctx=256, types=types_for(desc))
    tok = 1234
    A.step(tok)
    x = f64.embed(tok).astype(np.float32)[None, :]
    for l in range(desc.n_layer):
        x = oracle_moe(B, l, oracle_mixer(B, l, x, 0))
    hout, logits = f64.head(x[0].astype(np.float64), O.GLOBAL_LAYER, T["OUT_NORM"])
    assert rel_err(A.hidden(0), hout) < TOL
    assert rel_err(A.logits(0), logits) < TOL
    A.close()
    B.close()


def test_planted_mistakes_fail_the_bar(desc, f64):
    got, want = moe_case(desc, f64, 1, Mistake(Mistake.KQ_MIN_SIGN))
    assert max(rel_err(got[ln], want[ln]) for ln in range(2)) > 20 * TOL
    # the gates move the mixer's output, not the residual it is added to: compared without it
    got, want, x = dn_case(desc, f64, Mistake(Mistake.BA_RAW_X))
    assert max(rel_err(got[ln] - x[ln], want[ln] - x[ln]) for ln in range(2)) > 20 * TOL
