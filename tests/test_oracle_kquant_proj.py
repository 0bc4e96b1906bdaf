"""The oracle's typed engine with K-quant mixer matrices, the types of the Ornith file (K-quant
attn_qkv / attn_gate / ssm_beta / ssm_alpha / ssm_out, attention q / k / v / output and token
embedding; tests/golden/gguf_header_ornith.json), against the independent float64 model (no GPU).

The K-quant row dots and row dequantisers are pinned in test_oracle_kquant.py and
test_oracle_dequant_kq.py. Here the composition is pinned: each K-quant projection part takes the
q8_K blocks of the normed layer input (crates/model/src/engine.rs:2270-2343 mv / mv_lanes; the
delta-net parts 2414-2444, the attention parts 2614-2703), the output projection the q8_K blocks of
the mixer's gated f32 outputs (mixer_out 2573-2609), and the token embedding is the dequantised
K-quant row (2251-2256), for the layer input and for the MTP entry. Planted mistakes (the min
term's sign in the embedding, K-quant rows on the un-normed input) fail the bar.
"""
import numpy as np
import pytest

import oracle as O
from f64_model import F64Model, Mistake
from test_oracle_f64 import TOL, eng_arrays, lanes_input, oracle_entry, oracle_mixer, oracle_moe, rel_err

SEED = 37
T = O.T
q3, q4, q5, q6, f32 = 11, 12, 13, 14, 0


def types_for():
    ty = {}
    for kind, t in (("DN_QKV", q4), ("DN_Z", q4), ("DN_BETA", q4), ("DN_ALPHA", q4), ("DN_OUT", q4)):
        ty[(0, T[kind])] = t                     # the Ornith delta-net layer
    for kind, t in (("DN_QKV", q5), ("DN_Z", q6), ("DN_BETA", f32), ("DN_ALPHA", f32), ("DN_OUT", q3)):
        ty[(1, T[kind])] = t                     # mixed K-quant types, F32 gates
    ty[(2, T["DN_OUT"])] = q6                    # Q8_0 projections, a K-quant output projection
    for kind, t in (("ATT_Q", q4), ("ATT_K", q5), ("ATT_V", q6), ("ATT_OUT", q4)):
        ty[(3, T[kind])] = t                     # the Ornith attention layer
    for layer in (0, 3):                         # Q3_K experts beside a Q6_K shared expert
        for kind, t in (("GATE_EXPS", q3), ("UP_EXPS", q3), ("DOWN_EXPS", q3), ("GATE_SHEXP", q6),
                        ("UP_SHEXP", q6), ("DOWN_SHEXP", q6)):
            ty[(layer, T[kind])] = t
    ty[(O.GLOBAL_LAYER, T["TOK_EMBD"])] = q4
    ty[(O.GLOBAL_LAYER, T["OUTPUT"])] = q6
    return ty


@pytest.fixture(scope="module")
def desc():
    return O.desc_small()


@pytest.fixture(scope="module")
def f64(desc):
    return F64Model(desc, SEED, types=types_for())


def engine(desc, n_ctx=256):
    return O.Engine(desc, seed=SEED, n_ctx=n_ctx, types=types_for())


def dn_case(desc, m, layer):
    e = engine(desc)
    conv, S, _, _ = eng_arrays(e, desc, e.n_ctx)
    rng = np.random.default_rng(11 + layer)
    conv[0, layer] = rng.standard_normal(conv[0, layer].shape).astype(np.float32)
    S[0, layer] = (0.1 * rng.standard_normal(S[0, layer].shape)).astype(np.float32)
    cv, st = conv[0, layer].astype(np.float64), S[0, layer].astype(np.float64)
    # an input of rms 5: its norm differs from it by that factor (planted un-normed mistake below)
    x = (5.0 * lanes_input(2, 9200 + layer)).astype(np.float32)
    got = oracle_mixer(e, layer, x, 0)
    want = np.array([m.dn_mixer(layer, x[ln].astype(np.float64), cv, st) for ln in range(2)])
    e.close()
    return got, want, x.astype(np.float64)


@pytest.mark.parametrize("layer", [0, 1, 2])
def test_delta_net_layer_with_kquant_projections(desc, f64, layer):
    got, want, x = dn_case(desc, f64, layer)
    for ln in range(2):
        assert rel_err(got[ln], want[ln]) < TOL, ln
        assert rel_err(got[ln] - x[ln], want[ln] - x[ln]) < TOL, ln   # the mixer's own output


def test_attention_layer_with_kquant_projections(desc, f64):
    pos0, l = 300, desc.full_attention_interval - 1
    e = engine(desc, 512)
    _, _, K, VT = eng_arrays(e, desc, e.n_ctx)
    rng = np.random.default_rng(16)
    K[0, :, :pos0] = rng.standard_normal(K[0, :, :pos0].shape).astype(np.float16).view(np.uint16)
    VT[0, :, :pos0] = rng.standard_normal(VT[0, :, :pos0].shape).astype(np.float16).view(np.uint16)
    Kf = K[0].view(np.float16).astype(np.float64)
    Vf = VT[0].view(np.float16).astype(np.float64)
    x = lanes_input(2, 9210)
    got = oracle_mixer(e, l, x, pos0)
    want = np.array([f64.att_mixer(l, x[ln].astype(np.float64), pos0 + ln, Kf, Vf) for ln in range(2)])
    for ln in range(2):
        assert rel_err(got[ln], want[ln]) < TOL, ln
    # the new K rows and V^T columns come from the K-quant k / v rows
    assert rel_err(K[0, :, pos0:pos0 + 2].view(np.float16).astype(np.float64), Kf[:, pos0:pos0 + 2]) < TOL
    assert rel_err(VT[0, :, pos0:pos0 + 2].view(np.float16).astype(np.float64), Vf[:, pos0:pos0 + 2]) < TOL
    e.close()


def test_decode_steps_and_mtp_entry_with_kquant_embedding(desc, f64):
    """steps of the typed engine against the float64 composition layer by layer (each layer from the
    oracle's own input), the K-quant embedding as the first layer's input and in the MTP entry"""
    A, B = engine(desc), engine(desc)
    conv, S, K, VT = eng_arrays(B, desc, B.n_ctx)

    def layer(l, x, pos):
        xo = np.asarray(x, np.float32)[None, :]
        att = l == desc.n_layer or (l + 1) % desc.full_attention_interval == 0
        if att:
            ai = l // desc.full_attention_interval if l < desc.n_layer else K.shape[0] - 1
            want1 = f64.att_mixer(l, xo[0].astype(np.float64), pos, K[ai].view(np.float16).astype(np.float64),
                                  VT[ai].view(np.float16).astype(np.float64))
        else:
            ri = l - (l + 1) // desc.full_attention_interval
            want1 = f64.dn_mixer(l, xo[0].astype(np.float64), conv[0, ri].astype(np.float64),
                                 S[0, ri].astype(np.float64))
        x1 = oracle_mixer(B, l, xo, pos)
        assert rel_err(x1[0], want1) < TOL, (l, pos, "mixer")
        x2 = oracle_moe(B, l, x1)
        assert rel_err(x2[0], f64.moe(l, x1[0].astype(np.float64))) < TOL, (l, pos, "moe")
        return x2[0]

    for pos, t in enumerate((101, 2047, 3333)):
        A.step(t)
        # a K-quant row dequantises exactly in f32 (d * scale * code - dmin * min rounds once, and
        # the f64 value rounded to f32 is that value): the oracle's own input
        x = f64.embed(t).astype(np.float32)
        for l in range(desc.n_layer):
            x = layer(l, x, pos)
        hout, logits = f64.head(x.astype(np.float64), O.GLOBAL_LAYER, T["OUT_NORM"])
        assert rel_err(A.hidden(0), hout) < TOL, pos
        assert rel_err(A.logits(0), logits) < TOL, pos
    h = A.hidden(0)
    assert rel_err(oracle_entry(B, 77, h)[0], f64.entry(77, h.astype(np.float64))) < TOL
    A.close()
    B.close()


def test_planted_mistakes_fail_the_bar(desc):
    # the embedding's min term with the wrong sign
    bad = F64Model(desc, SEED, Mistake(Mistake.KQ_MIN_SIGN), types=types_for())
    good = F64Model(desc, SEED, types=types_for())
    e = engine(desc)
    h = np.asarray(O.synth_normal(SEED, 9220, 2048), np.float32)
    got = oracle_entry(e, 77, h)[0]
    assert rel_err(got, good.entry(77, h.astype(np.float64))) < TOL
    assert rel_err(got, bad.entry(77, h.astype(np.float64))) > 20 * TOL
    e.close()
    # K-quant projection rows on the un-normed input
    got, want, x = dn_case(desc, F64Model(desc, SEED, Mistake(Mistake.KQ_RAW_X), types=types_for()), 0)
    assert max(rel_err(got[ln] - x[ln], want[ln] - x[ln]) for ln in range(2)) > 20 * TOL
