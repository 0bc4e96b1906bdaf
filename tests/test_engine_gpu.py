"""Engine parity on the GPU: the MI355X engine (C ABI) against the CPU oracle engine on the same
synthetic model, same tokens. Bar: bit-exact logits, hidden states, argmaxes and KV cache rows
(the reference's verify-lane batch invariance makes its own noise zero on an all-Q8_0 model)."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

N_CTX = 512


@pytest.fixture(scope="module", params=["fused", "per_phase"])
def small(request):
    """Both run modes: one persistent fused launch per run, and one launch per phase."""
    import oxe_amd as A
    d = O.desc_small()
    g = A.Engine(d, seed=3, n_ctx=N_CTX)
    if request.param == "per_phase":
        g.set_fused(False)
    elif not g.fused:
        pytest.skip("the fused run kernel needs a 256-CU device")
    return d, g, O.Engine(d, seed=3, n_ctx=N_CTX)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def test_verify_two_lanes_bitexact(small):
    d, g, o = small
    toks = [1234, 77]
    ag = g.verify(toks)
    ao = o.verify(toks)
    for ln in range(2):
        lg, lo = g.logits(ln), o.logits(ln)
        hg, ho = g.hidden(ln), o.hidden(ln)
        assert np.array_equal(bits(hg), bits(ho)), f"hidden lane {ln}: max diff {np.abs(hg - ho).max()}"
        assert np.array_equal(bits(lg), bits(lo)), f"logits lane {ln}: max diff {np.abs(lg - lo).max()}"
    assert list(ag) == list(ao)
    g.commit(2)
    o.commit(2)


def test_steps_and_rollback_bitexact(small):
    d, g, o = small
    # a rejected second lane, then more single steps
    for toks, m in [([5, 4000], 1), ([17], 1), ([300, 301], 2), ([9, 10], 1)]:
        ag, ao = g.verify(toks), o.verify(toks)
        assert list(ag) == list(ao)
        for ln in range(len(toks)):
            assert np.array_equal(bits(g.logits(ln)), bits(o.logits(ln))), (toks, ln)
        g.commit(m)
        o.commit(m)
        assert g.pos == o.pos


def test_mtp_run_and_seed_bitexact(small):
    d, g, o = small
    p = g.pos
    h = o.hidden(0)
    dg = g.mtp_run([42], p, h[None, :])
    do = o.mtp_run([42], p, h[None, :])
    assert dg == do
    assert np.array_equal(bits(g.hidden(0)), bits(o.hidden(0)))
    g.mtp_seed([43, 44], p + 1, np.stack([h, h * 0.5]))
    o.mtp_seed([43, 44], p + 1, np.stack([h, h * 0.5]))
    n_ctx = g.n_ctx
    # MTP layer K rows at p+1, p+2 (att index n_att-1 = 1 for the 4-layer model: 1 main + MTP)
    hd, nkv = 256, 2
    layer_bytes = nkv * n_ctx * hd * 2
    kg = g.state(0, layer_bytes, offset=layer_bytes, dtype=np.uint16).reshape(nkv, n_ctx, hd)
    ko = np.ctypeslib.as_array(O.lib().oxo_kcache(o.h), (2 * nkv * n_ctx * hd,)).reshape(2, nkv, n_ctx, hd)[1]
    assert np.array_equal(kg[:, : p + 3], ko[:, : p + 3])


def test_no_topk_ties(small):
    d, g, o = small
    assert g.counter(64) == 0


@pytest.mark.parametrize("mode", ["fused", "per_phase"])
def test_verify_sweep_bitexact(mode):
    """Many short verify runs (one and two lanes) from several prompt lengths, each committed: every
    lane's hidden row and logits bit-exact. Catches rare, value-dependent rounding differences (an
    f32 product folded into its f16 conversion changed about one run in ten here)."""
    import oxe_amd as A
    d = O.desc_small()
    for plen, nl in ((5, 2), (6, 1), (14, 2), (30, 2)):
        prompt = [int(v) % d.n_vocab for v in O.bench_prompt(plen + 8)]
        o = O.Engine(d, seed=0, n_ctx=256)
        g = A.Engine(d, seed=0, n_ctx=256)
        if mode == "per_phase":
            g.set_fused(False)
        elif not g.fused:
            pytest.skip("the fused run kernel needs a 256-CU device")
        for tk in prompt[:plen]:
            assert g.step(tk) == o.step(tk)
        for it in range(6):
            toks = [prompt[plen + it], (prompt[it] * 7 + 11) % d.n_vocab][:nl]
            assert list(g.verify(toks)) == list(o.verify(toks))
            for ln in range(nl):
                assert np.array_equal(bits(g.hidden(ln)), bits(o.hidden(ln))), (plen, it, ln, "hidden")
                assert np.array_equal(bits(g.logits(ln)), bits(o.logits(ln))), (plen, it, ln, "logits")
            g.commit(1)
            o.commit(1)
        g.close()
        o.close()


def test_lm_head_claimed_tail_bitexact():
    """The fused LM head with its tail claimed from a counter (a vocabulary of 40000 rows: 4 tiles of
    32 rows per workgroup, then 226 tiles in claimed pairs): every logit of both lanes and the
    argmaxes against the oracle, over several runs (the counter is re-armed by each launch's last
    workgroup)."""
    import oxe_amd as A
    d = O.desc_small(n_vocab=40000)
    g = A.Engine(d, seed=11, n_ctx=N_CTX)
    if not g.fused:
        pytest.skip("the fused run kernel needs a 256-CU device")
    o = O.Engine(d, seed=11, n_ctx=N_CTX)
    for toks in ([39999, 12], [5, 31000], [20000]):
        ag, ao = g.verify(toks), o.verify(toks)
        assert list(ag) == list(ao), toks
        for ln in range(len(toks)):
            assert np.array_equal(bits(g.logits(ln)), bits(o.logits(ln))), (toks, ln)
        g.commit(1)
        o.commit(1)
    g.close()
    o.close()


@pytest.mark.parametrize("which", ["created", "null"])
def test_engine_on_caller_stream(which):
    """oxe_engine_create_on: an engine whose launches and copies all go to the caller's stream (a
    torch stream, or the null stream) decodes bit for bit like one on its own stream: a batched
    prompt, verify runs and device-driven MTP steps (graph steps on the created stream, eager ones
    on the null stream, which cannot be captured)."""
    import oxe_amd as A
    import torch
    d = O.desc_small()
    ref = A.Engine(d, seed=5, n_ctx=N_CTX)
    st = torch.cuda.Stream() if which == "created" else None
    g = A.Engine(d, seed=5, n_ctx=N_CTX, stream=st.cuda_stream if st is not None else 0)
    assert (g.stream() or 0) == (st.cuda_stream if st is not None else 0)
    prompt = [int(v) % d.n_vocab for v in O.bench_prompt(20)]
    xr, xg = ref.mtp_prefill_batched(prompt), g.mtp_prefill_batched(prompt)
    assert xr == xg
    assert np.array_equal(bits(g.hidden(0)), bits(ref.hidden(0)))
    graph = which == "created"
    out = []
    for e, x in ((ref, xr), (g, xg)):
        e.mtp_device_begin(x, 64)
        e.mtp_device_steps(6, use_graph=graph)
        out.append(e.mtp_device_end(64))
    assert list(out[0][0]) == list(out[1][0]) and out[0][1] == out[1][1]
    for ln in range(2):
        assert np.array_equal(bits(g.logits(ln)), bits(ref.logits(ln))), ln
    g.close()
    ref.close()
