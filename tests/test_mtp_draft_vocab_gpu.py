"""Restricted-vocabulary draft head on the GPU (MtpWeights::set_draft_vocab, crates/model/src/mtp.rs:
166-197; the reference's mini_mtp_restricted_draft_head, crates/model/src/tests.rs:1116-1177), in both
run modes, against the oracle's restricted head.

The draft runs' LM head becomes the output matrix's rows of the vocabulary (gathered on the device),
its argmax mapped back to token ids; verify runs keep the whole head. Checked: each draft of a direct
MTP run equals the oracle's restricted draft (and is in the vocabulary); a vocabulary of every id
drafts what the whole head drafts; host- and device-driven MTP steps emit the oracle driver's ids with
its drafted / accepted counts; restoring the whole head drafts as before."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

SEED = 13


def small_vocab(d):
    v = [i for i in range(d.n_vocab) if i % 3 == 0][::-1]
    return v + [v[0], d.n_vocab + 5]


def drafts(eng, toks, start):
    """three direct MTP draft runs after plain steps over `toks` (positions start..)"""
    for t in toks:
        eng.step(t)
    h = np.asarray(eng.hidden(0), np.float32).copy()
    out = []
    for i, tok in enumerate([77, 1234, 9]):
        out.append(int(eng.mtp_run([tok], start + i, h[None, :])))
        h = np.asarray(eng.hidden(0), np.float32).copy()
    return out


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "per_phase"])
def test_direct_drafts_match_oracle(fused):
    import oxe_amd as A
    d = O.desc_small()
    toks = [3, 17, 42]
    results = {}
    for name, vocab in (("whole", None), ("all", list(range(d.n_vocab))), ("small", small_vocab(d))):
        g = A.Engine(d, seed=SEED, n_ctx=512)
        g.set_fused(fused)
        ref = O.Engine(d, seed=SEED, n_ctx=512)
        if vocab is not None:
            rows = g.mtp_set_draft_vocab(vocab)
            n = ref.set_draft_vocab(vocab)
            assert rows == (n + 15) // 16 * 16
        print(f"draft head {name}", flush=True)
        got, want = drafts(g, toks, len(toks)), drafts(ref, toks, len(toks))
        assert got == want, name
        results[name] = got
        g.close()
        ref.close()
    assert results["all"] == results["whole"]
    assert all(t % 3 == 0 for t in results["small"])


@pytest.mark.parametrize("fused", [True, False], ids=["fused", "per_phase"])
def test_mtp_steps_with_small_vocabulary_match_oracle_driver(fused):
    import oxe_amd as A
    d = O.desc_small()
    g = A.Engine(d, seed=SEED, n_ctx=512)
    g.set_fused(fused)
    ref = O.Engine(d, seed=SEED, n_ctx=512)
    g.mtp_set_draft_vocab(small_vocab(d))
    ref.set_draft_vocab(small_vocab(d))
    drv = O.Driver(ref)
    prompt = [int(v) % d.n_vocab for v in O.bench_prompt(20)]
    x = g.mtp_prefill_batched(prompt)
    assert x == drv.prefill(prompt)
    for i in range(6):
        want = drv.step(x)
        assert g.mtp_step(x) == want, i
        x = want[-1]
    n = 8
    g.mtp_device_begin(x, 2 * n + 4)
    g.mtp_device_steps(n, use_graph=True)
    gen, nxt = g.mtp_device_end(2 * n + 4)
    want = []
    for _ in range(n):
        o = drv.step(x)
        want += o
        x = o[-1]
    assert [int(t) for t in gen] == want and nxt == x
    st = drv.stats()
    gs = g.mtp_stats()
    assert (gs["steps"], gs["accepted"], gs["drafted"]) == (st["steps"], st["accepted"], st["drafted"])
    # the whole head again: drafts as before the restriction
    assert g.mtp_set_draft_vocab([]) == 0
    g.close()
    ref.close()
