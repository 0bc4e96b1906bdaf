"""The oracle's restricted-vocabulary draft head (MtpWeights::set_draft_vocab, crates/model/src/mtp.rs:
166-197; the reference's test mini_mtp_restricted_draft_head, crates/model/src/tests.rs:1116-1177),
no GPU.

(a) A draft vocabulary of every id drafts exactly what the whole head drafts: same outputs, same
drafted / accepted counts. (b) A small vocabulary (every 3rd id, given unsorted with a duplicate and
an id past the vocabulary) changes only the drafts: the output stays the plain greedy sequence, every
draft is in the vocabulary, and each draft is the first maximum of the draft run's own logits over
the vocabulary's ids (numpy, from the logits the oracle keeps). (c) The plan mode drafts the same.
"""
import numpy as np
import pytest

import oracle as O

SEED = 41


@pytest.fixture(scope="module")
def desc():
    return O.desc_small()


def greedy(desc, prompt, n):
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    x = 0
    for t in prompt:
        x = e.step(t)
    out = [x]
    while len(out) < n:
        x = e.step(x)
        out.append(x)
    e.close()
    return out


def run(desc, prompt, n, vocab=None, plan=0):
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    if vocab is not None:
        e.set_draft_vocab(vocab)
    if plan:
        assert e.set_plan(plan) == plan
    d = O.Driver(e)
    x = d.prefill(prompt)
    ids = [x]
    while len(ids) < n:
        out = d.step(x)
        ids += out
        x = out[-1]
    st = d.stats()
    e.close()
    return ids[:n], st


def test_every_id_drafts_like_the_whole_head(desc):
    prompt = [3, 17, 42, 5, 9, 33, 1]
    want = greedy(desc, prompt, 12)
    ids_full, st_full = run(desc, prompt, 12)
    ids_all, st_all = run(desc, prompt, 12, vocab=list(range(desc.n_vocab)))
    assert ids_full == want and ids_all == want
    assert (st_all["drafted"], st_all["accepted"]) == (st_full["drafted"], st_full["accepted"])


def small_vocab(desc):
    v = [i for i in range(desc.n_vocab) if i % 3 == 0][::-1]
    return v + [v[0], desc.n_vocab + 5]


def test_small_vocabulary_changes_only_the_drafts(desc):
    prompt = [3, 17, 42, 5, 9, 33, 1]
    want = greedy(desc, prompt, 12)
    ids, _ = run(desc, prompt, 12, vocab=small_vocab(desc))
    assert ids == want


def test_drafts_are_the_first_maximum_over_the_vocabulary(desc):
    vocab = small_vocab(desc)
    keep = np.array(sorted({i for i in vocab if i < desc.n_vocab}), np.int64)
    e = O.Engine(desc, seed=SEED, n_ctx=256)
    assert e.set_draft_vocab(vocab) == len(keep)
    for t in [3, 17, 42]:
        e.step(t)
    h = e.hidden(0).copy()
    whole = []
    for pos, tok in enumerate([77, 1234, 9]):
        d = e.mtp_run([tok], 3 + pos, h[None, :])
        lg = e.logits(0).astype(np.float64)
        assert d % 3 == 0 and d < desc.n_vocab
        assert d == int(keep[np.argmax(lg[keep])])          # argmax: the first maximum
        whole.append(int(np.argmax(lg)))
        h = e.hidden(0).copy()
    assert any(w % 3 != 0 for w in whole)                   # the whole head would have drafted otherwise
    with pytest.raises(ValueError):
        e.set_draft_vocab([desc.n_vocab + 1])
    assert e.set_draft_vocab([]) == 0                        # the whole head again
    e.close()


def test_plan_mode_drafts_the_same(desc):
    prompt = [3, 17, 42, 5, 9, 33, 1]
    a = run(desc, prompt, 10, vocab=small_vocab(desc))
    b = run(desc, prompt, 10, vocab=small_vocab(desc), plan=3)
    assert a == b
