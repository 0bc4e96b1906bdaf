"""The server's engine on the GPU: the `Engine` trait (crates/server/src/engine.rs:28-190) as
OxeEngine implements it (crates/server/src/oxe_engine.rs:317-634), through the oxe_srv_* C ABI.

What the reference's server tests hold of it, restated for this engine (crates/server/src/
tests.rs and the trait's docs): greedy output is the same with and without speculation (MTP steps,
lookup drafts, rewinds), a restored snapshot or a loaded state continues bit for bit like the
uninterrupted run (its MTP draft state included), the prefix store's row segments plus a snapshot
file rebuild the sequence, and the trait's error cases give its messages. Plain greedy decoding on
this engine is checked against the oracle here and in the decode tests."""
import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

SEED = 5
N_CTX = 512


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def first_max(row):
    return int(np.argmax(row))   # numpy: the first index of the maximum, as sampling::argmax


@pytest.fixture(scope="module")
def d():
    return O.desc_small()


@pytest.fixture(scope="module")
def prompt(d):
    return [int(v) % d.n_vocab for v in O.bench_prompt(37)]


def server(d, mtp):
    import oxe_amd as A
    e = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    return A.ServerEngine(e, mtp=mtp)


@pytest.fixture(scope="module")
def plain(d, prompt):
    """greedy continuation of the prompt by the plain server engine (decode_argmax): x0, x1, ..."""
    s = server(d, False)
    x = first_max(s.prefill(prompt))
    out = [x]
    for _ in range(40):
        x = s.decode_argmax(x)
        out.append(x)
    return out


def test_plain_greedy_matches_oracle(d, plain):
    p = [int(v) % d.n_vocab for v in O.bench_prompt(37)]
    o = O.Engine(d, seed=SEED, n_ctx=N_CTX)
    x = None
    for t in p:
        x = o.step(t)
    ref = [x]
    for _ in range(6):
        x = o.step(x)
        ref.append(x)
    o.close()
    assert plain[:7] == ref


def test_prefill_logits_and_decode_argmax_plain_and_mtp(d, prompt, plain):
    import oxe_amd as A
    sp, sm = server(d, False), server(d, True)
    e = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    lp, lm = sp.prefill(prompt), sm.prefill(prompt)
    x = e.prefill(prompt)
    assert np.array_equal(bits(lp), bits(lm)) and np.array_equal(bits(lp), bits(e.logits(0)))
    assert first_max(lp) == x == plain[0]
    assert sp.n_past() == sm.n_past() == len(prompt)
    xp = xm = plain[0]
    for i in range(8):
        xp, xm = sp.decode_argmax(xp), sm.decode_argmax(xm)
        assert xp == xm == plain[i + 1]
    # decode = prefill of one token: the row of that token
    row = sp.decode(xp)
    assert first_max(row) == plain[9] and sp.n_past() == len(prompt) + 9
    assert sp.spec_max_depth() == 0 and sm.spec_max_depth() == 3


def test_decode_spec_argmax_is_greedy(d, prompt, plain):
    s = server(d, True)
    x = first_max(s.prefill(prompt))
    out, steps, acc = [x], 0, 0
    while len(out) < 30:
        extra, g = s.decode_spec_argmax(x)
        assert extra == g[:-1] and 1 <= len(g) <= 2
        out += g
        steps += 1
        acc += len(extra)
        x = g[-1]
        assert s.n_past() == len(prompt) + len(out) - 1   # the bonus token is not in the state yet
    assert out == plain[:len(out)]
    assert s.spec_counters() == (steps, acc)
    assert server(d, False).decode_spec_argmax(plain[0]) is None


def test_decode_spec_rows_equal_plain_decode_rows(d, prompt, plain):
    sm, sp = server(d, True), server(d, False)
    x = first_max(sm.prefill(prompt))
    sp.prefill(prompt)
    for _ in range(6):
        extra, rows = sm.decode_spec(x)
        toks = [x] + extra
        assert len(rows) == len(toks)
        for t, r in zip(toks, rows):
            assert np.array_equal(bits(sp.decode(t)), bits(r))
        x = first_max(rows[-1])


def test_spec_rewind_after_an_accepted_step(d, prompt, plain):
    """MtpDriver::rewind through spec_rewind: a step whose draft is accepted (forced to the greedy
    token through the engine's draft-override hook, mtp.rs:328-330) keeps only its first token,
    and decoding continues greedily from there"""
    import oxe_amd as A
    s = server(d, True)
    x = first_max(s.prefill(prompt))
    p0 = s.n_past()
    out = s.engine.mtp_step(x, plain[1])
    assert out == [plain[1], plain[2]] and s.n_past() == p0 + 2
    with pytest.raises(A.EngineError, match="keep out of range"):
        s.spec_rewind(3)
    s.spec_rewind(1)
    assert s.n_past() == p0 + 1
    # x committed; plain[1] is the next input, as if the caller stopped after it
    assert s.decode_argmax(plain[1]) == plain[2]
    x, out = plain[2], [plain[2]]
    while len(out) < 12:
        extra, g = s.decode_spec_argmax(x)
        out += g
        x = g[-1]
    assert out == plain[2:2 + len(out)]


def test_decode_verify_lookup_drafts(d, prompt, plain):
    import oxe_amd as A
    s = server(d, False)
    x = first_max(s.prefill(prompt))
    p0 = s.n_past()
    acc, g = s.decode_verify(x, [plain[1], 7, 9])       # k = 1 (two verify lanes)
    assert acc == [plain[1]] and g == [plain[1], plain[2]] and s.n_past() == p0 + 2
    s.spec_rewind(1)                                     # keep x only
    assert s.n_past() == p0 + 1
    s.spec_rewind(1)                                     # nothing pending: no change
    assert s.n_past() == p0 + 1
    acc, g = s.decode_verify(plain[1], [(plain[2] + 1) % d.n_vocab])
    assert acc == [] and g == [plain[2]] and s.n_past() == p0 + 2
    assert s.spec_counters() == (2, 1)
    assert s.decode_verify(plain[2], []) is None
    assert server(d, True).decode_verify(plain[0], [plain[1]]) is None
    with pytest.raises(A.EngineError, match="token out of vocab"):
        s.decode_verify(plain[2], [d.n_vocab])
    assert s.decode_argmax(plain[2]) == plain[3]


@pytest.mark.parametrize("mtp", [False, True])
def test_snapshot_restore_continues_bit_for_bit(d, prompt, mtp):
    import oxe_amd as A
    s = server(d, mtp)
    x = first_max(s.prefill(prompt))

    def run(x, n):
        toks, rows = [], []
        for _ in range(n):
            if mtp:
                extra, r = s.decode_spec(x)
                toks.append([x] + extra)
                rows += r
                x = first_max(r[-1])
            else:
                r = s.decode(x)
                toks.append([x])
                rows.append(r)
                x = first_max(r)
        return x, toks, rows

    x, _, _ = run(x, 3)
    snap = s.snapshot()
    p = s.n_past()
    assert snap.pos == p and A.ServerEngine.snapshot_bytes(snap) > 0
    c0 = s.spec_counters()
    x1, t1, r1 = run(x, 6)
    c1 = s.spec_counters()
    late = s.snapshot()
    s.restore(snap)
    assert s.n_past() == p
    x2, t2, r2 = run(x, 6)
    assert (x2, t2) == (x1, t1)
    assert all(np.array_equal(bits(a), bits(b)) for a, b in zip(r1, r2))
    # the restored MTP driver drafts exactly as the uninterrupted run did
    c2 = s.spec_counters()
    assert (c2[0] - c1[0], c2[1] - c1[1]) == (c1[0] - c0[0], c1[1] - c0[1])
    # a reused snapshot buffer; a snapshot ahead of the position is refused
    s.restore(snap)
    snap = s.snapshot_reuse(snap)
    assert snap.pos == p
    if late.pos > p:
        with pytest.raises(A.EngineError, match="ahead of the current position"):
            s.restore(late)


@pytest.mark.parametrize("mtp", [False, True])
def test_save_load_state_hands_off_to_a_fresh_engine(d, prompt, mtp):
    import oxe_amd as A
    a = server(d, mtp)
    x = first_max(a.prefill(prompt))
    for _ in range(3):
        x = a.decode_spec_argmax(x)[1][-1] if mtp else a.decode_argmax(x)
    n = a.n_past()
    buf = a.save_state_vec()
    assert a.state_size_hint() >= a.engine.write_state().nbytes
    b = server(d, mtp)
    b.prefill(prompt[:5])                  # a different sequence before the load
    b.load_state(buf, n)
    assert b.n_past() == n and b.state_id() == a.state_id()
    assert np.array_equal(b.save_state_vec(), buf)
    for _ in range(6):
        if mtp:
            ea, ra = a.decode_spec(x)
            eb, rb = b.decode_spec(x)
            assert ea == eb and all(np.array_equal(bits(u), bits(v)) for u, v in zip(ra, rb))
            x = first_max(ra[-1])
        else:
            ra, rb = a.decode(x), b.decode(x)
            assert np.array_equal(bits(ra), bits(rb))
            x = first_max(ra)
    if mtp:   # every step drafted (room for two lanes): a's three earlier steps on top of b's
        assert a.spec_counters()[0] == b.spec_counters()[0] + 3
    with pytest.raises(A.EngineError):
        b.load_state(buf[:-1], n)
    other = server(d, not mtp)
    with pytest.raises(A.EngineError):
        other.load_state(buf, n)


@pytest.mark.parametrize("mtp", [False, True])
def test_kv_rows_and_snapshot_file_rebuild_the_sequence(d, prompt, mtp):
    """the prefix store's path: KV row segments + a snapshot file restore a sequence in a fresh
    engine (kv_rows_save / kv_rows_load / snap_save / snap_load)"""
    import oxe_amd as A
    a = server(d, mtp)
    x = first_max(a.prefill(prompt))
    for _ in range(2):
        x = a.decode_spec_argmax(x)[1][-1] if mtp else a.decode_argmax(x)
    p = a.n_past()
    snap = a.snapshot()
    f = a.snap_save(snap)
    assert np.array_equal(f, a.snap_save_live())
    assert f[:8].view(np.uint64)[0] == p
    assert a.kv_row_bytes() == a.engine.kv_row_bytes()
    seg = [a.kv_rows_save(0, 20), a.kv_rows_save(20, p)]
    with pytest.raises(A.EngineError, match="beyond the current position"):
        a.kv_rows_save(0, p + 1)
    b = server(d, mtp)
    b.prefill(prompt[:9])
    b.kv_rows_load(0, 20, seg[0])
    b.kv_rows_load(20, p, seg[1])
    with pytest.raises(A.EngineError, match="position does not match its rows"):
        b.snap_load(f, p - 1)
    b.snap_load(f, p)
    assert b.n_past() == p
    for _ in range(5):
        ra, rb = a.decode(x), b.decode(x)
        assert np.array_equal(bits(ra), bits(rb))
        x = first_max(ra)
    other = server(d, not mtp)
    with pytest.raises(A.EngineError, match="MTP state does not match this engine"):
        other.snap_load(f, p)


def test_kv_rows_are_write_state_order(d, prompt):
    a = server(d, False)
    a.prefill(prompt)
    p = a.n_past()
    rows = a.kv_rows_save(0, p)
    st = a.engine.write_state()
    assert rows.nbytes == a.kv_row_bytes() * p
    assert np.array_equal(rows, st[: rows.nbytes])


def test_reset_is_a_fresh_engine(d, prompt, plain):
    for mtp in (False, True):
        s = server(d, mtp)
        s.prefill(prompt[:20])
        for _ in range(3):
            s.decode_argmax(5)
        s.reset()
        assert s.n_past() == 0
        f = server(d, mtp)
        assert np.array_equal(bits(s.prefill(prompt)), bits(f.prefill(prompt)))
        x = plain[0]
        for i in range(5):
            if mtp:
                ea, ga = s.decode_spec_argmax(x)
                eb, gb = f.decode_spec_argmax(x)
                assert (ea, ga) == (eb, gb)
                x = ga[-1]
            else:
                x = s.decode_argmax(x)
                assert x == f.decode_argmax(plain[i]) == plain[i + 1]


def test_trait_errors(d, prompt):
    import oxe_amd as A
    s = server(d, True)
    with pytest.raises(A.EngineError, match="empty prefill"):
        s.prefill([])
    with pytest.raises(A.EngineError, match=f"token {d.n_vocab} out of vocab"):
        s.prefill([1, d.n_vocab])
    with pytest.raises(A.EngineError, match="context full"):
        s.prefill([1] * (s.n_ctx() + 1))
    with pytest.raises(A.EngineError, match="out of vocab"):
        s.decode_argmax(d.n_vocab)
    with pytest.raises(A.EngineError, match="rewind without a step"):
        s.spec_rewind(1)
    assert s.n_past() == 0


def test_draft_vocab_from_the_environment(d, prompt, plain, tmp_path, monkeypatch):
    """OXE_MTP_DRAFT_VOCAB=<ranking> [OXE_MTP_DRAFT_K=<k>] (oxe_engine.rs:215-222): the draft head is
    restricted to the ranking's first k ids (lines that do not start with an id are skipped); the
    output is still the greedy sequence. A missing file or a ranking with no id is refused."""
    import oxe_amd as A
    rk = tmp_path / "ranking.txt"
    ids = [i for i in range(d.n_vocab) if i % 3 == 0]
    rk.write_text("# most frequent first\n" + "\n".join(f"{i} {100 - j}" for j, i in enumerate(ids)) + "\n")
    monkeypatch.setenv("OXE_MTP_DRAFT_VOCAB", str(rk))
    monkeypatch.setenv("OXE_MTP_DRAFT_K", "500")
    s = server(d, True)
    x = first_max(s.prefill(prompt))
    out = [x]
    while len(out) < 24:
        _, g = s.decode_spec_argmax(x)
        out += g
        x = g[-1]
    assert out == plain[:len(out)]
    s.close()
    monkeypatch.setenv("OXE_MTP_DRAFT_VOCAB", str(tmp_path / "missing.txt"))
    e = A.Engine(d, seed=SEED, n_ctx=N_CTX)
    with pytest.raises(RuntimeError, match="cannot be read"):
        A.ServerEngine(e, mtp=True)
    (tmp_path / "empty.txt").write_text("not an id\n")
    monkeypatch.setenv("OXE_MTP_DRAFT_VOCAB", str(tmp_path / "empty.txt"))
    with pytest.raises(RuntimeError, match="empty draft vocabulary"):
        A.ServerEngine(e, mtp=True)
    e.close()
