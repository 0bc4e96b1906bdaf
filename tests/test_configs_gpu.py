"""BASELINE configs 3, 4 and 5 at the sizes BASELINE.json states, on the GPU against the oracle.

  config 3  the 3 delta-net + 1 attention stack with 4096 prior positions: K and V^T of every prior
            position N(0,1) (stored f16), S ~ N(0,0.1), conv state N(0,0.5), handed to both engines
            (Engine::read_state on the device, the oracle's arrays directly); a 1-lane and a 2-lane
            verify return the oracle's logits, hidden rows, new K rows and delta-net state bit for bit
            in both run modes. n_kv = 4352: the attention output reads V^T rows past the 2048
            positions held in LDS from memory.
  config 4  the 35B-A3B model, the reference bench prompt of 512 ids (batched prompt path), then 264
            device-driven MTP-1 steps: the generated ids (as the reference's bench records them,
            every token fed to the target) equal the oracle's (tests/golden/config4_ids.npz, written by
            tests/golden/make_golden.py through MtpDriver::prefill and MtpDriver::step), and so does
            the generated_hash.
  config 5  2048 prompt tokens of the 4-layer model through the batched prefill: SHA-256 of
            Engine::write_state's bytes, of the last logits and h_nextn, and the next token equal the
            oracle's token-by-token decoding (tests/golden/config5_state.npz).
"""
import hashlib
import os

import numpy as np
import pytest

import oracle as O

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
HD, NKV, NCH, NVH, HV = 256, 2, 8192, 32, 128


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def config3_state(d, n_pos, seed=3):
    """write_state bytes for n_pos positions: per attention layer (the MTP layer included) the K rows
    of each kv head, then the V^T rows; then conv [n_rec][8192][3] and S [n_rec][32][128][128]"""
    rng = np.random.default_rng(seed)
    n_att = d.n_layer // d.full_attention_interval + 1
    n_rec = d.n_layer - (n_att - 1)
    K = rng.standard_normal((n_att, NKV, n_pos, HD)).astype(np.float16)
    VT = rng.standard_normal((n_att, NKV * HD, n_pos)).astype(np.float16)
    conv = (0.5 * rng.standard_normal((n_rec, NCH, 3))).astype(np.float32)
    S = (0.1 * rng.standard_normal((n_rec, NVH, HV, HV))).astype(np.float32)
    parts = []
    for ai in range(n_att):
        for h in range(NKV):
            parts.append(K[ai, h].tobytes())
        parts.append(VT[ai].tobytes())
    blob = np.frombuffer(b"".join(parts) + conv.tobytes() + S.tobytes(), np.uint8)
    return blob, K, VT, conv, S


def oracle_with_state(d, n_ctx, n_pos, K, VT, conv, S):
    o = O.Engine(d, seed=3, n_ctx=n_ctx)
    L = O.lib()
    nc = int(o.n_ctx)
    n_att, n_rec = K.shape[0], conv.shape[0]
    kc = np.ctypeslib.as_array(L.oxo_kcache_mut(o.h), (n_att * NKV * nc * HD,)).reshape(n_att, NKV, nc, HD)
    vc = np.ctypeslib.as_array(L.oxo_vcache_mut(o.h), (n_att * NKV * HD * nc,)).reshape(n_att, NKV * HD, nc)
    kc[:, :, :n_pos] = K.view(np.uint16)
    vc[:, :, :n_pos] = VT.view(np.uint16)
    cs = np.ctypeslib.as_array(L.oxo_conv_state(o.h), (2 * conv.size,))
    ss = np.ctypeslib.as_array(L.oxo_ssm_state(o.h), (2 * S.size,))
    cur = L.oxo_cur_slot(o.h)
    cs[cur * conv.size:(cur + 1) * conv.size] = conv.ravel()
    ss[cur * S.size:(cur + 1) * S.size] = S.ravel()
    L.oxo_set_pos(o.h, n_pos)
    return o


@pytest.mark.parametrize("mode", ["fused", "per_phase"])
def test_config3_mixers_at_4096_positions(dev, mode):
    import oxe_amd as A
    d = O.desc_small()
    n_pos, n_ctx = 4096, 4352
    blob, K, VT, conv, S = config3_state(d, n_pos)
    L = O.lib()
    for toks in ([1234], [1234, 77]):
        # fresh engines per run: a verify's lane 0 updates the oracle's current slot in place
        g = A.Engine(d, seed=3, n_ctx=n_ctx)
        if mode == "per_phase":
            g.set_fused(False)
        elif not g.fused:
            pytest.skip("the fused run kernel needs a 256-CU device")
        g.read_state(blob, n_pos)
        o = oracle_with_state(d, n_ctx, n_pos, K, VT, conv, S)
        print(f"config 3 verify {toks} at {n_pos} ({mode})", flush=True)
        ag, ao = g.verify(toks), o.verify(toks)
        assert list(ag) == list(ao)
        for ln in range(len(toks)):
            assert np.array_equal(bits(g.logits(ln)), bits(o.logits(ln))), ln
            assert np.array_equal(bits(g.hidden(ln)), bits(o.hidden(ln))), ln
        # committed: the new K rows of the attention layer and the delta-net state of the last lane,
        # read back through write_state (reference order)
        m = len(toks)
        g.commit(m)
        o.commit(m)
        assert g.pos == o.pos == n_pos + m
        got = g.write_state()
        nc = int(o.n_ctx)
        kc = np.ctypeslib.as_array(L.oxo_kcache(o.h), (K.shape[0] * NKV * nc * HD,)).reshape(K.shape[0], NKV, nc, HD)
        row_bytes = (n_pos + m) * HD * 2
        for h in range(NKV):
            g_rows = got[h * row_bytes:(h + 1) * row_bytes].view(np.uint16).reshape(n_pos + m, HD)
            assert np.array_equal(g_rows[n_pos:], kc[0, h, n_pos:n_pos + m]), h
        ss = np.ctypeslib.as_array(L.oxo_ssm_state(o.h), (2 * S.size,))
        cur = L.oxo_cur_slot(o.h)
        assert np.array_equal(got[-S.size * 4:].view(np.uint32), ss[cur * S.size:(cur + 1) * S.size].view(np.uint32))
        g.close()
        o.close()


def test_config4_bench_ids_equal_oracle(dev):
    import oxe_amd as A
    path = os.path.join(GOLDEN, "config4_ids.npz")
    gold = np.load(path)
    n_steps = int(gold["steps"])
    d = A.desc_35b_a3b()
    g = A.Engine(d, seed=0, n_ctx=512 + 2 * n_steps + 320)
    print("config 4: batched prompt of 512", flush=True)
    x0 = g.mtp_prefill_batched(gold["prompt"])
    assert x0 == int(gold["ids"][0])
    cap = 2 * n_steps + 16
    g.mtp_device_begin(x0, cap)
    g.mtp_device_steps(n_steps, use_graph=True)
    toks, x = g.mtp_device_end(cap)
    gen = np.array([x0] + [int(t) for t in toks], np.uint32)
    want = gold["ids"]
    assert len(gen) == len(want)
    bad = np.flatnonzero(gen != want)
    assert bad.size == 0, f"first differing id at {bad[:4]}"
    assert A.hash_ids(gen) == str(gold["generated_hash"])
    g.close()


def test_config5_prefill_2048_state_hashes(dev):
    import oxe_amd as A
    gold = np.load(os.path.join(GOLDEN, "config5_state.npz"))
    d = O.desc_small()
    toks = gold["prompt"]
    g = A.Engine(d, seed=7, n_ctx=len(toks) + 256)
    print("config 5: prefill 2048", flush=True)
    nx = g.prefill(toks)
    sha = lambda b: hashlib.sha256(b).hexdigest()  # noqa: E731
    state = g.write_state()
    assert state.size == int(gold["state_bytes"])
    assert sha(state.tobytes()) == str(gold["state_sha"])
    assert sha(np.asarray(g.logits(0), np.float32).tobytes()) == str(gold["logits_sha"])
    assert sha(np.asarray(g.hidden(0), np.float32).tobytes()) == str(gold["hidden_sha"])
    assert nx == int(gold["next"])
    g.close()


def test_config5_prefill_2048_full_model_state_hashes(dev):
    """Config 5 at its stated size: the config-4 model (35B-A3B shape, 40 layers, seed 0) prefills the
    2048-token bench prompt in one batched call; the whole recurrent state in the reference's byte
    order (every attention layer's K rows and V^T columns, then the conv and delta-net states), the
    last token's logits and hidden state and the next id equal the oracle's after 2048 single-token
    steps (tests/golden/make_golden.py config5_full_state)."""
    import oxe_amd as A
    gold = np.load(os.path.join(GOLDEN, "config5_full_state.npz"))
    d = A.desc_35b_a3b()
    toks = gold["prompt"]
    n = len(toks)
    g = A.Engine(d, seed=0, n_ctx=n + 256)
    print("config 5 (40 layers): prefill 2048", flush=True)
    nx = g.prefill(toks)
    sha = lambda b: hashlib.sha256(b).hexdigest()  # noqa: E731
    state = g.write_state().tobytes()
    assert len(state) == int(gold["state_bytes"])
    n_att = d.n_layer // d.full_attention_interval + 1
    kv_bytes = n_att * 2 * d.n_head_kv * n * d.head_dim * 2
    n_rec = d.n_layer - (n_att - 1)
    conv_bytes = n_rec * 8192 * 3 * 4
    parts = dict(kv_sha=state[:kv_bytes], conv_sha=state[kv_bytes:kv_bytes + conv_bytes],
                 ssm_sha=state[kv_bytes + conv_bytes:])
    bad = [name for name, b in parts.items() if sha(b) != str(gold[name])]
    assert not bad, f"state parts differing from the oracle: {bad}"
    assert sha(state) == str(gold["state_sha"])
    assert sha(np.asarray(g.logits(0), np.float32).tobytes()) == str(gold["logits_sha"])
    assert sha(np.asarray(g.hidden(0), np.float32).tobytes()) == str(gold["hidden_sha"])
    assert nx == int(gold["next"])
    g.close()
