"""Writes the golden fixtures of this directory from the CPU oracle (test infrastructure).

The reference stores no numeric vectors for its decode path (its goldens are FNV hashes keyed to
the aarch64 kernel path, crates/model/src/tests/longctx.rs:648-722), so these fixtures are the
oracle's outputs on fixed inputs, pinned here so that any later change of the oracle or of the
device path shows up as a diff against committed data:
  config1_slice.npz  64 rows of the config-1 Q8_0 GEMV (W [4096 x 2048] seed 0), 2 lanes:
                     codes, scales, x, quantized x, int32 block sums, y
  route.npz          router softmax -> top-8 -> renormalised weights for 2 lanes of 256 logits
  dn_step.npz        one gated delta-rule head step (S_v 128)
  attn_head.npz      one attention head (head_dim 256, n_kv 256, pos_last 200)
  engine_small.npz   argmax ids and FNV-1a-64 hashes of logits / h_nextn of the 4-layer model over
                     a prompt and 6 greedy steps
  config4_ids.npz    BASELINE config 4 at its stated size: the 35B-A3B model (seed 0), the reference
                     bench prompt of 512 ids prefilled through MtpDriver::prefill, then 264 greedy
                     MTP-1 steps; the generated ids as the reference's bench records them (every
                     token fed to the target, oxe.rs:2108-2133) and their generated_hash
  config5_state.npz  BASELINE config 5 on the 4-layer model (seed 7): 2048 prompt tokens decoded token
                     by token; SHA-256 of Engine::write_state's bytes (K rows, V^T rows, conv state, S),
                     of the last token's logits and h_nextn, and the next token
  config5_full_state.npz  the same on the config-4 model (35B-A3B, 40 layers, seed 0), config 5's
                     stated model (~40 GB of host memory, tens of minutes on 8 threads)
Run: python tests/golden/make_golden.py [name ...]   (no name: the small fixtures; config4_ids needs
~40 GB of host memory and several minutes on 16 threads)
"""
import hashlib
import ctypes as C
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(HERE, "..", "..", "oracle"))
import oracle as O  # noqa: E402


def fnv64(a):
    h = 0xCBF29CE484222325
    for b in np.ascontiguousarray(a).view(np.uint8).tobytes():
        h = ((h ^ b) * 0x100000001B3) & 0xFFFFFFFFFFFFFFFF
    return h


def fp(a):
    return O.ptr(a, C.c_float)


def config1_slice():
    wq, wd, x, xq, xd = O.config1_inputs(0)
    wq, wd = wq[:64].copy(), wd[:64].copy()
    y, isum = O.gemv_q8_0(wq, wd, xq, xd, want_isum=True)
    return dict(wq=wq, wd=wd, x=x, xq=xq, xd=xd, isum=isum, y=y)


def route():
    L = O.lib()
    lg = O.synth_normal(7, 9001, 2 * 256, 0.0, 2.0).reshape(2, 256)
    probs = np.empty_like(lg)
    ids = np.empty((2, 8), np.int32)
    w = np.empty((2, 8), np.float32)
    for l in range(2):
        wp = np.empty(256, np.float32)
        L.oxo_soft_max_f32(256, fp(probs[l]), fp(lg[l]), np.float32(1.0), None, fp(wp))
        scratch = np.empty(256, np.int32)
        tie = C.c_int(0)
        L.oxo_argsort_top_k_f32(fp(probs[l]), 256, 8, O.ptr(ids[l], C.c_int32), O.ptr(scratch, C.c_int32), C.byref(tie))
        assert tie.value == 0
        sel = probs[l][ids[l]].copy()
        s = np.float32(L.oxo_vec_sum_f32(8, fp(sel)))
        s = min(max(s, np.float32(6.103515625e-5)), np.float32(np.inf))
        w[l] = sel / np.float32(s)
    return dict(logits=lg, probs=probs, ids=ids, weights=w)


def dn_step():
    L = O.lib()
    sv = 128
    s = (O.synth_normal(7, 9002, sv * sv) * np.float32(0.1)).reshape(sv, sv)
    q = O.synth_normal(7, 9003, sv)
    k = O.synth_normal(7, 9004, sv)
    v = O.synth_normal(7, 9005, sv)
    L.oxo_gdn_l2_norm_f32(fp(q), sv, np.float32(1e-6))
    L.oxo_gdn_l2_norm_f32(fp(k), sv, np.float32(1e-6))
    g, beta = np.float32(-0.25), np.float32(0.6)
    so = np.empty_like(s)
    out = np.empty(sv, np.float32)
    L.oxo_gated_delta_net_step_f32_from(fp(so), fp(s), fp(q), fp(k), fp(v), g, beta, sv, fp(out))
    return dict(s_in=s, q=q, k=k, v=v, g=np.float32(g), beta=np.float32(beta), s_out=so, out=out)


def attn_head():
    L = O.lib()
    hd, n_kv, pos = 256, 256, 200
    q = O.synth_normal(7, 9006, hd)
    k = O.synth_normal(7, 9007, n_kv * hd, 0.0, 0.3).astype(np.float16).reshape(n_kv, hd)
    k_last = O.synth_normal(7, 9008, hd, 0.0, 0.3).astype(np.float16)
    vt = O.synth_normal(7, 9009, hd * (n_kv + 32)).astype(np.float16).reshape(hd, n_kv + 32)
    out = np.empty(hd, np.float32)
    u16 = lambda a: O.ptr(a.view(np.uint16), C.c_uint16)  # noqa: E731
    L.oxo_attn_head_f16(fp(q), u16(k), hd, u16(k_last), u16(vt), n_kv + 32, n_kv, pos, hd, np.float32(1 / 16), fp(out))
    return dict(q=q, k=k, k_last=k_last, vt=vt, pos_last=np.int32(pos), out=out)


def engine_small():
    d = O.desc_small()
    e = O.Engine(d, seed=3, n_ctx=256)
    prompt = (O.bench_prompt(4) % d.n_vocab).astype(np.uint32)
    ids, hl, hh = [], [], []
    x = None
    for t in prompt:
        x = e.step(int(t))
    for _ in range(6):
        ids.append(x)
        hl.append(fnv64(e.logits(0)))
        hh.append(fnv64(e.hidden(0)))
        x = e.step(x)
    return dict(prompt=prompt, ids=np.array(ids, np.uint32), logits_fnv=np.array(hl, np.uint64),
                hidden_fnv=np.array(hh, np.uint64))


def config4_ids(n_prompt=512, n_steps=264):
    sys.path.insert(0, os.path.join(HERE, "..", "..", "snapdragon-engine_amd"))
    import oxe_amd as A
    d = O.desc_35b_a3b()
    e = O.Engine(d, seed=0, n_ctx=n_prompt + 2 * n_steps + 64)
    O.lib().oxo_set_keep_logits(e.h, 0)
    drv = O.Driver(e)
    prompt = O.bench_prompt(n_prompt)
    x = drv.prefill(prompt)
    gen = []
    for i in range(n_steps):
        gen.append(x)
        out = drv.step(x)
        gen += out[:-1]
        x = out[-1]
        if i % 16 == 0:
            print(f"config4: step {i} pos {e.pos}", flush=True)
    gen.append(x)
    ids = np.array(gen, np.uint32)
    return dict(prompt=prompt, steps=np.int32(n_steps), ids=ids, generated_hash=np.array(A.hash_ids(ids)),
                stats=np.array(list(drv.stats().values()), np.int64))


def config5_state(n=2048, d=None, seed=7):
    d = O.desc_small() if d is None else d
    e = O.Engine(d, seed=seed, n_ctx=n + 256)
    O.lib().oxo_set_keep_logits(e.h, 1)
    toks = (O.bench_prompt(n) % d.n_vocab).astype(np.uint32)
    x = None
    for i, t in enumerate(toks):
        x = e.step(int(t))
        if i % 256 == 0:
            print(f"config5: token {i}", flush=True)
    HD, NKV, NCH, NVH, HV = d.head_dim, d.n_head_kv, 8192, d.ssm_n_vheads, 128
    n_ctx = int(e.n_ctx)
    n_att = d.n_layer // d.full_attention_interval + 1
    n_rec = d.n_layer - (n_att - 1)
    L = O.lib()
    kc = np.ctypeslib.as_array(L.oxo_kcache(e.h), (n_att * NKV * n_ctx * HD,)).reshape(n_att, NKV, n_ctx, HD)
    vc = np.ctypeslib.as_array(L.oxo_vcache(e.h), (n_att * NKV * HD * n_ctx,)).reshape(n_att, NKV * HD, n_ctx)
    conv_len, ssm_len = n_rec * NCH * 3, n_rec * NVH * HV * HV
    cur = L.oxo_cur_slot(e.h)
    conv = np.ctypeslib.as_array(L.oxo_conv_state(e.h), (2 * conv_len,))[cur * conv_len:(cur + 1) * conv_len]
    ssm = np.ctypeslib.as_array(L.oxo_ssm_state(e.h), (2 * ssm_len,))[cur * ssm_len:(cur + 1) * ssm_len]
    kv = []
    for ai in range(n_att):
        for h in range(NKV):
            kv.append(kc[ai, h, :n].tobytes())
        kv.append(np.ascontiguousarray(vc[ai, :, :n]).tobytes())
    sha = lambda b: hashlib.sha256(b).hexdigest()  # noqa: E731
    state = b"".join(kv) + conv.tobytes() + ssm.tobytes()
    return dict(prompt=toks, state_sha=np.array(sha(state)), kv_sha=np.array(sha(b"".join(kv))),
                conv_sha=np.array(sha(conv.tobytes())), ssm_sha=np.array(sha(ssm.tobytes())),
                logits_sha=np.array(sha(e.logits(0).tobytes())), hidden_sha=np.array(sha(e.hidden(0).tobytes())),
                next=np.uint32(x), state_bytes=np.int64(len(state)))


def config5_full_state(n=2048):
    """config 5 at its stated size: the config-4 model (35B-A3B, 40 layers, seed 0)"""
    return config5_state(n, O.desc_35b_a3b(), 0)


MAKERS = dict(config1_slice=config1_slice, route=route, dn_step=dn_step, attn_head=attn_head,
              engine_small=engine_small)
LARGE = dict(config4_ids=config4_ids, config5_state=config5_state, config5_full_state=config5_full_state)

# GGUF header fixtures: the fields the tests use of the reference's own test fixtures
# tests/fixtures/{qwen36,ornith}.json (model_inspect.py's reading of the real Qwen3.6 and Ornith
# files: metadata, tensor table, layer / expert layout), copied as data
GGUF_FIXTURE_KEYS = ["source", "file", "file_bytes", "gguf_version", "data_offset", "header_bytes_read",
                     "n_metadata", "architecture", "layers", "experts", "kv_bytes_per_token_f16",
                     "recurrent_state_bytes", "tensor_bytes", "metadata", "tensors"]


def gguf_headers(ref="/root/reference/tests/fixtures"):
    import json
    for name in ("qwen36", "ornith"):
        fx = json.load(open(os.path.join(ref, name + ".json")))
        with open(os.path.join(HERE, f"gguf_header_{name}.json"), "w") as f:
            json.dump({k: fx[k] for k in GGUF_FIXTURE_KEYS}, f, separators=(",", ":"))
        print("wrote", f"gguf_header_{name}.json")


if __name__ == "__main__":
    names = sys.argv[1:]
    if not names:
        for name, fn in MAKERS.items():
            np.savez_compressed(os.path.join(HERE, name + ".npz"), **fn())
            print("wrote", name)
        gguf_headers()
    for name in names:
        fn = {**MAKERS, **LARGE}[name]
        np.savez_compressed(os.path.join(HERE, name + ".npz"), **fn())
        print("wrote", name)
