"""Weights from a GGUF file on the GPU (Gguf::open + ModelDesc::from_header + WeightStore::load,
crates/gguf/src/lib.rs, crates/model/src/desc.rs, weights.rs).

The synthetic model is written as a qwen35moe GGUF file with the reference's tensor names and ggml
layouts (tests/gguf_writer.py, from the oracle's generator); an engine created from the file must
decode bit for bit like the engine that generates the same weights on the device (prefill,
logits, hidden states, speculative steps), which checks every tensor's name, shape, Q8_0 block
split, projection concatenation and gate / up interleave at once. The reference's real Qwen3.6 and
Ornith files (headers rebuilt from its fixtures, sparse files of the real size): both files' types
all load and run."""
import json
import os

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

pytestmark = pytest.mark.gpu

SEED = 5


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def scratch_dir():
    return "/dev/shm" if os.path.isdir("/dev/shm") and os.access("/dev/shm", os.W_OK) else "/tmp"


def test_engine_from_gguf_decodes_like_the_synthetic_engine():
    import oxe_amd as A
    d = O.desc_small()
    path = os.path.join(scratch_dir(), f"oxe_test_synth_{os.getpid()}.gguf")
    try:
        print("writing the synthetic model as GGUF", flush=True)
        W.write_synth_model(path, O, d, SEED)
        print(f"wrote {os.path.getsize(path) >> 20} MiB; loading", flush=True)
        g = A.Engine.from_gguf(path, n_ctx=512)
        s = A.Engine(d, seed=SEED, n_ctx=512)
        for f, _ in d._fields_:
            a, b = getattr(g.desc, f), getattr(d, f)
            assert (list(a) == list(b)) if f == "rope_sections" else a == b, f
        toks = [int(v) % d.n_vocab for v in O.bench_prompt(40)]
        print("prefill and steps", flush=True)
        assert g.prefill(toks) == s.prefill(toks)
        assert np.array_equal(bits(g.logits(0)), bits(s.logits(0)))
        assert np.array_equal(bits(g.hidden(0)), bits(s.hidden(0)))
        x = s.step(7)
        assert g.step(7) == x
        assert np.array_equal(bits(g.logits(0)), bits(s.logits(0)))
        # MTP head: draft, verify, accept through the loaded nextn block
        for _ in range(4):
            og, os_ = g.mtp_step(x), s.mtp_step(x)
            assert og == os_
            x = os_[-1]
        assert np.array_equal(bits(g.hidden(0)), bits(s.hidden(0)))
        g.close()
        s.close()
    finally:
        if os.path.exists(path):
            os.remove(path)


def real_header_file(name):
    """the reference's real model file rebuilt from its header fixture: the header, then a sparse
    data section of the real size (every weight byte zero)"""
    fx = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", f"gguf_header_{name}.json")))
    ids = {"F32": 0, "Q8_0": 8, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14, "BF16": 30}

    def typed(k, v):
        if isinstance(v, str):
            return (k, "str", v)
        if isinstance(v, int):
            return (k, "u32", v)
        if isinstance(v, float):
            return (k, "f32", v)
        return (k, "arr", ("i32", v))

    hdr, data_offset = W.header_at([typed(k, v) for k, v in fx["metadata"].items()],
                                   [(n, ids[t], s, o) for n, t, s, o, _ in fx["tensors"]])
    path = os.path.join(scratch_dir(), f"oxe_test_{name}_{os.getpid()}.gguf")
    with open(path, "wb") as f:
        f.write(hdr)
        f.truncate(data_offset + fx["tensor_bytes"])   # sparse: no data written
    return path


def test_real_qwen36_file_loads_and_decodes():
    """the reference's Qwen3.6 file (header from its fixture, a sparse 21 GiB file of the real size):
    K-quant experts (Q4_K gate / up, Q5_K and Q6_K down), F32 ssm_beta / ssm_alpha, the Q6_K LM
    head and the MTP layer's BF16 routers all load; with every weight zero each logit is +0, so the
    first strict maximum is row 0"""
    import oxe_amd as A
    path = real_header_file("qwen36")
    try:
        print("loading the sparse Qwen3.6 file", flush=True)
        g = A.Engine.from_gguf(path, n_ctx=256)
        assert not g.fused
        assert g.step(1) == 0
        lg = np.asarray(g.logits(0), np.float32)
        assert lg.shape[0] == g.desc.n_vocab and not np.any(bits(lg))
        g.close()
    finally:
        if os.path.exists(path):
            os.remove(path)


def test_real_ornith_file_loads_and_decodes():
    """the reference's Ornith file (header from its fixture, a sparse 16 GiB file of the real size):
    Q4_K delta-net projections (attn_qkv, attn_gate, ssm_beta, ssm_alpha, ssm_out) and attention
    matrices, a Q4_K token embedding, Q3_K / Q4_K experts, Q6_K shared experts and LM head, beside the
    MTP layer's Q8_0 matrices, all load; with every weight zero each logit is +0, so the first strict
    maximum is row 0, and an MTP step runs through the Q8_0 MTP layer over the K-quant embedding"""
    import oxe_amd as A
    path = real_header_file("ornith")
    try:
        print("loading the sparse Ornith file", flush=True)
        g = A.Engine.from_gguf(path, n_ctx=256)
        assert not g.fused
        assert g.step(1) == 0
        lg = np.asarray(g.logits(0), np.float32)
        assert lg.shape[0] == g.desc.n_vocab and not np.any(bits(lg))
        g.close()
        g = A.Engine.from_gguf(path, n_ctx=256)
        assert g.mtp_prefill_batched([1, 2, 3]) == 0
        assert all(t == 0 for t in g.mtp_step(0))
        g.close()
    finally:
        if os.path.exists(path):
            os.remove(path)


def test_repack_q8_0_splits_ggml_blocks(dev):
    """oxe_hip_repack_q8_0: ggml Q8_0 blocks -> codes + scales, exactly the oracle's arrays; the
    repacked weights run the GEMV to the oracle's bits; k not a multiple of 32 is refused"""
    import oxe_amd as A
    import torch
    for rows, k in ((300, 2048), (7, 512), (1, 32)):
        q, d = O.synth_q8(9, 2, O.T["DN_OUT"], rows, k)
        blocks = torch.from_numpy(np.frombuffer(W.q8_blocks(q, d), np.uint8).reshape(rows, k // 32 * 34).copy()).to(dev)
        gq, gd = A.repack_q8_0(blocks, k)
        assert np.array_equal(gq.cpu().numpy(), q)
        assert np.array_equal(gd.cpu().numpy().view(np.uint16), d)
    x = (O.synth_normal(9, 11, 2 * 2048).reshape(2, 2048)).astype(np.float32)
    xq, xd = O.quantize_q8_0(x)
    q, d = O.synth_q8(9, 3, O.T["DN_OUT"], 256, 2048)
    blocks = torch.from_numpy(np.frombuffer(W.q8_blocks(q, d), np.uint8).reshape(256, 64 * 34).copy()).to(dev)
    gq, gd = A.repack_q8_0(blocks, 2048)
    y = A.gemv_q8_0(gq, gd, torch.from_numpy(xq).to(dev), torch.from_numpy(xd.view(np.int16)).to(dev))
    assert np.array_equal(y.cpu().numpy().view(np.uint32), O.gemv_q8_0(q, d, xq, xd).view(np.uint32))
    with pytest.raises(RuntimeError):
        A.repack_q8_0(torch.zeros((2, 34), dtype=torch.uint8, device=dev), 48)


def test_bf16_routers_load_as_their_f32_widening():
    """BF16 routers (the Qwen3.6 file's MTP layer has them) are widened to f32 at load, as the
    reference converts BF16 small tensors (crates/model/src/mtp.rs:109-128): a file with BF16 routers
    decodes bit for bit like the same file with those values stored as F32"""
    import oxe_amd as A
    d = O.desc_small()
    conv = {f"blk.{il}.{n}" for il in (0, d.n_layer) for n in ("ffn_gate_inp.weight", "ffn_gate_inp_shexp.weight")}

    def bf16_bits(x):
        u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
        r = (u + 0x7FFF + ((u >> 16) & 1)) >> 16          # round to nearest even
        return r.astype(np.uint16)

    def variant(as_bf16):
        out = []
        for name, ty, shape, payload in W.synth_model_tensors(O, d, SEED):
            if name in conv:
                import io
                buf = io.BytesIO()
                payload(buf)
                b = bf16_bits(np.frombuffer(buf.getvalue(), np.float32))
                data = b.tobytes() if as_bf16 else (b.astype(np.uint32) << 16).tobytes()
                out.append((name, W.GGML["BF16"] if as_bf16 else ty, shape, (lambda data: lambda f: f.write(data))(data)))
            else:
                out.append((name, ty, shape, payload))
        return out

    paths = [os.path.join(scratch_dir(), f"oxe_test_bf16_{i}_{os.getpid()}.gguf") for i in range(2)]
    try:
        for p, as_bf16 in zip(paths, (False, True)):
            print(f"writing {'BF16' if as_bf16 else 'F32'} routers", flush=True)
            W.write(p, W.qwen35moe_meta(d), variant(as_bf16))
        ga, gb = A.Engine.from_gguf(paths[0], n_ctx=512), A.Engine.from_gguf(paths[1], n_ctx=512)
        toks = [int(v) % d.n_vocab for v in O.bench_prompt(24)]
        assert ga.prefill(toks) == gb.prefill(toks)
        x = ga.step(3)
        assert gb.step(3) == x
        for _ in range(3):
            ra, rb = ga.mtp_step(x), gb.mtp_step(x)
            assert ra == rb
            x = ra[-1]
        assert np.array_equal(bits(ga.logits(0)), bits(gb.logits(0)))
        assert np.array_equal(bits(ga.hidden(0)), bits(gb.hidden(0)))
        ga.close()
        gb.close()
    finally:
        for p in paths:
            if os.path.exists(p):
                os.remove(p)


def _sparse_synth_file(path, desc, extra=(), meta_over=None):
    """the synthetic model's header (+ extra tensors) over a sparse data region: enough for every
    check the loader makes before reading a payload"""
    tensors = [(n, t, s) for n, t, s, _ in W.synth_model_tensors(O, desc, 0)] + list(extra)
    meta = W.qwen35moe_meta(desc)
    if meta_over:
        meta = [(k, vt, meta_over.get(k, v)) for k, vt, v in meta]
    hdr, data_offset, offs = W.header(meta, tensors)
    end = max(o + W.tensor_bytes(t, s) for o, (_, t, s) in zip(offs, tensors))
    with open(path, "wb") as f:
        f.write(hdr)
        f.truncate(data_offset + end)


def test_mtp_head_with_own_embedding_or_head_is_refused():
    """the reference's MTP loader refuses nextn.embed_tokens / nextn.shared_head_head (mtp.rs:97-99)"""
    import oxe_amd as A
    d = O.desc_small()
    for name in ("nextn.embed_tokens.weight", "nextn.shared_head_head.weight"):
        path = os.path.join("/tmp", f"oxe_test_nextn_{os.getpid()}.gguf")
        try:
            _sparse_synth_file(path, d, [(f"blk.{d.n_layer}.{name}", W.GGML["Q8_0"], [d.n_embd, d.n_vocab])])
            with pytest.raises(A.GgufError, match="MTP head with its own embedding/head is not supported"):
                A.Engine.from_gguf(path, n_ctx=256)
        finally:
            if os.path.exists(path):
                os.remove(path)


def test_load_into_engine_with_another_descriptor_is_refused():
    """oxe_engine_load_gguf: a file whose norms' eps or RoPE base differs from the engine's is refused"""
    import oxe_amd as A
    d = O.desc_small()
    g = A.Engine(d, seed=0, n_ctx=256)
    try:
        for key, val in (("qwen35moe.attention.layer_norm_rms_epsilon", 1e-5), ("qwen35moe.rope.freq_base", 5e6)):
            path = os.path.join("/tmp", f"oxe_test_desc_{os.getpid()}.gguf")
            try:
                _sparse_synth_file(path, d, meta_over={key: val})
                f = A.Gguf(path)
                with pytest.raises(A.GgufError, match="descriptor"):
                    g.load_gguf(f)
                f.close()
            finally:
                if os.path.exists(path):
                    os.remove(path)
    finally:
        g.close()
