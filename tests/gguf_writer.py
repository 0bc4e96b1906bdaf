"""GGUF v3 writer for the tests (the format the reference reads, crates/gguf/src/lib.rs): header,
typed metadata, tensor table with aligned data offsets, payload streamed tensor by tensor. Also
writes the synthetic model (include/oxe_model.h) as a qwen35moe GGUF file with the reference's
tensor names and ggml layouts (Q8_0 blocks of fp16 d + 32 int8 codes, shape[0] contiguous), so a
file-loaded engine can be compared with the engine that generates the same weights on the device.
Test infrastructure only."""
import struct

import numpy as np

# GGUF metadata value types
VT = dict(u8=0, i8=1, u16=2, i16=3, u32=4, i32=5, f32=6, bool=7, str=8, arr=9, u64=10, i64=11, f64=12)
_FMT = dict(u8="<B", i8="<b", u16="<H", i16="<h", u32="<I", i32="<i", f32="<f", bool="<B", u64="<Q", i64="<q",
            f64="<d")
GGML = dict(F32=0, F16=1, Q8_0=8, Q4_K=12, Q5_K=13, Q6_K=14, BF16=30)
_BLK = {0: (1, 4), 1: (1, 2), 8: (32, 34), 11: (256, 110), 12: (256, 144), 13: (256, 176), 14: (256, 210),
        30: (1, 2), 2: (32, 18), 3: (32, 20), 6: (32, 22), 7: (32, 24), 9: (32, 36), 10: (256, 84), 15: (256, 292)}


def _str(s):
    b = s.encode() if isinstance(s, str) else s
    return struct.pack("<Q", len(b)) + b


def _value(vt, v):
    if vt == "str":
        return _str(v)
    if vt == "arr":
        it, items = v
        out = struct.pack("<IQ", VT[it], len(items))
        return out + b"".join(_value(it, x) for x in items)
    return struct.pack(_FMT[vt], v)


def tensor_bytes(ty, shape):
    n = int(np.prod(shape, dtype=np.uint64)) if shape else 1
    blk, size = _BLK[ty]
    return n // blk * size


def header(meta, tensors, alignment=32, version=3):
    """meta: [(key, vtype, value)]; tensors: [(name, ggml type id, shape)] -> (header bytes,
    data offset, [tensor offsets]) with each tensor's data aligned to `alignment`."""
    out = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, vt, v in meta:
        out += _str(k) + struct.pack("<I", VT[vt]) + _value(vt, v)
    offs, off = [], 0
    for name, ty, shape in tensors:
        off = (off + alignment - 1) // alignment * alignment
        offs.append(off)
        out += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", ty, off)
        off += tensor_bytes(ty, shape)
    data_offset = (len(out) + alignment - 1) // alignment * alignment
    return out, data_offset, offs


def header_at(meta, tensors, alignment=32, version=3):
    """header with explicit data offsets: tensors [(name, ggml type id, shape, offset)]"""
    out = b"GGUF" + struct.pack("<IQQ", version, len(tensors), len(meta))
    for k, vt, v in meta:
        out += _str(k) + struct.pack("<I", VT[vt]) + _value(vt, v)
    for name, ty, shape, off in tensors:
        out += _str(name) + struct.pack("<I", len(shape)) + b"".join(struct.pack("<Q", d) for d in shape)
        out += struct.pack("<IQ", ty, off)
    return out, (len(out) + alignment - 1) // alignment * alignment


def write(path, meta, tensors, alignment=32, version=3):
    """tensors: [(name, ggml type id, shape, payload)] with payload bytes or a callable writing them
    to the open file"""
    hdr, data_offset, offs = header(meta, [(n, t, s) for n, t, s, _ in tensors], alignment, version)
    with open(path, "wb") as f:
        f.write(hdr)
        f.write(b"\0" * (data_offset - len(hdr)))
        for (name, ty, shape, payload), off in zip(tensors, offs):
            pos = f.tell() - data_offset
            assert pos <= off
            f.write(b"\0" * (off - pos))
            start = f.tell()
            if callable(payload):
                payload(f)
            else:
                f.write(payload)
            assert f.tell() - start == tensor_bytes(ty, shape), name
    return data_offset


def q8_blocks(q, d):
    """codes [rows][k] int8 + fp16 scales [rows][k/32] -> ggml Q8_0 blocks (d, then 32 codes)"""
    rows, k = q.shape
    out = np.empty((rows, k // 32, 34), np.uint8)
    out[:, :, 0:2] = np.ascontiguousarray(d).view(np.uint8).reshape(rows, k // 32, 2)
    out[:, :, 2:] = q.reshape(rows, k // 32, 32).view(np.uint8)
    return out.tobytes()


def qwen35moe_meta(desc):
    """the qwen35moe metadata the reference reads (desc.rs:69-140), typed as llama.cpp writes it"""
    a = "qwen35moe"
    return [
        ("general.architecture", "str", a),
        (f"{a}.block_count", "u32", desc.n_layer + 1),
        (f"{a}.context_length", "u32", desc.n_ctx_train),
        (f"{a}.embedding_length", "u32", desc.n_embd),
        (f"{a}.attention.head_count", "u32", desc.n_head),
        (f"{a}.attention.head_count_kv", "u32", desc.n_head_kv),
        (f"{a}.rope.dimension_sections", "arr", ("i32", list(desc.rope_sections))),
        (f"{a}.rope.freq_base", "f32", desc.rope_freq_base),
        (f"{a}.attention.layer_norm_rms_epsilon", "f32", desc.rms_eps),
        (f"{a}.expert_count", "u32", desc.n_expert),
        (f"{a}.expert_used_count", "u32", desc.n_expert_used),
        (f"{a}.attention.key_length", "u32", desc.head_dim),
        (f"{a}.attention.value_length", "u32", desc.head_dim),
        (f"{a}.expert_feed_forward_length", "u32", desc.ff_exp),
        (f"{a}.expert_shared_feed_forward_length", "u32", desc.ff_shexp),
        (f"{a}.ssm.conv_kernel", "u32", desc.ssm_conv_kernel),
        (f"{a}.ssm.state_size", "u32", desc.ssm_d_state),
        (f"{a}.ssm.group_count", "u32", desc.ssm_n_kheads),
        (f"{a}.ssm.time_step_rank", "u32", desc.ssm_n_vheads),
        (f"{a}.ssm.inner_size", "u32", desc.ssm_d_inner),
        (f"{a}.full_attention_interval", "u32", desc.full_attention_interval),
        (f"{a}.rope.dimension_count", "u32", desc.n_rot),
        (f"{a}.nextn_predict_layers", "u32", 1),
        ("general.file_type", "u32", 7),
    ]


def synth_model_tensors(O, desc, seed, types=None):
    """(name, type, shape, payload) of every tensor of the synthetic model, generated by the
    oracle from the same counter-based generator the device uses. types: {(layer, kind): ggml type}
    for matrices written as K-quants (11..14, the oracle's synthetic blocks) or F32 (0) instead of
    Q8_0 (layer GLOBAL_LAYER: the LM head), as the oracle's typed engine builds them."""
    T, G = O.T, O.GLOBAL_LAYER
    E, V = desc.n_embd, desc.n_vocab
    NCH = desc.ssm_d_inner + 2 * desc.ssm_n_kheads * desc.ssm_d_state
    NH, HD, NKV, NEXP, FF = desc.n_head, desc.head_dim, desc.n_head_kv, desc.n_expert, desc.ff_exp
    F32 = GGML["F32"]
    types = types or {}

    def ty(layer, kind):
        return types.get((layer, kind), GGML["Q8_0"])

    def mat(layer, kind, rows, k):
        t = ty(layer, kind)
        if t == GGML["Q8_0"]:
            return lambda f: f.write(q8_blocks(*O.synth_q8(seed, layer, kind, rows, k)))
        if t == F32:
            return lambda f: f.write(O.synth_f32(seed, layer, kind, rows * k).tobytes())
        return lambda f: f.write(O.synth_kq(seed, layer, kind, t, rows, k).tobytes())

    def matx(layer, kind, rows, k):
        t = ty(layer, kind)

        def w(f):
            for e in range(NEXP):
                if t == GGML["Q8_0"]:
                    f.write(q8_blocks(*O.synth_q8(seed, layer, kind, rows, k, expert=e)))
                else:
                    f.write(O.synth_kq(seed, layer, kind, t, rows, k, expert=e).tobytes())
        return w

    q8, q8x = mat, matx

    def f32(layer, kind, n):
        return lambda f: f.write(O.synth_f32(seed, layer, kind, n).tobytes())

    out = [("output.weight", ty(G, T["OUTPUT"]), [E, V], q8(G, T["OUTPUT"], V, E)),
           ("output_norm.weight", F32, [E], f32(G, T["OUT_NORM"], E)),
           ("token_embd.weight", ty(G, T["TOK_EMBD"]), [E, V], q8(G, T["TOK_EMBD"], V, E))]
    for il in range(desc.n_layer + 1):
        p = f"blk.{il}."
        att = il == desc.n_layer or (il + 1) % desc.full_attention_interval == 0
        t = [(p + "attn_norm.weight", F32, [E], f32(il, T["ATTN_NORM"], E)),
             (p + "post_attention_norm.weight", F32, [E], f32(il, T["POST_NORM"], E))]
        if not att:
            t += [(p + "attn_qkv.weight", ty(il, T["DN_QKV"]), [E, NCH], q8(il, T["DN_QKV"], NCH, E)),
                  (p + "attn_gate.weight", ty(il, T["DN_Z"]), [E, desc.ssm_d_inner], q8(il, T["DN_Z"], desc.ssm_d_inner, E)),
                  (p + "ssm_beta.weight", ty(il, T["DN_BETA"]), [E, desc.ssm_n_vheads], q8(il, T["DN_BETA"], desc.ssm_n_vheads, E)),
                  (p + "ssm_alpha.weight", ty(il, T["DN_ALPHA"]), [E, desc.ssm_n_vheads], q8(il, T["DN_ALPHA"], desc.ssm_n_vheads, E)),
                  (p + "ssm_out.weight", ty(il, T["DN_OUT"]), [desc.ssm_d_inner, E], q8(il, T["DN_OUT"], E, desc.ssm_d_inner)),
                  (p + "ssm_conv1d.weight", F32, [desc.ssm_conv_kernel, NCH],
                   f32(il, T["DN_CONV"], NCH * desc.ssm_conv_kernel)),
                  (p + "ssm_a", F32, [desc.ssm_n_vheads], f32(il, T["DN_A"], desc.ssm_n_vheads)),
                  (p + "ssm_dt.bias", F32, [desc.ssm_n_vheads], f32(il, T["DN_DT"], desc.ssm_n_vheads)),
                  (p + "ssm_norm.weight", F32, [desc.ssm_d_state], f32(il, T["DN_NORM"], desc.ssm_d_state))]
        else:
            t += [(p + "attn_q.weight", ty(il, T["ATT_Q"]), [E, 2 * NH * HD], q8(il, T["ATT_Q"], 2 * NH * HD, E)),
                  (p + "attn_k.weight", ty(il, T["ATT_K"]), [E, NKV * HD], q8(il, T["ATT_K"], NKV * HD, E)),
                  (p + "attn_v.weight", ty(il, T["ATT_V"]), [E, NKV * HD], q8(il, T["ATT_V"], NKV * HD, E)),
                  (p + "attn_output.weight", ty(il, T["ATT_OUT"]), [NH * HD, E], q8(il, T["ATT_OUT"], E, NH * HD)),
                  (p + "attn_q_norm.weight", F32, [HD], f32(il, T["ATT_QNORM"], HD)),
                  (p + "attn_k_norm.weight", F32, [HD], f32(il, T["ATT_KNORM"], HD))]
        t += [(p + "ffn_gate_inp.weight", F32, [E, NEXP], f32(il, T["ROUTER"], NEXP * E)),
              (p + "ffn_gate_inp_shexp.weight", F32, [E], f32(il, T["SHEXP_GATE"], E)),
              (p + "ffn_gate_shexp.weight", ty(il, T["GATE_SHEXP"]), [E, desc.ff_shexp], q8(il, T["GATE_SHEXP"], desc.ff_shexp, E)),
              (p + "ffn_up_shexp.weight", ty(il, T["UP_SHEXP"]), [E, desc.ff_shexp], q8(il, T["UP_SHEXP"], desc.ff_shexp, E)),
              (p + "ffn_down_shexp.weight", ty(il, T["DOWN_SHEXP"]), [desc.ff_shexp, E], q8(il, T["DOWN_SHEXP"], E, desc.ff_shexp)),
              (p + "ffn_gate_exps.weight", ty(il, T["GATE_EXPS"]), [E, FF, NEXP], q8x(il, T["GATE_EXPS"], FF, E)),
              (p + "ffn_up_exps.weight", ty(il, T["UP_EXPS"]), [E, FF, NEXP], q8x(il, T["UP_EXPS"], FF, E)),
              (p + "ffn_down_exps.weight", ty(il, T["DOWN_EXPS"]), [FF, E, NEXP], q8x(il, T["DOWN_EXPS"], E, FF))]
        if il == desc.n_layer:
            t += [(p + "nextn.eh_proj.weight", ty(il, T["EH_PROJ"]), [2 * E, E], q8(il, T["EH_PROJ"], E, 2 * E)),
                  (p + "nextn.enorm.weight", F32, [E], f32(il, T["ENORM"], E)),
                  (p + "nextn.hnorm.weight", F32, [E], f32(il, T["HNORM"], E)),
                  (p + "nextn.shared_head_norm.weight", F32, [E], f32(il, T["HEAD_NORM"], E))]
        out += t
    return out


def write_synth_model(path, O, desc, seed, types=None):
    return write(path, qwen35moe_meta(desc), synth_model_tensors(O, desc, seed, types))
