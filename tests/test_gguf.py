"""GGUF reader and model descriptor (crates/gguf/src/lib.rs:268-400, crates/model/src/desc.rs:69-178)
on the CPU: the library's host-side parser through the C ABI.

Pinned by: the reference's own header fixtures (its tests/fixtures/qwen36.json and ornith.json,
copied as tests/golden/gguf_header_*.json: the tensor table model_inspect.py read from the real
Qwen3.6 and Ornith files, and their metadata) -
a header rebuilt from each fixture parses to exactly that table and to the layer / expert layout
the fixture records; synthetic files holding every metadata value type, long arrays, non-default
alignment and multi-dimensional tensors; and every error case the reference checks."""
import json
import os
import struct

import numpy as np
import pytest

import gguf_writer as W
import oracle as O

FIXTURES = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GGML_NAME = {0: "F32", 1: "F16", 8: "Q8_0", 11: "Q3_K", 12: "Q4_K", 13: "Q5_K", 14: "Q6_K", 30: "BF16"}
NAME_ID = {v: k for k, v in GGML_NAME.items()}


def A():
    import oxe_amd
    return oxe_amd


def small_meta():
    return [("general.architecture", "str", "toy"),
            ("general.alignment", "u32", 64),
            ("u8", "u8", 200), ("i8", "i8", -3), ("u16", "u16", 60000), ("i16", "i16", -30000),
            ("u32", "u32", 4000000000), ("i32", "i32", -7), ("f32", "f32", 1.5), ("bool", "bool", 1),
            ("u64", "u64", 2 ** 40), ("i64", "i64", 5), ("f64", "f64", 0.1), ("str", "str", "héllo"),
            ("arr", "arr", ("i32", [11, 11, 10, 0])),
            ("nested", "arr", ("arr", [("u8", [1, 2]), ("u8", [3])])),
            ("long_u32", "arr", ("u32", list(range(5000)))),
            ("long_str", "arr", ("str", ["t%d" % i for i in range(4100)])),
            ("after", "u32", 42)]


def small_tensors():
    return [("a", 0, [3, 2]), ("b", 8, [64, 2]), ("c", 12, [256, 1]), ("d", 8, [32, 2, 3]), ("e", 30, [5])]


def small_file(tmp_path, alignment=64):
    ts = [(n, t, s, bytes(W.tensor_bytes(t, s))) for n, t, s in small_tensors()]
    path = tmp_path / "small.gguf"
    W.write(path, small_meta(), ts, alignment=alignment)
    return path


def test_small_file_parses(tmp_path):
    path = small_file(tmp_path)
    hdr, data_offset, offs = W.header(small_meta(), small_tensors(), alignment=64)
    with A().Gguf(path) as g:
        info = g.info()
        assert info["version"] == 3 and info["n_tensors"] == 5 and info["n_meta"] == len(small_meta())
        assert info["header_bytes"] == len(hdr) and info["data_offset"] == data_offset
        assert data_offset % 64 == 0
        assert info["file_bytes"] == os.path.getsize(path)
        got = g.tensors()
        for (name, ty, shape), off, t in zip(small_tensors(), offs, got):
            assert t == (name, ty, shape, off, W.tensor_bytes(ty, shape))
        assert g.str("general.architecture") == "toy"
        assert g.u64("u8") == 200 and g.u64("u16") == 60000 and g.u64("u32") == 4000000000
        assert g.u64("u64") == 2 ** 40 and g.u64("i64") == 5 and g.u64("bool") is None
        assert g.u64("i8") is None and g.u64("i32") is None          # negative: not an unsigned value
        assert g.f64("f32") == 1.5 and g.f64("f64") == 0.1 and g.f64("u8") == 200.0
        assert g.str("str") == "héllo" and g.str("u8") is None
        assert g.array("arr") == (5, 4, [11.0, 11.0, 10.0, 0.0])
        assert g.array("nested")[:2] == (9, 2)
        assert g.array("long_u32") == (4, 5000, None)                # counted, not kept
        assert g.array("long_str") == (8, 4100, None)
        assert g.u64("after") == 42                                   # parsing resumed after the long arrays
        assert g.u64("missing") is None and g.array("u8") is None
        assert [k for k, _ in g.meta_keys()] == [k for k, _, _ in small_meta()]


def test_in_memory_parse_and_bounds(tmp_path):
    path = small_file(tmp_path)
    data = open(path, "rb").read()
    with A().Gguf(data=data) as g:
        assert g.info()["file_bytes"] == len(data)
        g.check_bounds(len(data))
        with pytest.raises(A().GgufError, match="e: data beyond end of file"):
            g.check_bounds(len(data) - 1)


def _err(data, match):
    with pytest.raises(A().GgufError, match=match):
        A().Gguf(data=data)


def test_header_errors():
    good, _, _ = W.header([("k", "u32", 1)], [("t", 0, [4])])
    _err(b"GGUX" + good[4:], "not a GGUF file")
    _err(good[:4] + struct.pack("<I", 1) + good[8:], "unsupported GGUF version 1")
    for cut in (3, 10, 30, len(good) - 3):
        # a cut inside the entries trips the count check first when the rest cannot hold them
        _err(good[:cut], "truncated GGUF header|not a GGUF file|more than its")
    # counts the remaining bytes cannot hold are refused before allocation
    _err(good[:8] + struct.pack("<QQ", 2 ** 40, 1) + good[24:], "more than its")
    hdr, _ = W.header_at([], [("t", 0, [1, 1, 1, 1, 1], 0)])
    _err(hdr, "5 dimensions")
    hdr, _ = W.header_at([], [("t", 0, [2 ** 63 + 1], 0)])
    _err(hdr, "dimension above 2\\^63")
    hdr, _ = W.header_at([], [("t", 99, [4], 0)])
    _err(hdr, "unknown ggml type id 99")
    hdr, _ = W.header_at([], [("t", 8, [33], 0)])
    _err(hdr, "33 elements not a multiple of Q8_0 block 32")
    hdr, _ = W.header_at([], [("t", 0, [2 ** 40, 2 ** 40], 0)])
    _err(hdr, "element count overflows")
    hdr, _ = W.header_at([("general.alignment", "u32", 24)], [])
    _err(hdr, "general.alignment 24 is not a power of two")
    bad = b"GGUF" + struct.pack("<IQQ", 3, 0, 1) + W._str("k") + struct.pack("<I", 77) + b"\0" * 16
    _err(bad, "unknown metadata value type 77")


def test_file_errors(tmp_path):
    path = small_file(tmp_path)
    data = open(path, "rb").read()
    short = tmp_path / "short.gguf"
    short.write_bytes(data[:-1])
    with pytest.raises(A().GgufError, match="e: data beyond end of file"):
        A().Gguf(short)
    with pytest.raises(A().GgufError, match="cannot open"):
        A().Gguf(tmp_path / "absent.gguf")


def _typed(k, v):
    if isinstance(v, str):
        return (k, "str", v)
    if isinstance(v, bool):
        return (k, "bool", int(v))
    if isinstance(v, int):
        return (k, "u32", v)
    if isinstance(v, float):
        return (k, "f32", v)
    if isinstance(v, list):
        return (k, "arr", ("i32", v))
    raise TypeError(v)


@pytest.mark.parametrize("fixture", ["qwen36", "ornith"])
def test_reference_fixture_tensor_table_and_desc(fixture):
    """A header rebuilt from the fixture's metadata and tensor table parses back to that table
    (names, types, shapes, data offsets, byte sizes, total bytes) and to the fixture's layer and
    expert layout through ModelDesc::from_header."""
    fx = json.load(open(os.path.join(FIXTURES, f"gguf_header_{fixture}.json")))
    meta = [_typed(k, v) for k, v in fx["metadata"].items()]
    ts = [(n, NAME_ID[t], shape, off) for n, t, shape, off, _ in fx["tensors"]]
    hdr, data_offset = W.header_at(meta, ts)
    with A().Gguf(data=hdr) as g:
        got = g.tensors()
        assert len(got) == len(fx["tensors"])
        for (n, ty, shape, off, nb), r in zip(got, fx["tensors"]):
            assert (n, GGML_NAME[ty], shape, off, nb) == (r[0], r[1], r[2], r[3], r[4])
        assert sum(t[4] for t in got) == fx["tensor_bytes"]
        assert g.info()["data_offset"] == data_offset
        g.check_bounds(data_offset + max(t[3] + t[4] for t in got))
        d = g.model_desc()
    lay = fx["layers"]
    assert d.n_layer == lay["target"] and d.has_mtp == 1 and lay["block_count"] == d.n_layer + 1
    assert d.full_attention_interval == lay["full_attention_interval"]
    att = [il for il in range(d.n_layer) if (il + 1) % d.full_attention_interval == 0]
    assert att == lay["full_attention"] and d.n_layer - len(att) == lay["recurrent"]
    assert (d.n_expert, d.n_expert_used) == (fx["experts"]["count"], fx["experts"]["used"])
    assert d.n_vocab == [t for t in fx["tensors"] if t[0] == "output.weight"][0][2][1]
    m = fx["metadata"]
    assert (d.n_embd, d.n_head, d.n_head_kv, d.head_dim) == (
        m["qwen35moe.embedding_length"], m["qwen35moe.attention.head_count"],
        m["qwen35moe.attention.head_count_kv"], m["qwen35moe.attention.key_length"])
    assert list(d.rope_sections) == m["qwen35moe.rope.dimension_sections"]
    assert d.rms_eps == np.float32(m["qwen35moe.attention.layer_norm_rms_epsilon"])
    assert d.rope_freq_base == np.float32(m["qwen35moe.rope.freq_base"])
    # the KV / recurrent budgets the fixture records follow from the descriptor
    assert 2 * 2 * d.n_head_kv * d.head_dim * len(att) == fx["kv_bytes_per_token_f16"]
    nch = d.ssm_d_inner + 2 * d.ssm_n_kheads * d.ssm_d_state
    rec = 4 * ((d.ssm_conv_kernel - 1) * nch + d.ssm_d_state * d.ssm_d_inner) * lay["recurrent"]
    assert rec == fx["recurrent_state_bytes"]


def test_desc_errors():
    fx = json.load(open(os.path.join(FIXTURES, "gguf_header_qwen36.json")))
    meta = [_typed(k, v) for k, v in fx["metadata"].items()]
    ts = [(n, NAME_ID[t], shape, off) for n, t, shape, off, _ in fx["tensors"]]

    def desc_err(meta, ts, match):
        hdr, _ = W.header_at(meta, ts)
        with A().Gguf(data=hdr) as g:
            with pytest.raises(A().GgufError, match=match):
                g.model_desc()

    desc_err([m if m[0] != "general.architecture" else (m[0], "str", "llama") for m in meta], ts,
             "architecture llama is not supported")
    desc_err([m for m in meta if m[0] != "qwen35moe.expert_count"], ts, "missing qwen35moe.expert_count")
    desc_err([m if m[0] != "qwen35moe.full_attention_interval" else (m[0], "u32", 3) for m in meta], ts,
             "layer 2: tensors say Recurrent, full_attention_interval says Attention")
    desc_err(meta, [t for t in ts if t[0] != "blk.5.ssm_a"], "layer 5: cannot classify")
    desc_err(meta, [t if t[0] != "blk.0.attn_qkv.weight" else (t[0], t[1], [2048, 8000], t[3]) for t in ts],
             "layer 0: attn_qkv shape")
    desc_err(meta, [t for t in ts if t[0] != "output.weight"], "no output.weight")
    desc_err([m for m in meta if m[0] != "qwen35moe.rope.dimension_sections"], ts, "dimension_sections")


def test_synthetic_model_file_header_gives_the_engine_desc():
    """the writer's synthetic model (the engine's weights as a qwen35moe file) declares the shape
    the engine is created with"""
    d0 = O.desc_small()
    ts = [(n, t, s) for n, t, s, _ in W.synth_model_tensors(O, d0, 0)]
    hdr, _, _ = W.header(W.qwen35moe_meta(d0), ts)
    with A().Gguf(data=hdr) as g:
        d = g.model_desc()
    for f, _ in d._fields_:
        a, b = getattr(d, f), getattr(d0, f)
        if f == "rope_sections":
            assert list(a) == list(b)
        else:
            assert a == b, f
