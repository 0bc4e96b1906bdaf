"""Python binding of liboxe_amd.so (the MI355X C ABI declared in include/oxe_amd.h).

PyTorch is used only for device memory and the current HIP stream; every computation runs in the
library's own gfx950 kernels. Loading fails loudly when the library is missing: there is no CPU
fallback anywhere on the product path.
"""
import ctypes as C
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboxe_amd.so")

_lib = None


class NotBuilt(RuntimeError):
    pass


def lib():
    global _lib
    if _lib is None:
        # torch ships its own libamdhip64.so.7 (same soname as the system ROCm one this library
        # links): load torch first so one HIP runtime serves both in this process.
        import torch  # noqa: F401
        if not os.path.exists(LIB_PATH):
            raise NotBuilt(f"{LIB_PATH} is missing: run `python snapdragon-engine_amd/build.py` (or __graft_entry__.build())")
        L = C.CDLL(LIB_PATH)
        vp, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        sig = {
            "oxe_hip_quantize_row_q8_0": (i32, [vp, i64, i64, vp, vp, vp]),
            "oxe_hip_gemv_q8_0": (i32, [i64, i64, i32, vp, vp, vp, vp, vp, vp, vp]),
            "oxe_hip_repack_q8_0": (i32, [vp, i64, i64, vp, vp, vp]),
            "oxe_hip_gemm_q8_0": (i32, [i64, i64, i64, vp, vp, vp, vp, vp, i64, vp]),
            "oxe_hip_eval_unary": (i32, [i32, C.c_uint32, i64, i64, vp, vp]),
            "oxe_hip_quantize_row_q8_K": (i32, [vp, i64, i64, vp, vp]),
            "oxe_hip_vl_gemv": (i32, [i32, i64, i64, i32, vp, vp, vp, vp]),
            "oxe_hip_route_f32": (i32, [vp, i64, vp, vp, vp, vp]),
        }
        for name, (res, args) in sig.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


class ModelDesc(C.Structure):
    """oxe_model_desc of include/oxe_model.h (the reference's ModelDesc, crates/model/src/desc.rs:15-140)."""
    _fields_ = [
        ("n_layer", C.c_int32), ("n_embd", C.c_int32), ("n_vocab", C.c_int32),
        ("n_head", C.c_int32), ("n_head_kv", C.c_int32), ("head_dim", C.c_int32),
        ("n_expert", C.c_int32), ("n_expert_used", C.c_int32), ("ff_exp", C.c_int32), ("ff_shexp", C.c_int32),
        ("ssm_conv_kernel", C.c_int32), ("ssm_d_state", C.c_int32), ("ssm_n_kheads", C.c_int32),
        ("ssm_n_vheads", C.c_int32), ("ssm_d_inner", C.c_int32),
        ("full_attention_interval", C.c_int32), ("n_rot", C.c_int32), ("rope_sections", C.c_int32 * 4),
        ("rms_eps", C.c_float), ("rope_freq_base", C.c_float), ("n_ctx_train", C.c_int32), ("has_mtp", C.c_int32),
    ]


def desc_35b_a3b(**over):
    """The qwen35moe 35B-A3B shape (40 layers, 3 delta-net : 1 attention, 256 experts top-8, vocab
    151936, MTP block), as the reference reads it from GGUF metadata (desc.rs:69-140)."""
    d = ModelDesc(n_layer=40, n_embd=2048, n_vocab=151936, n_head=16, n_head_kv=2, head_dim=256,
                  n_expert=256, n_expert_used=8, ff_exp=512, ff_shexp=512, ssm_conv_kernel=4,
                  ssm_d_state=128, ssm_n_kheads=16, ssm_n_vheads=32, ssm_d_inner=4096,
                  full_attention_interval=4, n_rot=64, rms_eps=9.999999974752427e-07,
                  rope_freq_base=1e7, n_ctx_train=262144, has_mtp=1)
    d.rope_sections[:] = [11, 11, 10, 0]
    for k, v in over.items():
        setattr(d, k, v)
    return d


def bench_prompt(n):
    """oxe bench's prompt ids (crates/oxe-cli/src/bin/oxe.rs:428-435): (i*2654435761 mod 2^32) % 150000 + 1000."""
    import numpy as np
    i = np.arange(n, dtype=np.uint64)
    return (((i * 2654435761) & 0xFFFFFFFF) % 150000 + 1000).astype(np.uint32)


def hash_bytes(b):
    """The reference's 64-bit content hash (crates/model/src/weights.rs:254-272): four multiply-rotate
    lanes over 32-byte words, a tail lane over the remaining bytes, then the lanes folded."""
    M = 0xFFFFFFFFFFFFFFFF
    K = (0x9E3779B97F4A7C15, 0xC2B2AE3D27D4EB4F, 0x165667B19E3779F9, 0xD6E8FEB86659FD93)
    rotl = lambda v, r: ((v << r) | (v >> (64 - r))) & M  # noqa: E731
    h = [0x243F6A8885A308D3, 0x13198A2E03707344, 0xA4093822299F31D0, 0x082EFA98EC4E6C89]
    words = len(b) // 32
    for i in range(words):
        for l in range(4):
            w = int.from_bytes(b[i * 32 + l * 8:i * 32 + l * 8 + 8], "little")
            h[l] = rotl(((h[l] ^ w) * K[l]) & M, 31)
    x = (len(b) * K[0]) & M
    for v in b[words * 32:]:
        x = rotl(((x ^ v) * K[1]) & M, 17)
    for l, v in enumerate(h):
        x = rotl(((x ^ v) * K[l]) & M, 23)
    return x ^ (x >> 29)


def hash_ids(ids):
    """`generated_hash` of the reference's bench (sha_ids, crates/oxe-cli/src/bin/oxe.rs:417-419):
    hash_bytes of the ids as little-endian u32, as 16 hex digits."""
    b = b"".join(int(v).to_bytes(4, "little") for v in ids)
    return f"{hash_bytes(b):016x}"


def exported_symbols():
    """Names the header declares and the library must export."""
    hdr = os.path.join(HERE, "..", "include", "oxe_amd.h")
    names = []
    with open(hdr) as f:
        for line in f:
            line = line.strip()
            if line.startswith("OXE_API"):
                name = line.split("(")[0].split()[-1].lstrip("*")
                names.append(name)
    return names


def _p(t):
    return C.c_void_p(t.data_ptr()) if t is not None else None


def _stream():
    import torch
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def check(rc, what):
    if rc != 0:
        msg = _last_error()
        raise RuntimeError(f"{what} failed with status {rc}" + (f": {msg}" if msg else ""))


# ---- kernel-level entry points (torch tensors on cuda)

def quantize_q8_0(x):
    """x: float32 [..., k] on the GPU -> (codes int8 [..., k], scales uint16 [..., k/32])."""
    import torch
    x = x.contiguous()
    k = x.shape[-1]
    nrows = x.numel() // k
    q = torch.empty(x.shape, dtype=torch.int8, device=x.device)
    d = torch.empty(x.shape[:-1] + (k // 32,), dtype=torch.int16, device=x.device)
    check(lib().oxe_hip_quantize_row_q8_0(_p(x), k, nrows, _p(q), _p(d), _stream()), "quantize_q8_0")
    return q, d


def gemv_q8_0(wq, wd, xq, xd, y=None, isum=None):
    """y[l, r] = Q8_0 GEMV of lanes l (1..4) over rows r; optional int32 block sums [nl, nr, k/32]."""
    import torch
    nr, k = wq.shape
    nl = xq.shape[0]
    if y is None:
        y = torch.empty((nl, nr), dtype=torch.float32, device=wq.device)
    rc = lib().oxe_hip_gemv_q8_0(k, nr, nl, _p(wq), _p(wd), _p(xq), _p(xd), _p(y), _p(isum), _stream())
    if rc != 1:   # oxe_vl_gemv's convention: 1 done, 0 not handled (nothing written)
        raise RuntimeError(f"gemv_q8_0 failed with status {rc}" + (": not handled" if rc == 0 else ""))
    return y


def gemm_q8_0(wq, wd, xq, xd, y=None):
    """y[t, r] = Q8_0 GEMM of token rows t (any count) over weight rows r (prefill; int8 MFMA)."""
    import torch
    nr, k = wq.shape
    nt = xq.shape[0]
    if y is None:
        y = torch.empty((nt, nr), dtype=torch.float32, device=wq.device)
    check(lib().oxe_hip_gemm_q8_0(k, nr, nt, _p(wq), _p(wd), _p(xq), _p(xd), _p(y), y.stride(0), _stream()), "gemm_q8_0")
    return y


def repack_q8_0(blocks, k):
    """ggml Q8_0 blocks (uint8 [nrows, k/32*34] on the GPU) -> (codes int8 [nrows, k], scales int16
    [nrows, k/32]) in this build's layout (oxe_hip_repack_q8_0)"""
    import torch
    nrows = blocks.shape[0]
    q = torch.empty((nrows, k), dtype=torch.int8, device=blocks.device)
    d = torch.empty((nrows, k // 32), dtype=torch.int16, device=blocks.device)
    check(lib().oxe_hip_repack_q8_0(_p(blocks), nrows, k, _p(q), _p(d), _stream()), "repack_q8_0")
    return q, d


def quantize_q8_K(x):
    """x: float32 [..., k] on the GPU (k a multiple of 256) -> ggml block_q8_K bytes, uint8
    [..., k/256 * 292] (quantize_row_q8_K)"""
    import torch
    x = x.contiguous()
    k = x.shape[-1]
    nrows = x.numel() // k
    y = torch.empty(x.shape[:-1] + (k // 256 * 292,), dtype=torch.uint8, device=x.device)
    check(lib().oxe_hip_quantize_row_q8_K(_p(x), k, nrows, _p(y), _stream()), "quantize_q8_K")
    return y


def vl_gemv(ty, w, k, y, s=None):
    """K-quant lane GEMV (oxe_vl_gemv): w uint8 [nr, k/256 * block bytes] (ggml blocks of type ty:
    3 Q3_K, 4 Q4_K, 5 Q5_K, 6 Q6_K), y uint8 [nl, k/256 * 292] (q8_K lanes) -> float32 [nl, nr];
    None when the type / shape is not handled (the reference's 0 return)"""
    import torch
    nr, nl = w.shape[0], y.shape[0]
    if s is None:
        s = torch.empty((nl, nr), dtype=torch.float32, device=w.device)
    rc = lib().oxe_hip_vl_gemv(ty, k, nr, nl, _p(w), _p(y), _p(s), _stream())
    if rc < 0:
        raise RuntimeError(f"vl_gemv failed with status {rc}")
    return s if rc == 1 else None


def route_f32(logits, tie_count=None):
    """Routing of rows of 256 router logits (float32 [n, 256] on the GPU): top-8 ids int32 [n, 8] and
    renormalised weights float32 [n, 8] (Engine::route; std::sort order on tied probabilities);
    tie_count (uint32 [1] on the GPU, optional) counts rows that took the sort path."""
    import torch
    logits = logits.contiguous()
    n = logits.shape[0]
    ids = torch.empty((n, 8), dtype=torch.int32, device=logits.device)
    w = torch.empty((n, 8), dtype=torch.float32, device=logits.device)
    if tie_count is None:
        tie_count = torch.zeros(1, dtype=torch.int32, device=logits.device)
    check(lib().oxe_hip_route_f32(_p(logits), n, _p(ids), _p(w), _p(tie_count), _stream()), "route_f32")
    return ids, w


def eval_unary(fn, start, n, stride, y):
    """y[i] = device scalar function fn at the float with bits start + i*stride (parity hook)."""
    check(lib().oxe_hip_eval_unary(fn, start, n, stride, _p(y), _stream()), "eval_unary")
    return y


# ---- engine level --------------------------------------------------------------------------

def _engine_sigs(L):
    vp, i64, i32, u32p, f32p = C.c_void_p, C.c_int64, C.c_int, C.POINTER(C.c_uint32), C.POINTER(C.c_float)
    sig = {
        "oxe_last_error": (C.c_char_p, []),
        "oxe_engine_create": (i32, [vp, C.c_uint64, i32, C.POINTER(C.c_void_p)]),
        "oxe_engine_create_on": (i32, [vp, C.c_uint64, i32, vp, C.POINTER(C.c_void_p)]),
        "oxe_engine_create_typed": (i32, [vp, C.c_uint64, i32, vp, C.POINTER(C.c_void_p)]),
        "oxe_engine_verify_probe": (i32, [vp, u32p, i32, i32, u32p, C.POINTER(C.c_float), C.POINTER(C.c_int)]),
        "oxe_engine_destroy": (None, [vp]),
        "oxe_engine_synth_weights": (i32, [vp]),
        "oxe_engine_verify": (i32, [vp, u32p, i32, u32p]),
        "oxe_engine_commit": (i32, [vp, i32]),
        "oxe_engine_step": (i32, [vp, C.c_uint32, u32p]),
        "oxe_engine_mtp_run": (i32, [vp, u32p, i32, i32, f32p, i32, u32p]),
        "oxe_engine_mtp_seed": (i32, [vp, u32p, i32, i32, f32p]),
        "oxe_engine_pos": (i32, [vp]),
        "oxe_engine_n_ctx": (i32, [vp]),
        "oxe_engine_hidden": (i32, [vp, i32, f32p]),
        "oxe_engine_logits": (i32, [vp, i32, f32p]),
        "oxe_engine_counter": (i32, [vp, i32, u32p]),
        "oxe_engine_state_copy": (i32, [vp, i32, i32, i64, vp, i64]),
        "oxe_engine_set_pos": (i32, [vp, i32]),
        "oxe_engine_set_router": (i32, [vp, i32, i32, i32, f32p]),
        "oxe_engine_device_bytes": (i64, [vp]),
        "oxe_engine_state_bytes": (i64, [vp]),
        "oxe_engine_write_state": (i32, [vp, vp, i64]),
        "oxe_engine_read_state": (i32, [vp, vp, i64, i32]),
        "oxe_mtp_prefill": (i32, [vp, u32p, i32, u32p]),
        "oxe_mtp_prefill_batched": (i32, [vp, u32p, i32, u32p]),
        "oxe_engine_prefill": (i32, [vp, u32p, i32, u32p, f32p]),
        "oxe_engine_prefill_probe": (i32, [vp, u32p, i32, i32, C.POINTER(C.c_float), C.POINTER(C.c_int)]),
        "oxe_mtp_step": (i32, [vp, C.c_uint32, u32p, C.POINTER(C.c_int), i64]),
        "oxe_mtp_step_plain": (i32, [vp, C.c_uint32, u32p]),
        "oxe_engine_set_fused": (i32, [vp, i32]),
        "oxe_engine_fused": (i32, [vp]),
        "oxe_engine_set_trace": (i32, [vp, i32]),
        "oxe_engine_read_trace": (i64, [vp, vp, i64]),
        "oxe_mtp_rewind": (i32, [vp, i32]),
        "oxe_mtp_device_begin": (i32, [vp, C.c_uint32, i32]),
        "oxe_mtp_device_steps": (i32, [vp, i32, i32]),
        "oxe_mtp_device_end": (i32, [vp, u32p, i32, C.POINTER(C.c_int), u32p]),
        "oxe_mtp_set_force": (i32, [vp, C.POINTER(C.c_int32), i32]),
        "oxe_mtp_set_draft_vocab": (i32, [vp, C.POINTER(C.c_uint32), i32]),
        "oxe_mtp_stats": (i32, [vp, C.POINTER(C.c_int64)]),
        "oxe_mtp_step_force": (i32, [vp, C.c_uint32, u32p, C.POINTER(C.c_int), C.POINTER(C.c_int64), i32]),
        "oxe_mtp_set_depth": (i32, [vp, i32]),
        "oxe_srv_spec_set_depth": (i32, [vp, i32]),
        "oxe_engine_sync": (i32, [vp]),
        "oxe_mtp_device_probe": (i32, [vp, i32, i32, C.POINTER(C.c_float), C.POINTER(C.c_int)]),
        "oxe_engine_stream": (vp, [vp]),
        "oxe_gguf_open": (i32, [C.c_char_p, C.POINTER(C.c_void_p)]),
        "oxe_gguf_parse": (i32, [vp, C.c_uint64, C.POINTER(C.c_void_p)]),
        "oxe_gguf_check_bounds": (i32, [vp, C.c_uint64]),
        "oxe_gguf_close": (None, [vp]),
        "oxe_gguf_info": (i32, [vp, C.POINTER(C.c_uint32)] + [C.POINTER(C.c_uint64)] * 5),
        "oxe_gguf_tensor": (i32, [vp, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32),
                                  C.POINTER(C.c_uint32), C.POINTER(C.c_uint64), C.POINTER(C.c_uint64),
                                  C.POINTER(C.c_uint64)]),
        "oxe_gguf_meta": (i32, [vp, C.c_uint64, C.POINTER(C.c_char_p), C.POINTER(C.c_uint32)]),
        "oxe_gguf_meta_u64": (i32, [vp, C.c_char_p, C.POINTER(C.c_uint64)]),
        "oxe_gguf_meta_f64": (i32, [vp, C.c_char_p, C.POINTER(C.c_double)]),
        "oxe_gguf_meta_str": (i32, [vp, C.c_char_p, C.POINTER(C.c_char_p)]),
        "oxe_gguf_meta_array": (i32, [vp, C.c_char_p, C.POINTER(C.c_uint32), C.POINTER(C.c_uint64),
                                      C.POINTER(C.c_int)]),
        "oxe_gguf_meta_array_f64": (i32, [vp, C.c_char_p, C.c_uint64, C.POINTER(C.c_double)]),
        "oxe_gguf_model_desc": (i32, [vp, vp]),
        "oxe_engine_load_gguf": (i32, [vp, vp]),
        "oxe_engine_load_gguf_noalloc": (i32, [vp, vp]),
        "oxe_engine_create_from_gguf": (i32, [C.c_char_p, i32, C.POINTER(C.c_void_p)]),
        "oxe_engine_kv_row_bytes": (i64, [vp]),
        "oxe_engine_write_kv_rows": (i32, [vp, i32, i32, vp, i64]),
        "oxe_engine_read_kv_rows": (i32, [vp, i32, i32, vp, i64]),
        "oxe_srv_create": (i32, [vp, i32, C.POINTER(C.c_void_p)]),
        "oxe_srv_destroy": (None, [vp]),
        "oxe_srv_engine": (vp, [vp]),
        "oxe_srv_n_ctx": (i32, [vp]),
        "oxe_srv_n_vocab": (i32, [vp]),
        "oxe_srv_n_past": (i32, [vp]),
        "oxe_srv_reset": (i32, [vp]),
        "oxe_srv_prefill": (i32, [vp, u32p, i32, f32p]),
        "oxe_srv_decode": (i32, [vp, C.c_uint32, f32p]),
        "oxe_srv_decode_argmax": (i32, [vp, C.c_uint32, u32p]),
        "oxe_srv_decode_spec_argmax": (i32, [vp, C.c_uint32, u32p, C.POINTER(C.c_int), u32p, C.POINTER(C.c_int)]),
        "oxe_srv_decode_spec": (i32, [vp, C.c_uint32, u32p, C.POINTER(C.c_int), f32p, i32]),
        "oxe_srv_spec_rewind": (i32, [vp, i32]),
        "oxe_srv_decode_verify": (i32, [vp, C.c_uint32, u32p, i32, u32p, C.POINTER(C.c_int), u32p,
                                        C.POINTER(C.c_int)]),
        "oxe_srv_spec_max_depth": (i32, [vp]),
        "oxe_srv_spec_counters": (i32, [vp, C.POINTER(C.c_uint64), C.POINTER(C.c_uint64)]),
        "oxe_srv_snapshot": (i32, [vp, C.POINTER(C.c_void_p)]),
        "oxe_srv_restore": (i32, [vp, vp]),
        "oxe_snapshot_bytes": (i64, [vp]),
        "oxe_snapshot_pos": (i32, [vp]),
        "oxe_snapshot_free": (None, [vp]),
        "oxe_srv_state_size_hint": (i64, [vp]),
        "oxe_srv_save_bytes": (i64, [vp]),
        "oxe_srv_save_state": (i32, [vp, vp, i64, C.POINTER(C.c_int64)]),
        "oxe_srv_load_state": (i32, [vp, vp, i64, i32]),
        "oxe_srv_snap_file_bytes": (i64, [vp, vp]),
        "oxe_srv_snap_save": (i32, [vp, vp, vp, i64, C.POINTER(C.c_int64)]),
        "oxe_srv_snap_live_bytes": (i64, [vp]),
        "oxe_srv_snap_save_live": (i32, [vp, vp, i64, C.POINTER(C.c_int64)]),
        "oxe_srv_snap_load": (i32, [vp, vp, i64, i32]),
        "oxe_srv_state_layout": (i32, [vp, C.c_char_p, i32]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(L, name)
        fn.restype = res
        fn.argtypes = args


def _np_ptr(a, ct):
    return a.ctypes.data_as(C.POINTER(ct))


def _sigs():
    L = lib()
    if not hasattr(L, "_engine_sigs"):
        _engine_sigs(L)
        L._engine_sigs = True
    return L


def _last_error():
    e = _sigs().oxe_last_error()
    return e.decode(errors="replace") if e else ""


class GgufError(RuntimeError):
    pass


class Gguf:
    """A parsed GGUF file (crates/gguf Gguf / Header): metadata and tensor table; the payload is
    read only by the weight loader."""

    def __init__(self, path=None, data=None):
        L = _sigs()
        h = C.c_void_p()
        if data is not None:
            self._buf = bytes(data)
            rc = L.oxe_gguf_parse(self._buf, len(self._buf), C.byref(h))
        else:
            rc = L.oxe_gguf_open(os.fsencode(path), C.byref(h))
        if rc != 0:
            raise GgufError(_last_error())
        self.h = h

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.oxe_gguf_close(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def check_bounds(self, file_bytes):
        if lib().oxe_gguf_check_bounds(self.h, file_bytes) != 0:
            raise GgufError(_last_error())

    def info(self):
        v = C.c_uint32()
        n = [C.c_uint64() for _ in range(5)]
        check(lib().oxe_gguf_info(self.h, C.byref(v), *[C.byref(x) for x in n]), "gguf_info")
        keys = ("n_tensors", "n_meta", "data_offset", "header_bytes", "file_bytes")
        return dict(version=v.value, **{k: x.value for k, x in zip(keys, n)})

    def tensors(self):
        """[(name, ggml type id, shape, offset, bytes)] in file order"""
        out = []
        for i in range(self.info()["n_tensors"]):
            name, ty, nd = C.c_char_p(), C.c_uint32(), C.c_uint32()
            shape, off, nb = (C.c_uint64 * 4)(), C.c_uint64(), C.c_uint64()
            check(lib().oxe_gguf_tensor(self.h, i, C.byref(name), C.byref(ty), C.byref(nd), shape, C.byref(off),
                                        C.byref(nb)), "gguf_tensor")
            out.append((name.value.decode(), ty.value, list(shape[: nd.value]), off.value, nb.value))
        return out

    def meta_keys(self):
        out = []
        for i in range(self.info()["n_meta"]):
            k, t = C.c_char_p(), C.c_uint32()
            check(lib().oxe_gguf_meta(self.h, i, C.byref(k), C.byref(t)), "gguf_meta")
            out.append((k.value.decode(), t.value))
        return out

    def u64(self, key):
        v = C.c_uint64()
        return v.value if lib().oxe_gguf_meta_u64(self.h, key.encode(), C.byref(v)) == 0 else None

    def f64(self, key):
        v = C.c_double()
        return v.value if lib().oxe_gguf_meta_f64(self.h, key.encode(), C.byref(v)) == 0 else None

    def str(self, key):
        v = C.c_char_p()
        return v.value.decode() if lib().oxe_gguf_meta_str(self.h, key.encode(), C.byref(v)) == 0 else None

    def array(self, key):
        """(item type, length, items as floats or None when only counted)"""
        it, n, kept = C.c_uint32(), C.c_uint64(), C.c_int()
        if lib().oxe_gguf_meta_array(self.h, key.encode(), C.byref(it), C.byref(n), C.byref(kept)) != 0:
            return None
        items = None
        if kept.value:
            items = []
            for i in range(n.value):
                x = C.c_double()
                items.append(x.value if lib().oxe_gguf_meta_array_f64(self.h, key.encode(), i, C.byref(x)) == 0
                             else None)
        return it.value, n.value, items

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def model_desc(self):
        d = ModelDesc()
        if lib().oxe_gguf_model_desc(self.h, C.byref(d)) != 0:
            raise GgufError(_last_error())
        return d


# GGUF tensor name (after "blk.N." for layer tensors) -> tensor kind (include/oxe_model.h) of every
# matrix whose type the engine takes from the file (the names the reference's model reader checks,
# crates/model/src/desc.rs:140-175)
_MATRIX_KIND = {"attn_qkv.weight": 2, "attn_gate.weight": 3, "ssm_beta.weight": 4, "ssm_alpha.weight": 5,
                "ssm_out.weight": 10, "attn_q.weight": 11, "attn_k.weight": 12, "attn_v.weight": 13,
                "attn_output.weight": 16, "ffn_gate_exps.weight": 19, "ffn_up_exps.weight": 20,
                "ffn_down_exps.weight": 21, "ffn_gate_shexp.weight": 22, "ffn_up_shexp.weight": 23,
                "ffn_down_shexp.weight": 24, "nextn.eh_proj.weight": 25}
_GLOBAL_KIND = {"token_embd.weight": 29, "output.weight": 31}
_TYPE_ID = {"F32": 0, "Q8_0": 8, "Q3_K": 11, "Q4_K": 12, "Q5_K": 13, "Q6_K": 14}


def types_from_tensors(tensors):
    """{(layer, kind): ggml type id} of the matrices that are not Q8_0 in a GGUF tensor table
    ((name, type name) pairs, e.g. oxe_gguf's listing), the `types` argument of Engine: an engine
    with a model file's matrix types and synthetic weights."""
    out = {}
    for name, tname in tensors:
        if name.startswith("blk."):
            layer, rest = name[4:].split(".", 1)
            key = (int(layer), _MATRIX_KIND.get(rest))
        else:
            key = (63, _GLOBAL_KIND.get(name))
        if key[1] is None:
            continue
        if tname not in _TYPE_ID:
            raise ValueError(f"{name}: type {tname} is not a matrix type of the engine")
        if _TYPE_ID[tname] != 8:
            out[key] = _TYPE_ID[tname]
    return out


class Engine:
    """MI355X engine through the C ABI (Engine::{verify, commit, step, mtp_run, mtp_seed})."""

    def __init__(self, desc, seed=0, n_ctx=1024, synth=True, stream=None, types=None):
        """stream: a caller's hipStream_t (an int, e.g. torch.cuda.Stream().cuda_stream) that every
        launch and copy of the engine then goes to (oxe_engine_create_on); None: the engine's own.
        types: {(layer, kind): ggml type id} of matrices that are not Q8_0 (layer GLOBAL_LAYER = 63:
        the global tensors), as a model file holds them (oxe_engine_create_typed); the synthetic
        weights then fill each in its type."""
        import numpy as np
        L = lib()
        if not hasattr(L, "_engine_sigs"):
            _engine_sigs(L)
            L._engine_sigs = True
        self.desc = desc
        h = C.c_void_p()
        if types:
            tt = np.full(64 * 64, 8, np.int32)
            for (layer, kind), ty in types.items():
                tt[layer * 64 + kind] = ty
            rc = L.oxe_engine_create_typed(C.byref(desc), seed, n_ctx, tt.ctypes.data_as(C.c_void_p), C.byref(h))
        elif stream is None:
            rc = L.oxe_engine_create(C.byref(desc), seed, n_ctx, C.byref(h))
        else:
            rc = L.oxe_engine_create_on(C.byref(desc), seed, n_ctx, C.c_void_p(int(stream)), C.byref(h))
        if rc != 0:
            raise RuntimeError(f"oxe_engine_create: {rc} {L.oxe_last_error()}")
        self.h = h
        self.n_ctx = L.oxe_engine_n_ctx(h)
        if synth:
            check(L.oxe_engine_synth_weights(h), "synth_weights")

    @classmethod
    def from_gguf(cls, path, n_ctx=1024):
        """An engine with every weight from a GGUF file (oxe_engine_create_from_gguf)."""
        L = _sigs()
        h = C.c_void_p()
        rc = L.oxe_engine_create_from_gguf(os.fsencode(path), n_ctx, C.byref(h))
        if rc != 0:
            raise GgufError(f"oxe_engine_create_from_gguf: {rc} {_last_error()}")
        e = cls.__new__(cls)
        e.h = h
        e.n_ctx = L.oxe_engine_n_ctx(h)
        with Gguf(path) as g:
            e.desc = g.model_desc()
        return e

    def load_gguf(self, g):
        rc = lib().oxe_engine_load_gguf(self.h, g.h)
        if rc != 0:
            raise GgufError(f"oxe_engine_load_gguf: {rc} {_last_error()}")

    def load_gguf_noalloc(self, g):
        """load_gguf staged through the library's static device array (no device allocation)"""
        rc = lib().oxe_engine_load_gguf_noalloc(self.h, g.h)
        if rc != 0:
            raise GgufError(f"oxe_engine_load_gguf_noalloc: {rc} {_last_error()}")

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.oxe_engine_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def verify(self, toks):
        import numpy as np
        t = np.ascontiguousarray(toks, np.uint32)
        out = np.zeros(8, np.uint32)
        check(lib().oxe_engine_verify(self.h, _np_ptr(t, C.c_uint32), len(t), _np_ptr(out, C.c_uint32)), "verify")
        return out[: len(t)].copy()

    def verify_probe(self, toks, kind):
        """verify(toks) with HIP events around each launch of kernel kind `kind`: (mean us, launches)"""
        import numpy as np
        t = np.ascontiguousarray(toks, np.uint32)
        out = np.zeros(8, np.uint32)
        us, n = C.c_float(0.0), C.c_int(0)
        check(lib().oxe_engine_verify_probe(self.h, _np_ptr(t, C.c_uint32), len(t), kind, _np_ptr(out, C.c_uint32),
                                             C.byref(us), C.byref(n)), "verify_probe")
        return float(us.value), int(n.value)

    def commit(self, m):
        check(lib().oxe_engine_commit(self.h, m), "commit")

    def step(self, tok):
        import numpy as np
        out = np.zeros(1, np.uint32)
        check(lib().oxe_engine_step(self.h, tok, _np_ptr(out, C.c_uint32)), "step")
        return int(out[0])

    def mtp_run(self, toks, pos0, hs, head_last=True):
        import numpy as np
        t = np.ascontiguousarray(toks, np.uint32)
        h = np.ascontiguousarray(hs, np.float32)
        out = np.zeros(1, np.uint32)
        check(lib().oxe_engine_mtp_run(self.h, _np_ptr(t, C.c_uint32), len(t), pos0, _np_ptr(h, C.c_float),
                                       int(head_last), _np_ptr(out, C.c_uint32)), "mtp_run")
        return int(out[0])

    def mtp_seed(self, toks, pos0, hs):
        import numpy as np
        t = np.ascontiguousarray(toks, np.uint32)
        h = np.ascontiguousarray(hs, np.float32)
        check(lib().oxe_engine_mtp_seed(self.h, _np_ptr(t, C.c_uint32), len(t), pos0, _np_ptr(h, C.c_float)), "mtp_seed")

    @property
    def pos(self):
        return int(lib().oxe_engine_pos(self.h))

    def hidden(self, lane):
        import numpy as np
        out = np.empty(self.desc.n_embd, np.float32)
        check(lib().oxe_engine_hidden(self.h, lane, _np_ptr(out, C.c_float)), "hidden")
        return out

    def logits(self, lane):
        import numpy as np
        out = np.empty(self.desc.n_vocab, np.float32)
        check(lib().oxe_engine_logits(self.h, lane, _np_ptr(out, C.c_float)), "logits")
        return out

    def counter(self, which):
        import numpy as np
        out = np.zeros(1, np.uint32)
        check(lib().oxe_engine_counter(self.h, which, _np_ptr(out, C.c_uint32)), "counter")
        return int(out[0])

    def state(self, which, nbytes, offset=0, dtype=None):
        import numpy as np
        buf = np.empty(nbytes, np.uint8)
        check(lib().oxe_engine_state_copy(self.h, which, 0, offset, buf.ctypes.data_as(C.c_void_p), nbytes), "state_copy")
        return buf.view(dtype) if dtype is not None else buf

    def set_state(self, which, arr, offset=0):
        import numpy as np
        a = np.ascontiguousarray(arr)
        check(lib().oxe_engine_state_copy(self.h, which, 1, offset, a.ctypes.data_as(C.c_void_p), a.nbytes), "state_copy")

    def set_pos(self, pos):
        check(lib().oxe_engine_set_pos(self.h, pos), "set_pos")

    def set_router(self, layer, row0, rows):
        """Overwrite router rows [row0, row0 + len(rows)) of `layer` (test hook for routing ties)."""
        import numpy as np
        r = np.ascontiguousarray(rows, np.float32)
        check(lib().oxe_engine_set_router(self.h, layer, row0, r.shape[0], r.ctypes.data_as(C.POINTER(C.c_float))),
              "set_router")

    def write_state(self):
        """Engine::write_state bytes (reference order) as a numpy uint8 array."""
        import numpy as np
        n = int(lib().oxe_engine_state_bytes(self.h))
        buf = np.empty(n, np.uint8)
        check(lib().oxe_engine_write_state(self.h, buf.ctypes.data_as(C.c_void_p), n), "write_state")
        return buf

    def read_state(self, buf, n_pos):
        """Engine::read_state of write_state bytes for n_pos positions."""
        import numpy as np
        b = np.ascontiguousarray(buf, np.uint8)
        check(lib().oxe_engine_read_state(self.h, b.ctypes.data_as(C.c_void_p), b.nbytes, n_pos), "read_state")

    def kv_row_bytes(self):
        return int(lib().oxe_engine_kv_row_bytes(self.h))

    def write_kv_rows(self, a, b):
        """Engine::write_kv_rows: K and V^T rows of positions [a, b) as a numpy uint8 array."""
        import numpy as np
        buf = np.empty(self.kv_row_bytes() * (b - a), np.uint8)
        rc = lib().oxe_engine_write_kv_rows(self.h, a, b, buf.ctypes.data_as(C.c_void_p), buf.nbytes)
        if rc != 0:
            raise EngineError(f"save kv rows: {_last_error() or rc}")
        return buf

    def read_kv_rows(self, a, b, buf):
        import numpy as np
        x = np.ascontiguousarray(buf, np.uint8)
        rc = lib().oxe_engine_read_kv_rows(self.h, a, b, x.ctypes.data_as(C.c_void_p), x.nbytes)
        if rc != 0:
            raise EngineError(f"load kv rows: {_last_error() or rc}")

    def prefill(self, toks, hidden=False):
        """Batched prefill (Engine::prefill_ext, prefill.rs:763): argmax after the last token, and
        with hidden=True also every position's h_nextn [n][n_embd]."""
        import numpy as np
        t = np.ascontiguousarray(toks, np.uint32)
        nx = np.zeros(1, np.uint32)
        h = np.empty((len(t), self.desc.n_embd), np.float32) if hidden else None
        hp = _np_ptr(h, C.c_float) if hidden else None
        check(lib().oxe_engine_prefill(self.h, _np_ptr(t, C.c_uint32), len(t), _np_ptr(nx, C.c_uint32), hp), "prefill")
        return (int(nx[0]), h) if hidden else int(nx[0])

    def prefill_probe(self, toks, kind):
        """A prefill with HIP events around every launch of one kernel kind (12 every GEMM, 13 grouped
        expert GEMMs, 14 attention, 15 delta rule): (summed microseconds, launches)."""
        import numpy as np
        t = np.ascontiguousarray(toks, np.uint32)
        us, n = C.c_float(0), C.c_int(0)
        check(lib().oxe_engine_prefill_probe(self.h, _np_ptr(t, C.c_uint32), len(t), kind, C.byref(us), C.byref(n)),
              "prefill_probe")
        return float(us.value), int(n.value)

    # ---- MTP depth-1 driver (mtp.rs MtpDriver) ----
    def mtp_prefill_batched(self, toks):
        """MtpDriver::prefill_batched (mtp.rs:468-500)."""
        import numpy as np
        t = np.ascontiguousarray(toks, np.uint32)
        nx = np.zeros(1, np.uint32)
        check(lib().oxe_mtp_prefill_batched(self.h, _np_ptr(t, C.c_uint32), len(t), _np_ptr(nx, C.c_uint32)),
              "mtp_prefill_batched")
        return int(nx[0])

    def mtp_prefill(self, toks):
        import numpy as np
        t = np.ascontiguousarray(toks, np.uint32)
        nx = np.zeros(1, np.uint32)
        check(lib().oxe_mtp_prefill(self.h, _np_ptr(t, C.c_uint32), len(t), _np_ptr(nx, C.c_uint32)), "mtp_prefill")
        return int(nx[0])

    def mtp_step(self, x, override_d1=-1):
        import numpy as np
        out = np.zeros(8, np.uint32)
        n = C.c_int(0)
        check(lib().oxe_mtp_step(self.h, x, _np_ptr(out, C.c_uint32), C.byref(n), override_d1), "mtp_step")
        return [int(v) for v in out[: n.value]]

    def set_fused(self, on):
        """1: each run is one persistent fused launch; 0: one launch per phase (same bits)."""
        check(lib().oxe_engine_set_fused(self.h, int(on)), "set_fused")

    @property
    def fused(self):
        return bool(lib().oxe_engine_fused(self.h))

    def set_trace(self, on):
        check(lib().oxe_engine_set_trace(self.h, int(on)), "set_trace")

    def read_trace(self):
        """Last fused run's phase records: array [grid, 2048, 4] (phase id, start, passed, end), 100 MHz ticks."""
        import numpy as np
        buf = np.zeros(256 * 2048 * 4, np.uint64)
        n = lib().oxe_engine_read_trace(self.h, buf.ctypes.data_as(C.c_void_p), buf.size)
        if n < 0:
            raise RuntimeError("read_trace failed")
        return buf[:n].reshape(-1, 2048, 4)

    def mtp_set_depth(self, depth):
        """drafts per MTP step (MtpDriver.depth): host-driven steps 1..3, device-driven steps 1 or 2"""
        check(lib().oxe_mtp_set_depth(self.h, depth), "mtp_set_depth")

    def mtp_step_force(self, x, force):
        """one host-driven MTP step with force[i] >= 0 replacing draft i + 1 (draft_override)"""
        import numpy as np
        f = np.ascontiguousarray(force, np.int64)
        out = np.zeros(8, np.uint32)
        n = C.c_int(0)
        check(lib().oxe_mtp_step_force(self.h, x, _np_ptr(out, C.c_uint32), C.byref(n), _np_ptr(f, C.c_int64), len(f)),
              "mtp_step_force")
        return [int(v) for v in out[: n.value]]

    def mtp_step_plain(self, x):
        out = (C.c_uint32 * 1)()
        check(lib().oxe_mtp_step_plain(self.h, x, out), "mtp_step_plain")
        return int(out[0])

    def mtp_rewind(self, m):
        check(lib().oxe_mtp_rewind(self.h, m), "mtp_rewind")

    def mtp_set_draft_vocab(self, ids):
        """restrict every MTP draft run's LM head to the output rows of `ids` (MtpWeights::set_draft_vocab);
        an empty list restores the whole head. Returns the draft head's rows."""
        import numpy as np
        v = np.ascontiguousarray(ids, np.uint32)
        rc = lib().oxe_mtp_set_draft_vocab(self.h, v.ctypes.data_as(C.POINTER(C.c_uint32)), len(v))
        if rc < 0:
            raise EngineError(f"mtp_set_draft_vocab: {_last_error() or rc}")
        return rc

    def mtp_set_force(self, force):
        import numpy as np
        f = np.ascontiguousarray(force, np.int32)
        check(lib().oxe_mtp_set_force(self.h, f.ctypes.data_as(C.POINTER(C.c_int32)), len(f)), "mtp_set_force")

    def mtp_device_begin(self, x, out_cap):
        check(lib().oxe_mtp_device_begin(self.h, x, out_cap), "mtp_device_begin")

    def mtp_device_steps(self, k, use_graph=True):
        check(lib().oxe_mtp_device_steps(self.h, k, int(use_graph)), "mtp_device_steps")

    def mtp_device_end(self, cap):
        import numpy as np
        out = np.zeros(cap, np.uint32)
        n = C.c_int(0)
        nx = np.zeros(1, np.uint32)
        check(lib().oxe_mtp_device_end(self.h, _np_ptr(out, C.c_uint32), cap, C.byref(n), _np_ptr(nx, C.c_uint32)),
              "mtp_device_end")
        return [int(v) for v in out[: n.value]], int(nx[0])

    def mtp_stats(self):
        import numpy as np
        s = np.zeros(3, np.int64)
        lib().oxe_mtp_stats(self.h, s.ctypes.data_as(C.POINTER(C.c_int64)))
        return dict(steps=int(s[0]), accepted=int(s[1]), drafted=int(s[2]))

    def mtp_device_probe(self, k, kind):
        avg = C.c_float(0)
        n = C.c_int(0)
        check(lib().oxe_mtp_device_probe(self.h, k, kind, C.byref(avg), C.byref(n)), "mtp_device_probe")
        return float(avg.value), int(n.value)

    def sync(self):
        check(lib().oxe_engine_sync(self.h), "sync")

    def stream(self):
        return lib().oxe_engine_stream(self.h)


class EngineError(RuntimeError):
    """The server engine's error (crates/server/src/engine.rs EngineError) with its message."""


class Snapshot:
    """OxeSnapshot: the recurrent state of the current slot (device copy), the position and the
    MTP driver's state."""

    def __init__(self, h):
        self.h = h

    @property
    def pos(self):
        return int(lib().oxe_snapshot_pos(self.h))

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.oxe_snapshot_free(self.h)
            self.h = None

    def __del__(self):
        self.close()


class ServerEngine:
    """The reference server's `Engine` trait for oxe (crates/server/src/engine.rs:28-190,
    OxeEngine in crates/server/src/oxe_engine.rs:317-634) over an Engine, with or without the MTP
    depth-1 driver: the same method names, argument meaning, return values (None where the trait
    returns Ok(None)) and error messages (EngineError)."""

    def __init__(self, engine, mtp=True):
        L = _sigs()
        self.engine = engine
        self.mtp = bool(mtp)
        h = C.c_void_p()
        check(L.oxe_srv_create(engine.h, int(self.mtp), C.byref(h)), "oxe_srv_create")
        self.h = h
        self.n_vocab = int(L.oxe_srv_n_vocab(h))

    def close(self):
        if getattr(self, "h", None) and _lib is not None:
            _lib.oxe_srv_destroy(self.h)
            self.h = None

    def __del__(self):
        self.close()

    def _rc(self, rc, what):
        if rc < 0:
            raise EngineError(_last_error() if rc == -1 and _last_error() else f"{what}: status {rc}")
        return rc

    def n_ctx(self):
        return int(lib().oxe_srv_n_ctx(self.h))

    def n_past(self):
        return int(lib().oxe_srv_n_past(self.h))

    def reset(self):
        self._rc(lib().oxe_srv_reset(self.h), "reset")

    def prefill(self, tokens):
        import numpy as np
        t = np.ascontiguousarray(tokens, np.uint32)
        out = np.empty(self.n_vocab, np.float32)
        self._rc(lib().oxe_srv_prefill(self.h, _np_ptr(t, C.c_uint32), len(t), _np_ptr(out, C.c_float)), "prefill")
        return out

    def prefill_quiet(self, tokens):
        import numpy as np
        t = np.ascontiguousarray(tokens, np.uint32)
        self._rc(lib().oxe_srv_prefill(self.h, _np_ptr(t, C.c_uint32), len(t), None), "prefill")

    def decode(self, token):
        import numpy as np
        out = np.empty(self.n_vocab, np.float32)
        self._rc(lib().oxe_srv_decode(self.h, token, _np_ptr(out, C.c_float)), "decode")
        return out

    def decode_argmax(self, token):
        import numpy as np
        out = np.zeros(1, np.uint32)
        self._rc(lib().oxe_srv_decode_argmax(self.h, token, _np_ptr(out, C.c_uint32)), "decode_argmax")
        return int(out[0])

    def decode_spec_argmax(self, token):
        import numpy as np
        ex, g = np.zeros(8, np.uint32), np.zeros(8, np.uint32)
        ne, ng = C.c_int(0), C.c_int(0)
        rc = self._rc(lib().oxe_srv_decode_spec_argmax(self.h, token, _np_ptr(ex, C.c_uint32), C.byref(ne),
                                                        _np_ptr(g, C.c_uint32), C.byref(ng)), "decode_spec_argmax")
        if rc == 1:
            return None
        return [int(v) for v in ex[: ne.value]], [int(v) for v in g[: ng.value]]

    def decode_spec(self, token):
        import numpy as np
        ex = np.zeros(8, np.uint32)
        ne = C.c_int(0)
        rows = np.empty((8, self.n_vocab), np.float32)
        rc = self._rc(lib().oxe_srv_decode_spec(self.h, token, _np_ptr(ex, C.c_uint32), C.byref(ne),
                                                 _np_ptr(rows, C.c_float), rows.shape[0]), "decode_spec")
        if rc == 1:
            return None
        return [int(v) for v in ex[: ne.value]], [rows[i].copy() for i in range(ne.value + 1)]

    def spec_rewind(self, keep):
        self._rc(lib().oxe_srv_spec_rewind(self.h, keep), "spec_rewind")

    def decode_verify(self, token, drafts):
        import numpy as np
        d = np.ascontiguousarray(drafts, np.uint32)
        acc, g = np.zeros(8, np.uint32), np.zeros(8, np.uint32)
        na, ng = C.c_int(0), C.c_int(0)
        rc = self._rc(lib().oxe_srv_decode_verify(self.h, token, _np_ptr(d, C.c_uint32), len(d), _np_ptr(acc, C.c_uint32),
                                                   C.byref(na), _np_ptr(g, C.c_uint32), C.byref(ng)), "decode_verify")
        if rc == 1:
            return None
        return [int(v) for v in acc[: na.value]], [int(v) for v in g[: ng.value]]

    def spec_max_depth(self):
        return int(lib().oxe_srv_spec_max_depth(self.h))

    def spec_set_depth(self, depth):
        lib().oxe_srv_spec_set_depth(self.h, depth)

    def spec_counters(self):
        a, b = C.c_uint64(0), C.c_uint64(0)
        self._rc(lib().oxe_srv_spec_counters(self.h, C.byref(a), C.byref(b)), "spec_counters")
        return int(a.value), int(b.value)

    def snapshot(self):
        h = C.c_void_p()
        self._rc(lib().oxe_srv_snapshot(self.h, C.byref(h)), "snapshot")
        return Snapshot(h)

    def snapshot_reuse(self, old):
        h = C.c_void_p(old.h.value if isinstance(old.h, C.c_void_p) else old.h)
        self._rc(lib().oxe_srv_snapshot(self.h, C.byref(h)), "snapshot")
        old.h = None
        return Snapshot(h)

    def restore(self, snap):
        self._rc(lib().oxe_srv_restore(self.h, snap.h), "restore")

    @staticmethod
    def snapshot_bytes(snap):
        return int(lib().oxe_snapshot_bytes(snap.h))

    def state_size_hint(self):
        return int(lib().oxe_srv_state_size_hint(self.h))

    def state_id(self):
        buf = C.create_string_buffer(256)
        self._rc(lib().oxe_srv_state_layout(self.h, buf, 256), "state_layout")
        return f"oxe-state-v1 {buf.value.decode()} mtp={'true' if self.mtp else 'false'}"

    def save_state_vec(self):
        import numpy as np
        buf = np.empty(int(lib().oxe_srv_save_bytes(self.h)), np.uint8)
        w = C.c_int64(0)
        self._rc(lib().oxe_srv_save_state(self.h, buf.ctypes.data_as(C.c_void_p), buf.nbytes, C.byref(w)), "save_state")
        return buf[: w.value]

    def load_state(self, buf, n_pos):
        import numpy as np
        b = np.ascontiguousarray(buf, np.uint8)
        self._rc(lib().oxe_srv_load_state(self.h, b.ctypes.data_as(C.c_void_p), b.nbytes, n_pos), "load_state")

    def kv_row_bytes(self):
        return self.engine.kv_row_bytes()

    def kv_rows_save(self, a, b):
        return self.engine.write_kv_rows(a, b)

    def kv_rows_load(self, a, b, buf):
        self.engine.read_kv_rows(a, b, buf)

    def snap_save(self, snap):
        import numpy as np
        buf = np.empty(int(lib().oxe_srv_snap_file_bytes(self.h, snap.h)), np.uint8)
        w = C.c_int64(0)
        self._rc(lib().oxe_srv_snap_save(self.h, snap.h, buf.ctypes.data_as(C.c_void_p), buf.nbytes, C.byref(w)),
                 "snap_save")
        return buf[: w.value]

    def snap_save_live(self):
        import numpy as np
        buf = np.empty(int(lib().oxe_srv_snap_live_bytes(self.h)), np.uint8)
        w = C.c_int64(0)
        self._rc(lib().oxe_srv_snap_save_live(self.h, buf.ctypes.data_as(C.c_void_p), buf.nbytes, C.byref(w)),
                 "snap_save_live")
        return buf[: w.value]

    def snap_load(self, buf, n_pos):
        import numpy as np
        b = np.ascontiguousarray(buf, np.uint8)
        self._rc(lib().oxe_srv_snap_load(self.h, b.ctypes.data_as(C.c_void_p), b.nbytes, n_pos), "snap_load")
