"""The C-ABI library loads on the CPU host and exports every symbol include/oxe_amd.h declares."""
import ctypes
import os

import oxe_amd as A


def test_library_exports_header_symbols():
    assert os.path.exists(A.LIB_PATH), "build first: python snapdragon-engine_amd/build.py"
    lib = ctypes.CDLL(A.LIB_PATH)
    names = A.exported_symbols()
    assert len(names) >= 2
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_typed_engine_refuses_unsupported_type_mixes():
    """oxe_engine_create_typed checks the types before any device work: the combinations a model
    file's loader takes pass the check, any other returns -1 naming it"""
    import numpy as np
    import oracle as O
    lib = ctypes.CDLL(A.LIB_PATH)
    lib.oxe_engine_create_typed.restype = ctypes.c_int
    lib.oxe_engine_create_typed.argtypes = [ctypes.c_void_p, ctypes.c_uint64, ctypes.c_int, ctypes.c_void_p,
                                            ctypes.POINTER(ctypes.c_void_p)]
    lib.oxe_last_error.restype = ctypes.c_char_p
    d = O.desc_small()
    T = O.T
    cases = [
        ({(0, T["DN_QKV"]): 12}, "mix Q8_0"),                               # qkv K-quant, z Q8_0
        ({(3, T["ATT_Q"]): 12, (3, T["ATT_K"]): 12}, "mix Q8_0"),          # v left Q8_0
        ({(0, T["GATE_EXPS"]): 12}, "gate and up"),                         # up left Q8_0
        ({(0, T["ROUTER"]): 12}, "takes no other type"),
        ({(O.GLOBAL_LAYER, T["OUT_NORM"]): 14}, "takes no other type"),
        ({(4, T["EH_PROJ"]): 12}, "takes no other type"),
    ]
    for types, msg in cases:
        tt = np.full(64 * 64, 8, np.int32)
        for (layer, kind), ty in types.items():
            tt[layer * 64 + kind] = ty
        h = ctypes.c_void_p()
        rc = lib.oxe_engine_create_typed(ctypes.byref(d), 0, 256, tt.ctypes.data_as(ctypes.c_void_p), ctypes.byref(h))
        assert rc == -1, types
        assert msg in lib.oxe_last_error().decode(), (types, lib.oxe_last_error())
