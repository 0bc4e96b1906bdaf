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
