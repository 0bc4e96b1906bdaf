"""The device's expf / log1pf restatements (snapdragon-engine_amd/csrc/oxe_libm.h) against this
host's C library, exhaustively over all 2^32 float inputs, bit for bit (NaNs of either sign match).

The reference calls the C library's expf (sigmoid, softplus, the delta rule's e^g; oxe_ops.cpp:80-89,
221) and log1pf (softplus). The GPU must produce the same bits as the host library the oracle links;
the same header is compiled unchanged for gfx950, and the GPU tests compare the two on the device.
"""
import os
import subprocess

import pytest

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "snapdragon-engine_amd", "csrc")


@pytest.fixture(scope="module")
def checker(tmp_path_factory):
    exe = str(tmp_path_factory.mktemp("libm") / "libm_check")
    subprocess.check_call(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-I", CSRC,
                           os.path.join(HERE, "libm_check.cpp"), "-o", exe, "-lm"])
    return exe


@pytest.mark.parametrize("fn", [0, 1], ids=["expf", "log1pf"])
def test_libm_exhaustive(checker, fn):
    nt = max(1, min(8, os.cpu_count() or 1))
    out = subprocess.check_output([checker, str(fn), "0", "100000000", str(nt)], text=True, timeout=600)
    bad, first = out.split()
    assert int(bad) == 0, f"first mismatching input bits 0x{first}"
