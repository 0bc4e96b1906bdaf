"""The device's restatement of libstdc++'s std::sort (snapdragon-engine_amd/csrc/oxe_stdsort.h)
against this host's std::sort with the reference's top-k comparator x[a] > x[b]
(crates/kernels-sys/csrc/oxe_ops.cpp:157-164), on seeded rows full of ties (1, 2, 7, 40 levels,
all distinct; ascending and descending runs; 2 to 2048 elements). Unstable sorts differ exactly in
the order they leave equal elements in, so only identical permutations pass.
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "..", "snapdragon-engine_amd", "csrc")


def test_stdsort_restatement_equals_libstdcxx(tmp_path):
    exe = str(tmp_path / "stdsort_check")
    subprocess.check_call(["g++", "-O2", "-std=c++17", "-I", CSRC, os.path.join(HERE, "stdsort_check.cpp"), "-o", exe])
    bad, first = subprocess.check_output([exe, "6000", "1"], text=True, timeout=300).split()
    assert int(bad) == 0, f"first mismatching row {first}"
