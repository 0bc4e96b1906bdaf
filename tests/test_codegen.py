"""Code-generation guards on the built library's gfx950 device code (CPU only: the code objects
are read from liboxe_amd.so's offload bundles and disassembled with ROCm's llvm-objdump).

* No mixed-precision FMA (v_fma_mix*, v_mad_mix*): the compiler may fold an f32 multiply into the
  following f32 -> f16 conversion, rounding once instead of the reference's f32 rounding followed
  by the f16 conversion; f2h() pins the f32 value to prevent it.
* No packed fp32 arithmetic (the build disables it with -packed-fp32-ops)."""
import os
import shutil
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "snapdragon-engine_amd", "liboxe_amd.so")
LLVM = "/opt/rocm/llvm/bin"
MAGIC = b"__CLANG_OFFLOAD_BUNDLE__"


def device_disassembly(tmp_path):
    fat = tmp_path / "fatbin.bin"
    subprocess.check_call(["objcopy", "--dump-section", f".hip_fatbin={fat}", LIB, str(tmp_path / "lib.copy")])
    data = fat.read_bytes()
    offs = []
    i = data.find(MAGIC)
    while i >= 0:
        offs.append(i)
        i = data.find(MAGIC, i + 1)
    out = []
    for k, o in enumerate(offs):
        part = tmp_path / f"b{k}.bin"
        part.write_bytes(data[o:offs[k + 1] if k + 1 < len(offs) else len(data)])
        obj = tmp_path / f"b{k}.o"
        subprocess.check_call([f"{LLVM}/clang-offload-bundler", "--unbundle", "--type=o", f"--input={part}",
                               "--targets=hipv4-amdgcn-amd-amdhsa--gfx950", f"--output={obj}"])
        out.append(subprocess.run([f"{LLVM}/llvm-objdump", "-d", str(obj)], check=True, capture_output=True,
                                  text=True).stdout)
    return "\n".join(out)


@pytest.fixture(scope="module")
def disasm(tmp_path_factory):
    if not os.path.exists(LIB):
        pytest.skip("liboxe_amd.so is not built")
    if not (shutil.which("objcopy") and os.path.exists(f"{LLVM}/llvm-objdump")):
        pytest.skip("binutils / ROCm llvm tools not available")
    return device_disassembly(tmp_path_factory.mktemp("codegen"))


def offenders(text, needles):
    fn, hits = "?", []
    for line in text.splitlines():
        if line.endswith(">:"):
            fn = line.split("<", 1)[-1][:-2]
        elif any(n in line for n in needles):
            hits.append((fn, line.strip()))
    return hits


def test_device_code_present(disasm):
    assert "fused_kernel" in disasm and disasm.count("\n") > 10000


def test_no_mixed_precision_fma(disasm):
    hits = offenders(disasm, ("v_fma_mix", "v_mad_mix"))
    assert not hits, hits[:10]


def test_no_packed_fp32(disasm):
    hits = offenders(disasm, ("v_pk_fma_f32", "v_pk_mul_f32", "v_pk_add_f32"))
    assert not hits, hits[:10]
