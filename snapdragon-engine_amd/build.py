"""Build liboxe_amd.so: every HIP/C++ source under csrc/ compiled for gfx950 with hipcc.

Flags that the parity contract depends on:
  -ffp-contract=off                           no implicit multiply-add fusion (every fma is explicit)
  -fhip-fp32-correctly-rounded-divide-sqrt    IEEE f32 division and sqrt (the reference's libm/CPU ones)
  -Xclang -target-feature -Xclang -packed-fp32-ops   no packed-f32 instructions (unreliable on this pool)
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
LIB = os.path.join(HERE, "liboxe_amd.so")
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("OXE_OFFLOAD_ARCH", "gfx950")

FLAGS = [
    f"--offload-arch={ARCH}", "-O3", "-std=c++17", "-fPIC",
    "-ffp-contract=off", "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core results straight into VGPRs (no accumulation-register copies before the fp32 chain)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function", "-Wno-unused-variable",
    "-I", os.path.join(HERE, "..", "include"),
]


def sources():
    return sorted(os.path.join(CSRC, f) for f in os.listdir(CSRC) if f.endswith((".hip", ".cpp")))


def build(verbose=False, jobs=8):
    objdir = os.path.join(HERE, "_build")
    os.makedirs(objdir, exist_ok=True)
    srcs = sources()
    objs = []
    procs = []
    for s in srcs:
        o = os.path.join(objdir, os.path.basename(s) + ".o")
        objs.append(o)
        cmd = [HIPCC] + FLAGS + ["-c", s, "-o", o]
        if verbose:
            print(" ".join(cmd), flush=True)
        procs.append((s, subprocess.Popen(cmd, stderr=subprocess.PIPE, text=True)))
        if len(procs) >= jobs:
            _drain(procs)
    _drain(procs)
    tmp = LIB + ".tmp"
    subprocess.check_call([HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", tmp] + objs + ["-lpthread"])
    os.replace(tmp, LIB)
    return LIB


def _drain(procs):
    errs = []
    for s, p in procs:
        _, err = p.communicate()
        noise = [l for l in err.splitlines() if "packed-fp32-ops" not in l]
        if p.returncode != 0:
            errs.append(f"{s}:\n" + "\n".join(noise))
        elif noise:
            sys.stderr.write("\n".join(noise) + "\n")
    procs.clear()
    if errs:
        raise RuntimeError("hipcc failed:\n" + "\n".join(errs))


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
