"""Builds libcohx.so (HIP kernels + C ABI) for gfx950, in-tree.

Flags that carry the engine's float semantics:
  -ffp-contract=off                    no a*b+c fusion except explicit fmaf
  -fno-gpu-flush-denormals-to-zero     IEEE subnormals, as on the CPU
  -fhip-fp32-correctly-rounded-divide-sqrt   IEEE division / sqrt
Packed fp32 instructions are disabled (-packed-fp32-ops).
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libcohx.so")
SOURCES = ["csrc/kernels.hip", "csrc/cohx.cpp", "csrc/gen.cpp", "csrc/q35_kernels.hip", "csrc/q35.cpp",
           "csrc/gguf.cpp", "csrc/blas.cpp"]
HEADERS = ["csrc/device.h", "csrc/kernels.h", "csrc/internal.h", "../include/cohx.h"]
PROBE_SOURCE = "csrc/probe.hip"
PROBE_LIB = os.path.join(HERE, "libcohx_probe.so")
ARCH = os.environ.get("COHX_ARCH", "gfx950")

FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-fhip-fp32-correctly-rounded-divide-sqrt",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # matrix-core results straight into VGPRs (no AGPR copies before the VALU chain)
    "-mllvm", "-amdgpu-mfma-vgpr-form",
    "-Wall", "-Wno-unused-function", "-I", os.path.join(ROOT, "include"),
]


def _hipcc():
    for p in ("/opt/rocm/bin/hipcc", "hipcc"):
        if os.path.sep not in p or os.path.exists(p):
            return p
    return "hipcc"


def build(verbose=False):
    os.makedirs(os.path.join(HERE, "_build"), exist_ok=True)
    hipcc = _hipcc()

    def compile_one(src):
        obj = os.path.join(HERE, "_build", os.path.basename(src) + ".o")
        cmd = [hipcc, *FLAGS, "-x", "hip", "-c", os.path.join(HERE, src), "-o", obj]
        r = subprocess.run(cmd, capture_output=True, text=True)
        out = (r.stdout + r.stderr).splitlines()
        out = [l for l in out if "packed-fp32-ops" not in l]
        if r.returncode != 0 or verbose:
            sys.stderr.write("\n".join(out) + "\n")
        if r.returncode != 0:
            raise RuntimeError(f"hipcc failed on {src}")
        return obj

    with ThreadPoolExecutor(max_workers=len(SOURCES) + 1) as ex:
        objs = list(ex.map(compile_one, SOURCES + [PROBE_SOURCE]))
    probe_obj = objs.pop()
    tmp = LIB + ".tmp"
    # -z defs: an undefined symbol (say, a kernel stub the host pass dropped) fails the build
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp, *objs,
           "-L/opt/rocm/lib", "-lhipblaslt", "-Wl,-rpath,/opt/rocm/lib"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link failed")
    os.replace(tmp, LIB)
    # the instruction-rate probes of bench.py --valu-probe, a library of their own
    tmp = PROBE_LIB + ".tmp"
    r = subprocess.run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", "-Wl,-z,defs", "-o", tmp, probe_obj],
                       capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("probe link failed")
    os.replace(tmp, PROBE_LIB)
    return LIB


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
