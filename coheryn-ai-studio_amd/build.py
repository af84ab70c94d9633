"""Builds libcohx.so (HIP kernels + C ABI) for gfx950, in-tree.

The flags (the engine's float semantics: no contraction, IEEE subnormals,
division and square root; packed fp32 instructions off), the sources and the
link line come from build.manifest, which the Rust crate's build.rs reads too.
"""
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB = os.path.join(HERE, "libcohx.so")
MANIFEST = os.path.join(HERE, "build.manifest")
HEADERS = ["csrc/device.h", "csrc/kernels.h", "csrc/internal.h", "../include/cohx.h"]
PROBE_SOURCE = "csrc/probe.hip"
PROBE_LIB = os.path.join(HERE, "libcohx_probe.so")
ARCH = os.environ.get("COHX_ARCH", "gfx950")


def manifest(path=MANIFEST):
    """The [flags], [sources] and [link] lists of build.manifest (shared with
    the Rust crate's build.rs)."""
    sections, current = {}, None
    with open(path) as f:
        for line in f:
            line = line.split("#", 1)[0].strip()
            if not line:
                continue
            if line.startswith("[") and line.endswith("]"):
                current = sections.setdefault(line[1:-1], [])
            elif current is not None:
                current.append(line)
    return sections


_M = manifest()
SOURCES = _M["sources"]
FLAGS = [*_M["flags"], f"--offload-arch={ARCH}", "-I", os.path.join(ROOT, "include")]
LINK = _M["link"]


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
           *LINK]
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
