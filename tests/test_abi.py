"""CPU checks of the C ABI: the library loads and exports every entry point
include/cohx.h declares (no device calls)."""
import os
import re
import subprocess

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(ROOT, "coheryn-ai-studio_amd", "libcohx.so")
HEADER = os.path.join(ROOT, "include", "cohx.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(cohx_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_boundary():
    names = declared()
    for must in ("cohx_create", "cohx_upload_tensor", "cohx_seq_alloc", "cohx_seq_free",
                 "cohx_step", "cohx_destroy", "cohx_step_batch", "cohx_gen_sample",
                 "cohx_create_qwen35"):
        assert must in names


@pytest.mark.skipif(not os.path.exists(LIB), reason="libcohx.so not built")
def test_library_exports_every_declared_symbol():
    out = subprocess.run(["nm", "-D", "--defined-only", LIB], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [n for n in declared() if n not in exported]
    assert not missing, missing


@pytest.mark.skipif(not os.path.exists(LIB), reason="libcohx.so not built")
def test_library_loads_and_binds():
    import cohx
    lib = cohx.load_library()
    for name in declared():
        assert hasattr(lib, name)
