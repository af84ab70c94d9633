"""Host checks of device math restated from the C library: the log1pf used by
the Qwen3.5 softplus (qwen35/kernels.rs:22-24 calls f32::ln_1p) compiles as
plain C++ and must equal glibc's log1pf bit for bit."""
import os
import subprocess

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CSRC = os.path.join(ROOT, "coheryn-ai-studio_amd", "csrc")


def test_log1pf_restatement_equals_glibc(tmp_path):
    exe = tmp_path / "l1p"
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fno-fast-math", "-I", CSRC,
                    os.path.join(ROOT, "tests", "host_log1pf.cpp"), "-o", str(exe), "-lm"],
                   check=True)
    out = subprocess.run([str(exe), "3"], capture_output=True, text=True, timeout=300)
    print(out.stdout)
    assert out.returncode == 0, out.stdout
    assert "mismatches 0" in out.stdout


def test_expf_restatement_equals_glibc(tmp_path):
    """The GPU expf (csrc/expf.h: SwiGLU, softmax, the Qwen3.5 gates) against
    glibc's expf, bit for bit."""
    exe = tmp_path / "ef"
    subprocess.run(["g++", "-O2", "-ffp-contract=off", "-fno-fast-math", "-I", CSRC,
                    os.path.join(ROOT, "tests", "host_expf.cpp"), "-o", str(exe), "-lm"],
                   check=True)
    out = subprocess.run([str(exe), "7"], capture_output=True, text=True, timeout=300)
    print(out.stdout)
    assert out.returncode == 0, out.stdout
    assert "mismatches 0" in out.stdout
