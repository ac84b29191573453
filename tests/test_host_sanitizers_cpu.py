"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only): tests/host_sanitizer_driver.cpp is built together with the
library sources, host code instrumented and device code not, and run; any
sanitizer report (memory error, leak, undefined behaviour) fails the test.
The driver makes no GPU call, so it runs on any machine with hipcc."""
from __future__ import annotations

import os
import shlex
import shutil
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
SANITIZE = "-Xarch_host -fsanitize=address -Xarch_host -fsanitize=undefined -fno-gpu-sanitize"


def _hipcc():
    p = Path(os.environ.get("ROCM_PATH", "/opt/rocm")) / "bin" / "hipcc"
    return str(p) if p.exists() else shutil.which("hipcc")


def test_c_abi_host_code_is_sanitizer_clean(tmp_path):
    hipcc = _hipcc()
    if hipcc is None:
        pytest.skip("hipcc not available")
    exe = tmp_path / "drv"
    cmd = [hipcc, "--offload-arch=gfx950", "-O1", "-g", "-std=c++20",
           "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           *shlex.split(SANITIZE),
           "-I", str(ROOT / "include"), "-I", str(ROOT / "cudalab_amd" / "csrc"),
           str(ROOT / "cudalab_amd" / "csrc" / "cq_capi.cpp"),
           str(ROOT / "cudalab_amd" / "csrc" / "cq_kernels.hip"),
           str(ROOT / "cudalab_amd" / "csrc" / "cq_quantize.hip"),
           str(ROOT / "tests" / "host_sanitizer_driver.cpp"), "-o", str(exe)]
    b = subprocess.run(cmd, capture_output=True, text=True, timeout=600)
    assert b.returncode == 0, b.stderr[-2000:]
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=1:halt_on_error=1",
               UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    r = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-3000:]
    assert "ERROR: AddressSanitizer" not in out and "runtime error" not in out, out[-3000:]
    assert out.rstrip().endswith("done")
    assert "problem 4999: output y overlaps w of problem 7" in out
