"""The host C/C++ code under AddressSanitizer and UndefinedBehaviorSanitizer
(CPU only): tests/sanitize/Makefile builds the library's host side, the
oracle and the CPU baseline with both sanitizers and runs host_checks.cpp
(repack against the oracle, oracle and baseline at ragged shapes, every
argument check at extreme sizes). Any sanitizer report or failed expectation
fails this test."""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

SAN = Path(__file__).resolve().parent / "sanitize"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def test_host_code_under_asan_and_ubsan():
    if not (ROCM / "bin" / "hipcc").exists() or not (ROCM / "llvm" / "bin" / "clang++").exists():
        pytest.skip("ROCm clang/hipcc not present")
    if shutil.which("make") is None:
        pytest.skip("make not present")
    jobs = str(min(8, os.cpu_count() or 1))
    res = subprocess.run(["make", "-C", str(SAN), f"-j{jobs}", "run"], capture_output=True, text=True, timeout=1200)
    out = res.stdout + res.stderr
    assert res.returncode == 0, out[-6000:]
    assert "validation checks done: 0 failures" in out, out[-6000:]
    assert "runtime error" not in out and "ERROR: AddressSanitizer" not in out, out[-6000:]
