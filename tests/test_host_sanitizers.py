"""The C ABI's host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

tests/sanitize/Makefile compiles every mcoplib_amd/csrc/*.hip file for the host only (no device
code, nothing registered with a GPU runtime), instrumented, and links it with
tests/sanitize/host_abi_driver.cpp, which calls every entry point over a grid of shapes, dtypes,
flags and pointer alignments (about 340,000 calls, with and without MCOP_DEBUG_TRACE). Each call
must end in a documented status with a message; a sanitizer report fails the run."""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

SAN = Path(__file__).resolve().parent / "sanitize"


def test_c_abi_host_code_is_clean_under_sanitizers():
    if not (SAN / "Makefile").exists():
        pytest.skip("tests/sanitize is not part of this tree")
    for tool in ("/opt/rocm/bin/hipcc", "/opt/rocm/llvm/bin/clang++"):
        if not os.access(tool, os.X_OK):
            pytest.skip(f"{tool} not available")
    if shutil.which("make") is None:
        pytest.skip("make not available")
    jobs = str(min(8, os.cpu_count() or 1))
    r = subprocess.run(["make", "-C", str(SAN), "-j", jobs, "run"], capture_output=True,
                       text=True, timeout=600)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out[-4000:]
    summaries = [ln for ln in r.stdout.splitlines() if ln.startswith("calls ")]
    assert len(summaries) == 2, out[-4000:]
    for ln in summaries:
        assert "unexpected 0;" in ln and "launch 0;" not in ln, ln
    assert "Sanitizer" not in out and "runtime error" not in out, out[-4000:]
