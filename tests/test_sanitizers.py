"""Host code under AddressSanitizer and UndefinedBehaviorSanitizer, on the
CPU: libpda's C-ABI (validation, the split planner, workspace layouts, the
prefill range planner; tests/sanitize/pda_host_driver.cpp) and the oracle's
C++ restatement (tests/sanitize/oracle_driver.cpp), each built with both
sanitizers by tests/sanitize/Makefile and run to completion with
halt_on_error, so any finding fails the test. Building libpda's objects
with the sanitized host pass takes a minute or two."""

import os
import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent
HIPCC = Path("/opt/rocm/bin/hipcc")
CLANG = Path("/opt/rocm/llvm/bin/clang++")

pytestmark = pytest.mark.skipif(not (HIPCC.exists() and CLANG.exists()),
                                reason="needs ROCm's hipcc and clang++")

ENV = dict(os.environ, ASAN_OPTIONS="detect_leaks=0:halt_on_error=1:abort_on_error=0",
           UBSAN_OPTIONS="halt_on_error=1:print_stacktrace=1")


@pytest.fixture(scope="module")
def built(tmp_path_factory):
    out = tmp_path_factory.mktemp("sanitize")
    jobs = str(min(8, os.cpu_count() or 1))
    r = subprocess.run(["make", "-j", jobs, "-C", str(HERE / "sanitize"), f"OUT={out}"],
                       capture_output=True, text=True, timeout=1200)
    assert r.returncode == 0, r.stdout[-3000:] + r.stderr[-3000:]
    yield out
    shutil.rmtree(out, ignore_errors=True)


def run(binary):
    r = subprocess.run([str(binary)], capture_output=True, text=True, timeout=600, env=ENV)
    text = r.stdout + r.stderr
    print(text[-2000:])
    assert r.returncode == 0, text[-4000:]
    assert "runtime error" not in text and "AddressSanitizer" not in text
    assert "ok (0 failures)" in text


def test_libpda_host_code(built):
    run(built / "pda_host_driver")


def test_oracle(built):
    run(built / "oracle_driver")
