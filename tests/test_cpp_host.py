"""The C++ host API (include/spl_sage.hpp) on the CPU: runs tests/cpp/bin/host_tests,
the reference's host-side tests (tests.rs:17-22, 95-190, 245-262) restated in C++
against the in-tree libsage_hip.so, and the same program under AddressSanitizer
(with leak detection) and UndefinedBehaviorSanitizer against a copy of the
library whose host code is instrumented (tests/cpp/bin/san). Built by
__graft_entry__.build()."""
from __future__ import annotations

import os
import subprocess
from pathlib import Path

BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "host_tests"
SAN_BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "san" / "host_tests"
# Stop at the first report; UBSan reports exit non-zero instead of continuing.
SAN_ENV = {"ASAN_OPTIONS": "detect_leaks=1:halt_on_error=1:abort_on_error=0",
           "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1"}


def test_cpp_host_api():
    assert BIN.exists(), f"{BIN} is not built; run `python __graft_entry__.py` (build)"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout


def test_cpp_host_api_under_sanitizers():
    assert SAN_BIN.exists(), f"{SAN_BIN} is not built; run `python __graft_entry__.py` (build)"
    r = subprocess.run([str(SAN_BIN)], capture_output=True, text=True, timeout=120, env={**os.environ, **SAN_ENV})
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
    assert "runtime error" not in r.stderr and "Sanitizer" not in r.stderr, r.stderr
