"""The C++ host API (include/spl_sage.hpp) on the CPU: runs tests/cpp/bin/host_tests,
the reference's host-side tests (tests.rs:17-22, 95-190, 245-262) restated in C++
against the in-tree libsage_hip.so. Built by __graft_entry__.build()."""
from __future__ import annotations

import subprocess
from pathlib import Path

BIN = Path(__file__).resolve().parent / "cpp" / "bin" / "host_tests"


def test_cpp_host_api():
    assert BIN.exists(), f"{BIN} is not built; run `python __graft_entry__.py` (build)"
    r = subprocess.run([str(BIN)], capture_output=True, text=True, timeout=60)
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    assert "0 failure(s)" in r.stdout
