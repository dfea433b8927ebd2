"""CPU: the CPU checkers (oracle/cg_oracle.c) and the library's host-only C
(tensor, token tree and mask, COG1 files) built with AddressSanitizer and
UndefinedBehaviorSanitizer (tests/sanitize/Makefile) and run over random and
edge-case inputs (tests/sanitize/check.c): no sanitizer report, exit 0."""
from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

HERE = Path(__file__).resolve().parent / "sanitize"


def test_host_code_under_asan_and_ubsan(tmp_path):
    if shutil.which("gcc") is None:
        pytest.skip("gcc not available")
    b = subprocess.run(["make", "-C", str(HERE)], capture_output=True, text=True)
    assert b.returncode == 0, b.stdout + b.stderr
    r = subprocess.run([str(HERE / "_build" / "check"), str(tmp_path)], capture_output=True,
                       text=True, timeout=300)
    out = r.stdout + r.stderr
    assert r.returncode == 0, out
    assert "runtime error" not in out and "AddressSanitizer" not in out, out
    assert "sanitize check: ok" in out
