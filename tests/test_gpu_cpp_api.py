"""GPU: the C++ drop-in API (include/xspmm/*.hpp) driven from a C++ program,
as the reference's examples drive it (examples/01, 05, 06)."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
PROG = os.path.join(ROOT, "xspmm_amd", "bin", "api_checks")


def test_cpp_api_checks():
    if not os.path.exists(PROG):
        pytest.fail(f"{PROG} is not built (make -C xspmm_amd/csrc examples)")
    out = subprocess.run([PROG], capture_output=True, text=True, timeout=300)
    print(out.stdout)
    print(out.stderr)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "[FAIL]" not in out.stdout
    assert out.stdout.count("[PASS]") >= 17
