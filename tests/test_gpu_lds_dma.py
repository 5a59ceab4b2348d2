"""GPU: the direct-to-LDS load properties the batch kernel relies on when it
loads a batch's B rows straight into its LDS tile (xspmm_amd/csrc/spmm.hip,
start of a batch): lane l of `buffer_load_dwordx4 ... lds` writes its 16 bytes
at LDS offset 16 l of the 1 KB the load fills, and a lane whose offset lies past
the buffer resource's size writes zeros.  The probe checks
both on one wave with every access in bounds (tests/probes/lds_dma_probe.hip,
built by __graft_entry__.build() or make -C tests/probes)."""
from __future__ import annotations

import os
import subprocess

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
PROG = os.path.join(ROOT, "tests", "probes", "bin", "lds_dma_probe")


def test_lds_dma_layout_and_zero_fill():
    if not os.path.exists(PROG):
        pytest.fail(f"{PROG} is not built (make -C tests/probes)")
    print("running", PROG, flush=True)
    out = subprocess.run([PROG], capture_output=True, text=True, timeout=120)
    print(out.stdout)
    print(out.stderr)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "lds dma probe ok" in out.stdout
