"""GPU: the fp16 Tier-1 kernels that XSPMM_SPMM_KERNEL=batch|gather|panel
forces (a diagnostic switch, read once per process) each give the tile
product: against the fp64 CSR product on a random matrix with ragged M and K,
into an aligned C and into a C that starts 4 bytes into its allocation (the
vector stores must fall back to scalar ones there; both results must agree
bit for bit).  Each kernel runs in its own process, one after the other."""
from __future__ import annotations

import json
import os
import subprocess
import sys

import pytest

pytestmark = pytest.mark.gpu

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))

CHILD = r"""
import json, sys
import numpy as np, torch
sys.path.insert(0, sys.argv[1])
import oracle
import xspmm_amd as X
from xspmm_amd import synth
out = {}
for N in (96, 40):
    p = synth.random_csr(203, 150, N, 0.04, seed=N)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bm = X.csr_to_bcsr(A)
    B = torch.as_tensor(p.B).cuda()
    Ca = torch.full((p.M, N), float("nan"), dtype=torch.float32, device="cuda")
    flat = torch.full((p.M * N + 4,), float("nan"), dtype=torch.float32, device="cuda")
    Cm = flat[1:1 + p.M * N].view(p.M, N)
    X.spmm(Bm, B, Ca, N)
    X.spmm(Bm, B, Cm, N)
    torch.cuda.synchronize()
    ref = oracle.csr_spmm_f64(p.M, N, p.rp, p.ci, p.vals, p.B)
    a = Ca.cpu().numpy().astype(np.float64)
    e = float(np.linalg.norm(a - ref) / max(np.linalg.norm(ref), 1e-300))
    out[str(N)] = {"rel_frob": e, "finite": bool(np.all(np.isfinite(a))),
                   "same_misaligned": bool(np.array_equal(Ca.cpu().numpy(), Cm.cpu().numpy()))}
print(json.dumps(out))
"""


@pytest.mark.parametrize("kernel", ["batch", "gather", "panel"])
def test_forced_fp16_kernel(kernel):
    env = dict(os.environ, XSPMM_SPMM_KERNEL=kernel)
    print(f"forced kernel {kernel}", flush=True)
    r = subprocess.run([sys.executable, "-c", CHILD, ROOT], env=env, capture_output=True,
                       text=True, timeout=180)
    print(r.stdout[-2000:])
    print(r.stderr[-2000:])
    assert r.returncode == 0, r.stderr[-2000:]
    res = json.loads(r.stdout.strip().splitlines()[-1])
    for n, v in res.items():
        # the gather kernel needs N % 2 == 0 and the batch kernel N % 8 == 0;
        # other N fall through to the panel kernel, which takes any N
        assert v["finite"], (kernel, n, v)
        assert v["rel_frob"] <= 1e-5, (kernel, n, v)
        assert v["same_misaligned"], (kernel, n, v)
