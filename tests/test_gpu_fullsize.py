"""GPU parity at the benchmark configurations' full sizes.

The oracle cannot run the fp64 product of a whole 16384^2 matrix in seconds,
so at full size the checks are:
  * GPU CSR->BCSR of the whole matrix bit-exact against the oracle;
  * C against fp64 truth on a seeded sample of rows (any row/column index
    mistake shows up in a sample);
  * exact, size-independent identities of the kernel: scaling B by 2 scales C
    by exactly 2, and the Tier-2 pipeline (cluster -> permute -> convert ->
    SpMM -> unpermute) equals the un-clustered path row for row within the
    accumulation tolerance.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import xspmm_amd as X
from xspmm_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X")
    X.load()
    return torch


def sampled_truth(p, rows):
    out = np.zeros((len(rows), p.N), np.float64)
    B = p.B.astype(np.float64)
    v = p.vals.astype(np.float64)
    for i, r in enumerate(rows):
        a, b = int(p.rp[r]), int(p.rp[r + 1])
        out[i] = v[a:b] @ B[p.ci[a:b]]
    return out


def rel_frob(a, b):
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.parametrize("name", ["blocks", "templates", "pruned"])
def test_full_size_tier1(torch, name):
    p = synth.CONFIGS[name]()
    print(f"full-size {name}: M={p.M} K={p.K} N={p.N} nnz={p.nnz}", flush=True)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bm = X.csr_to_bcsr(A)
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(Bm.row_ptr.cpu().numpy().astype(np.int64), brp)
    np.testing.assert_array_equal(Bm.col_ind.cpu().numpy().astype(np.int64), bci)
    assert Bm.values.cpu().numpy().tobytes() == bv.tobytes()
    del bv
    Bd = torch.as_tensor(p.B).cuda()
    C = X.spmm(Bm, Bd)
    C2 = X.spmm(Bm, Bd * 2)
    torch.cuda.synchronize()
    assert torch.equal(C2, C * 2)
    rows = np.sort(np.random.default_rng(0).choice(p.M, size=512, replace=False))
    e = rel_frob(C.cpu().numpy()[rows].astype(np.float64), sampled_truth(p, rows))
    assert e <= 1e-5, e


def test_full_size_pipeline_templates(torch):
    p = synth.templates()
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bd = torch.as_tensor(p.B).cuda()
    C1, t1 = X.spmm_pipeline(A, Bd, optimize_pattern=True)
    C0, t0 = X.spmm_pipeline(A, Bd, optimize_pattern=False)
    torch.cuda.synchronize()
    print(f"pipeline timings clustered={t1} plain={t0}", flush=True)
    a, b = C1.cpu().numpy(), C0.cpu().numpy()
    assert rel_frob(a.astype(np.float64), b.astype(np.float64)) <= 1e-6
    rows = np.sort(np.random.default_rng(1).choice(p.M, size=512, replace=False))
    assert rel_frob(a[rows].astype(np.float64), sampled_truth(p, rows)) <= 1e-5
