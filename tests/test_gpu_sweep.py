"""GPU: the reference's Tier-1 density sweep (examples/05_core_spmm_benchmark.cpp).

Banded 16384 x 16384 matrices at 90, 50, 5, 0.5 and 0.1 % density
(bandwidth int(density * K / 2), values U(0.1, 1), examples/05:103-108),
B = ones (:117), N = 128: C[i, :] is row i's sum, the closed form behind
the reference's check against rocblas_sgemm (:147-181).  Here in fp16 (the
matrix-core path) against the fp64 row sums, relative Frobenius <= 1e-5
(the reference's own check is an absolute 1e-2); the BCSR block count is
checked against the band's closed form, and scaling B by 2 scales C by
exactly 2.
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
        pytest.fail("GPU tests need an MI355X (torch.cuda.is_available() is False)")
    X.load()
    return torch


def band_blocks(M, bw):
    """Blocks of a 16x16 tiling that a band |i - j| <= bw touches: block-row b
    spans block columns floor(max(0, 16b - bw) / 16) .. floor(min(M-1, 16b + 15 + bw) / 16)."""
    b = np.arange((M + 15) // 16)
    lo = np.maximum(0, 16 * b - bw) // 16
    hi = np.minimum(M - 1, 16 * b + 15 + bw) // 16
    return int((hi - lo + 1).sum())


@pytest.mark.parametrize("name", list(synth.SWEEP_DENSITIES))
def test_density_sweep_row_sums(torch, name):
    p = synth.CONFIGS[f"banded{name}"]()
    bw = p.meta["bandwidth"]
    print(f"banded {name} %: bandwidth {bw}, nnz {p.nnz}", flush=True)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bm = X.csr_to_bcsr(A)
    assert Bm.num_blocks == band_blocks(p.M, bw)
    del A
    B = torch.ones((p.K, p.N), dtype=torch.float16, device="cuda")
    C = X.spmm(Bm, B)
    C2 = X.spmm(Bm, B * 2)
    torch.cuda.synchronize()
    assert torch.equal(C2, C * 2)
    rs = np.add.reduceat(p.vals.astype(np.float64), p.rp[:-1].astype(np.int64))
    Ch = C.cpu().numpy()
    assert np.all(np.isfinite(Ch))
    # every column of C equals the row sum
    e = oracle.errors(Ch, np.repeat(rs[:, None], p.N, axis=1))
    print(f"  nnzb {Bm.num_blocks}: rel_frob {e['rel_frob']:.3e} max_abs {e['max_abs']:.3e}",
          flush=True)
    assert e["rel_frob"] <= 1e-5, e
