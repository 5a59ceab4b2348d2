"""GPU: the vendor comparison harness (libxspmm_vendor.so) computes the same
product as this library -- otherwise the benchmark's vendor columns would
compare different work.  rocSPARSE CSR / BSR and rocBLAS dense GEMM against
Tier-1 SpMM and fp64 truth, fp16 and fp32 inputs."""
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
    from xspmm_amd import vendor
    vendor.load()
    return torch


@pytest.mark.parametrize("vdtype", [np.float16, np.float32])
@pytest.mark.parametrize("N", [64, 136])
def test_vendor_products_match(torch, vdtype, N):
    from xspmm_amd import vendor as V
    p = synth.random_csr(1000, 800, N, 0.02, seed=5, dtype=vdtype)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp.astype(np.int32), p.ci.astype(np.int32), p.vals)
    Ab = X.csr_to_bcsr(A)
    B = torch.as_tensor(p.B).cuda()
    C = X.spmm(Ab, B)
    truth = oracle.csr_spmm_f64(p.M, N, p.rp, p.ci, p.vals, p.B)
    tol = 2e-3 if vdtype == np.float16 else 1e-5
    Cc, t1 = V.csr_spmm(A, B, warmup=1, iters=3)
    Kp = Ab.num_block_cols * 16
    Bp = torch.cat([B, torch.zeros((Kp - p.K, N), dtype=B.dtype, device=B.device)])
    Cb, t2 = V.bsr_spmm(Ab, Bp, warmup=1, iters=3)
    D = torch.as_tensor(np.asarray(synth_dense(p), dtype=vdtype)).cuda()
    Cd, t3 = V.dense_gemm(D, B, warmup=1, iters=3)
    torch.cuda.synchronize()
    for name, Cv, t in (("xspmm", C, 1.0), ("csr", Cc, t1), ("bsr", Cb, t2), ("dense", Cd, t3)):
        e = oracle.errors(Cv.cpu().numpy(), truth)
        print(name, t, e, flush=True)
        assert e["rel_frob"] <= tol, (name, e)
        assert t > 0


def synth_dense(p):
    D = np.zeros((p.M, p.K), np.float32)
    for r in range(p.M):
        a, b = int(p.rp[r]), int(p.rp[r + 1])
        D[r, p.ci[a:b]] = p.vals[a:b]
    return D
