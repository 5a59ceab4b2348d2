"""GPU: the Tier-2 pipeline's temporary device memory.

The pipeline sizes its BCSR arrays from the bound min(nnz, Mb * Kb) on the
block count while that bound's block values fit 1 GiB (the conversion's count
and fill then run with no host round trip), and exactly, after reading the
count, above it -- as the reference's conversion does
(src/core/conversion.cpp:66-73).  A matrix of full 16x16 blocks has
nnz = 256 * nnzb, so there the bound is 256x the exact size.
xspmm_pipeline_temp_bytes reports the most the last call held at once.
Products the packed kernels cover take packed column batches instead of BCSR
arrays, sized from a bound on the batch count while that fits 256 MiB.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
import xspmm_amd as X
from xspmm_amd import synth

pytestmark = pytest.mark.gpu

FUSED_LIMIT = 1 << 30


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X (torch.cuda.is_available() is False)")
    X.load()
    return torch


def block_diagonal(Mb, N, seed=0, dtype=np.float32):
    """Mb dense 16x16 blocks on the diagonal, values U(-1, 1); B U(-1, 1)."""
    rng = np.random.default_rng(seed)
    M = 16 * Mb
    blocks = rng.uniform(-1, 1, size=(Mb, 16, 16)).astype(dtype)
    rp = (np.arange(M + 1, dtype=np.int64) * 16).astype(np.int32)
    r = np.arange(M)
    ci = ((r // 16)[:, None] * 16 + np.arange(16)[None, :]).reshape(-1).astype(np.int32)
    vals = blocks.reshape(-1)
    B = rng.uniform(-1, 1, size=(M, N)).astype(dtype)
    return synth.Problem("blockdiag", M, M, N, rp, ci, vals, B, cluster=False), blocks


def test_full_blocks_take_exact_bcsr(torch):
    """262144^2 block-diagonal fp32: the BCSR bound's block values would take
    4 GiB and the packed batches' bound 300 MB, the exact arrays 17 MB; the
    pipeline tries the packed form, whose device decision rejects full
    blocks, and takes within 1.5x of the exact BCSR bytes; C equals the
    block products."""
    Mb, N = 16384, 16
    p, blocks = block_diagonal(Mb, N)
    sT, sI = 4, 4
    cap = min(p.nnz, Mb * Mb)
    assert cap * 256 * sT > FUSED_LIMIT
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    C, _ = X.spmm_pipeline(A, B, optimize_pattern=False, timings=False)
    torch.cuda.synchronize()
    used = X.pipeline_temp_bytes()
    exact = (Mb + 1) * sI + 4 + Mb * sI + Mb * 256 * sT  # row_ptr, flag, col_ind, values
    print(f"pipeline temporaries {used} B, exact {exact} B, bound {cap * 256 * sT} B", flush=True)
    assert exact <= used <= 1.5 * exact
    ref = np.einsum("bij,bjn->bin", blocks.astype(np.float64),
                    p.B.astype(np.float64).reshape(Mb, 16, N)).reshape(p.M, N)
    e = oracle.errors(C.cpu().numpy(), ref)
    assert e["rel_frob"] <= 1e-5, e


def test_small_matrix_keeps_fused_bound(torch):
    """A small matrix keeps the bound-sized arrays (no host round trip): the
    reported bytes cover min(nnz, Mb * Kb) blocks; C against fp64.  (The BCSR
    form is forced: this product would take the packed form.)"""
    p = synth.random_csr(500, 700, 64, 0.02, seed=4, dtype=np.float32)
    Mb, Kb = (p.M + 15) // 16, (p.K + 15) // 16
    cap = min(p.nnz, Mb * Kb)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    old = os.environ.get("XSPMM_PIPELINE_FORMAT")
    os.environ["XSPMM_PIPELINE_FORMAT"] = "bcsr"
    try:
        C, _ = X.spmm_pipeline(A, B, optimize_pattern=False, timings=False)
        torch.cuda.synchronize()
    finally:
        if old is None:
            del os.environ["XSPMM_PIPELINE_FORMAT"]
        else:
            os.environ["XSPMM_PIPELINE_FORMAT"] = old
    used = X.pipeline_temp_bytes()
    assert not X.pipeline_last_packed()
    assert used >= cap * 256 * 4 + cap * 4
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    ref = oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, p.B)
    assert oracle.errors(C.cpu().numpy(), ref)["rel_frob"] <= 1e-5


def test_packed_form_takes_no_block_arrays(torch):
    """The fp16 pipeline's packed form: per block-row and wave a batch count
    and offset, and 1152 bytes (A' operand and B-row indices) per batch,
    sized from the bound 2 nnz / 33 + min(Mb * 4, nnz) on the batch count;
    no padded blocks (which would take 512 bytes per block)."""
    p = synth.random_csr(2000, 6000, 64, 0.004, seed=5, dtype=np.float16)
    Mb = (p.M + 15) // 16
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    nnzb = len(bci)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    C, _ = X.spmm_pipeline(A, B, optimize_pattern=False, timings=False)
    torch.cuda.synchronize()
    assert X.pipeline_last_packed()
    used = X.pipeline_temp_bytes()
    bound = 2 * p.nnz // 33 + min(Mb * 4, p.nnz)
    print(f"packed form temporaries {used} B; BCSR blocks would take {nnzb * 512} B", flush=True)
    assert used < nnzb * 512 // 2
    assert used <= bound * 1152 + Mb * 64 + 16 * 256
    ref = oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, p.B)
    assert oracle.errors(C.cpu().numpy(), ref)["rel_frob"] <= 2e-3


def test_fp32_packed_form_takes_no_block_arrays(torch):
    """The fp32 pipeline's packed form: 272 bytes per batch of four columns
    (A' operand and B-row indices), sized from the bound nnz / 4 + 4 Mb;
    no padded blocks (which would take 1024 bytes per block)."""
    p = synth.random_csr(2000, 6000, 64, 0.004, seed=6, dtype=np.float32)
    Mb = (p.M + 15) // 16
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    nnzb = len(bci)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    C, _ = X.spmm_pipeline(A, B, optimize_pattern=False, timings=False)
    torch.cuda.synchronize()
    assert X.pipeline_last_packed()
    used = X.pipeline_temp_bytes()
    bound = p.nnz // 4 + 4 * Mb
    print(f"fp32 packed form temporaries {used} B; BCSR blocks would take {nnzb * 1024} B", flush=True)
    assert used < nnzb * 1024 // 2
    assert used <= bound * 272 + Mb * 32 + 16 * 256
    ref = oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, p.B)
    assert oracle.errors(C.cpu().numpy(), ref)["rel_frob"] <= 1e-5
