"""GPU: the column-batch kernel for N > 128.

One workgroup covers 256 columns: each block pair is streamed and compacted
once and every batch is multiplied with both 128-column chunks (taken
automatically when the grid keeps at least 1024 workgroups; the tests force
it with XSPMM_BATCH_WIDE=on).  Batches and
the per-chunk accumulation order are those of one workgroup per 128-column
chunk, so C must equal that path (XSPMM_BATCH_WIDE=off) bit for bit, and the
fp64 product within the fp16 tolerance.  Covers N a multiple of 256, a
partial second chunk (N = 136, 200, 264), several 256-column groups
(N = 512, 520), int32 and int64, ragged M and K, the prepared product (packed
batches, clustered: un-permuted store) against the pipeline, and the
headline matrix at N = 256.
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


def host(t):
    return t.detach().cpu().numpy()


def note(msg):
    print(msg, flush=True)


def both_paths(torch, Bm, Bd, N, monkeypatch):
    monkeypatch.setenv("XSPMM_BATCH_WIDE", "on")
    C_wide = torch.full((Bm.num_rows, N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm(Bm, Bd, C_wide, N)
    monkeypatch.setenv("XSPMM_BATCH_WIDE", "off")
    C_narrow = torch.full((Bm.num_rows, N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm(Bm, Bd, C_narrow, N)
    monkeypatch.delenv("XSPMM_BATCH_WIDE")
    torch.cuda.synchronize()
    return C_wide, C_narrow


WIDE = [(1000, 700, 136), (777, 1500, 200), (2048, 2048, 256), (515, 333, 264),
        (1200, 900, 512), (600, 4096, 520)]


@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("M,K,N", WIDE, ids=[f"{m}x{k}xN{n}" for m, k, n in WIDE])
def test_wide_n_equals_chunked_and_truth(torch, M, K, N, itype, monkeypatch):
    p = synth.random_csr(M, K, N, 0.03, seed=M + N, dtype=np.float16)
    A = X.CSRMatrix.from_host(M, K, p.rp.astype(itype), p.ci.astype(itype), p.vals)
    Bm = X.csr_to_bcsr(A)
    Bd = torch.as_tensor(p.B).cuda()
    C_wide, C_narrow = both_paths(torch, Bm, Bd, N, monkeypatch)
    assert torch.equal(C_wide, C_narrow)
    ref = oracle.csr_spmm_f64(M, N, p.rp, p.ci, p.vals, p.B)
    C = host(C_wide)
    assert np.all(np.isfinite(C))
    e = oracle.errors(C, ref)
    note(f"wide N {M}x{K} N={N} {itype.__name__}: rel_frob {e['rel_frob']:.3e}")
    assert e["rel_frob"] <= 1e-5, e


def test_wide_n_dense_blocks(torch, monkeypatch):
    # configs[1]'s shape of input (fully dense 16x16 blocks, 5 % of the grid)
    # at N = 256: every pair a batch of its own
    p = synth.blocks(M=2048, N=256)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bm = X.csr_to_bcsr(A)
    C_wide, C_narrow = both_paths(torch, Bm, torch.as_tensor(p.B).cuda(), p.N, monkeypatch)
    assert torch.equal(C_wide, C_narrow)
    ref = oracle.csr_spmm_f64(p.M, p.N, p.rp, p.ci, p.vals, p.B)
    assert oracle.errors(host(C_wide), ref)["rel_frob"] <= 1e-5


@pytest.mark.parametrize("wide", ["on", "off"])
@pytest.mark.parametrize("cluster", [False, True])
def test_wide_n_plan_equals_pipeline(torch, cluster, wide, monkeypatch):
    monkeypatch.setenv("XSPMM_BATCH_WIDE", wide)
    p = synth.random_csr(3000, 2500, 264, 0.02, seed=3, dtype=np.float16)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    C_pipe, _ = X.spmm_pipeline(A, B, optimize_pattern=cluster)
    plan = X.SpMMPlan(A, optimize_pattern=cluster)
    C_plan = plan.execute(B)
    torch.cuda.synchronize()
    plan.close()
    assert torch.equal(C_pipe, C_plan)


def test_wide_n_headline_matrix(torch, monkeypatch):
    p = synth.templates(N=256)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bm = X.csr_to_bcsr(A)
    C_wide, C_narrow = both_paths(torch, Bm, torch.as_tensor(p.B).cuda(), p.N, monkeypatch)
    assert torch.equal(C_wide, C_narrow)
    rows = np.sort(np.random.default_rng(0).choice(p.M, size=256, replace=False))
    ref = np.stack([p.vals[p.rp[r]:p.rp[r + 1]].astype(np.float64)
                    @ p.B[p.ci[p.rp[r]:p.rp[r + 1]]].astype(np.float64) for r in rows])
    assert oracle.errors(host(C_wide)[rows], ref)["rel_frob"] <= 1e-5
