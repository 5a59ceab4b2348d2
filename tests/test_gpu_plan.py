"""GPU: prepared Tier-2 products (xspmm_plan_*).

A plan runs the pipeline's clustering, permutation and conversion once;
execute() must return the pipeline's C bit for bit (the same kernels, with the
un-permutation fused into the fp16 store or done from the plan's workspace),
for every N, repeatedly, after the source matrix is freed, and with the
longest-row-first dispatch order precomputed.  The pipeline itself is checked
against the oracle elsewhere; here C is also compared with fp64 truth.
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


def note(msg):
    print(msg, flush=True)


def many_joins(rng, M, K, n_patterns=30):
    base = [rng.choice(K, size=int(rng.integers(5, 60)), replace=False) for _ in range(n_patterns)]
    rows = []
    for _ in range(M):
        b = base[int(rng.integers(0, len(base)))]
        keep = b[rng.random(len(b)) < 0.9]
        # distinct columns: duplicates would make the CSR sum differ from the
        # conversion's last-entry-wins rule that the fp64 truth below ignores
        rows.append(np.unique(np.concatenate([keep, rng.integers(0, K, size=int(rng.integers(0, 4)))])))
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum([len(x) for x in rows])
    return rp, np.concatenate(rows).astype(np.int64)


def truth(M, rp, ci, vals, B):
    return oracle.csr_spmm_f64(M, B.shape[1], rp, ci, vals.astype(np.float64), B.astype(np.float64))


@pytest.mark.parametrize("cluster", [True, False])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("vdtype", [np.float16, np.float32])
def test_plan_equals_pipeline(torch, vdtype, itype, cluster):
    rng = np.random.default_rng(7)
    M, K = 3001, 2500  # ragged M and K
    rp, ci = many_joins(rng, M, K)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(vdtype)
    A = X.CSRMatrix.from_host(M, K, rp.astype(itype), ci.astype(itype), vals)
    plan = X.SpMMPlan(A, optimize_pattern=cluster)
    note(f"plan {np.dtype(vdtype).name}/{np.dtype(itype).name} cluster={cluster} "
         f"blocks={plan.num_blocks} prep={plan.timings}")
    assert plan.clustered == cluster and plan.num_block_rows == (M + 15) // 16
    assert plan.timings["total_pipeline_ms"] > 0
    # fused (N % 8 == 0, fp16), workspace (other N, fp32), growing and shrinking N
    for N in (64, 8, 136, 13, 1, 64, 200):
        B_h = rng.uniform(-1, 1, size=(K, N)).astype(vdtype)
        B = torch.as_tensor(B_h).cuda()
        C_pipe, _ = X.spmm_pipeline(A, B, optimize_pattern=cluster)
        C_plan = plan.execute(B)
        torch.cuda.synchronize()
        assert torch.equal(C_pipe, C_plan), N
        if N in (13, 136):
            ref = truth(M, rp, ci, vals, B_h)
            e = oracle.errors(C_plan.cpu().numpy(), ref)
            assert e["rel_frob"] <= (2e-3 if vdtype == np.float16 else 1e-5), e
    plan.close()


@pytest.mark.parametrize("cluster", [True, False])
def test_plan_on_a_full_block_grid(torch, cluster):
    # every 16x16 block present: the pipeline takes the GEMM-tiled kernel,
    # and so does the plan (through its workspace when rows are permuted)
    rng = np.random.default_rng(12)
    M, K, N = 520, 300, 136
    D = rng.random((M, K)) < 0.3
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum(D.sum(1))
    ci = np.nonzero(D)[1].astype(np.int64)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(np.float16)
    A = X.CSRMatrix.from_host(M, K, rp.astype(np.int32), ci.astype(np.int32), vals)
    plan = X.SpMMPlan(A, optimize_pattern=cluster)
    assert plan.num_blocks == ((M + 15) // 16) * ((K + 15) // 16)
    for N in (136, 64, 12):
        B = torch.as_tensor(rng.uniform(-1, 1, size=(K, N)).astype(np.float16)).cuda()
        C_pipe, _ = X.spmm_pipeline(A, B, optimize_pattern=cluster)
        C_plan = plan.execute(B)
        torch.cuda.synchronize()
        assert torch.equal(C_pipe, C_plan), N


@pytest.mark.parametrize("cluster", [True, False])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_packed_plan_equals_unpacked_plan_and_pipeline(torch, itype, cluster, monkeypatch):
    # fp16 plans of sparse blocks keep the SpMM kernel's column batches; C is
    # the same as multiplying the BCSR matrix (and as the pipeline's)
    rng = np.random.default_rng(21)
    M, K = 5001, 4000
    rp, ci = many_joins(rng, M, K, n_patterns=200)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(np.float16)
    vals[rng.random(len(vals)) < 0.05] = 0  # explicit zeros keep their columns' blocks
    A = X.CSRMatrix.from_host(M, K, rp.astype(itype), ci.astype(itype), vals)
    packed = X.SpMMPlan(A, optimize_pattern=cluster)
    monkeypatch.setenv("XSPMM_PLAN_PACK", "off")
    plain = X.SpMMPlan(A, optimize_pattern=cluster)
    monkeypatch.delenv("XSPMM_PLAN_PACK")
    note(f"packed batches {packed.packed_batches}, blocks {packed.num_blocks}")
    assert packed.packed_batches > 0 and plain.packed_batches == -1
    for N in (8, 64, 128, 200, 24, 12):
        B = torch.as_tensor(rng.uniform(-1, 1, size=(K, N)).astype(np.float16)).cuda()
        C1 = packed.execute(B)
        C2 = plain.execute(B)
        C3, _ = X.spmm_pipeline(A, B, optimize_pattern=cluster)
        torch.cuda.synchronize()
        assert torch.equal(C1, C2), N
        assert torch.equal(C1, C3), N
    packed.close()
    plain.close()


def test_plan_outlives_its_source_matrix(torch):
    rng = np.random.default_rng(8)
    M, K, N = 2000, 1800, 64
    rp, ci = many_joins(rng, M, K)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(np.float16)
    B_h = rng.uniform(-1, 1, size=(K, N)).astype(np.float16)
    B = torch.as_tensor(B_h).cuda()
    A = X.CSRMatrix.from_host(M, K, rp.astype(np.int32), ci.astype(np.int32), vals)
    C_pipe, _ = X.spmm_pipeline(A, B)
    plan = X.SpMMPlan(A)
    del A
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    # reuse the freed memory for something else before executing
    junk = torch.full((4 << 20,), 7, dtype=torch.int32, device="cuda")
    C_plan = plan.execute(B)
    torch.cuda.synchronize()
    assert torch.equal(C_pipe, C_plan)
    del junk


@pytest.mark.parametrize("N", [64, 128])
def test_plan_with_dispatch_order(torch, N):
    # more than 2048 block-rows with skewed lengths: the plan precomputes the
    # longest-row-first order that the pipeline recomputes per call
    rng = np.random.default_rng(9)
    M, K = 48000, 4096
    deg = np.minimum((rng.pareto(1.3, size=M) * 3 + 1).astype(np.int64), 2000)
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum(deg)
    ci = rng.integers(0, K, size=int(rp[-1])).astype(np.int64)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(np.float16)
    A = X.CSRMatrix.from_host(M, K, rp.astype(np.int32), ci.astype(np.int32), vals)
    B = torch.as_tensor(rng.uniform(-1, 1, size=(K, N)).astype(np.float16)).cuda()
    for cluster in (False, True):
        C_pipe, _ = X.spmm_pipeline(A, B, optimize_pattern=cluster)
        plan = X.SpMMPlan(A, optimize_pattern=cluster)
        for _ in range(3):
            C_plan = plan.execute(B)
            torch.cuda.synchronize()
            assert torch.equal(C_pipe, C_plan)
        plan.close()


def test_plan_degenerate_shapes(torch):
    for M, K, rp, ci in [
        (37, 50, np.zeros(38, np.int64), np.zeros(0, np.int64)),   # no entries
        (1, 1, np.array([0, 1]), np.array([0])),
        (0, 16, np.zeros(1, np.int64), np.zeros(0, np.int64)),      # no rows
    ]:
        vals = np.ones(len(ci), np.float16)
        A = X.CSRMatrix.from_host(M, K, rp.astype(np.int32), ci.astype(np.int32), vals)
        B = torch.ones((K, 16), dtype=torch.float16, device="cuda")
        plan = X.SpMMPlan(A)
        C = plan.execute(B)
        torch.cuda.synchronize()
        C_pipe, _ = X.spmm_pipeline(A, B)
        assert torch.equal(C, C_pipe)
        plan.close()


def test_plan_rejects_bad_arguments(torch):
    A = X.CSRMatrix.from_host(2, 16, np.array([0, 1, 2], np.int32), np.array([0, 99], np.int32),
                              np.ones(2, np.float16))
    with pytest.raises(X.XspmmInvalidArgument):
        X.SpMMPlan(A)  # column out of range
    A = X.CSRMatrix.from_host(2, 16, np.array([0, 1, 2], np.int32), np.array([0, 5], np.int32),
                              np.ones(2, np.float16))
    with pytest.raises(X.XspmmInvalidArgument):
        X.SpMMPlan(A, hw_block_size=8)
    plan = X.SpMMPlan(A)
    with pytest.raises(TypeError):
        plan.execute(torch.ones((16, 8), dtype=torch.float32, device="cuda"))
    plan.close()
    with pytest.raises(RuntimeError):
        plan.execute(torch.ones((16, 8), dtype=torch.float16, device="cuda"))


def test_plan_headline_matrix_matches_pipeline(torch):
    p = synth.templates()
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    C_pipe, _ = X.spmm_pipeline(A, B)
    plan = X.SpMMPlan(A)
    note(f"templates plan blocks={plan.num_blocks} prep={plan.timings}")
    C_plan = plan.execute(B)
    torch.cuda.synchronize()
    assert torch.equal(C_pipe, C_plan)
