"""GPU parity at the benchmark configurations that the other files do not
run at their own workload, and regression tests of the Tier-1 launcher's
input handling.

  * configs[0] ``cpu_ref`` (1024^2 fp32, 1 %, N = 64) at its exact workload:
    Tier-1 with int32 and int64 indices over the whole C against the oracle's
    fp64 tile product, and the Tier-2 pipeline and prepared product with
    clustering off (the config) and on, against the fp64 CSR product.
  * configs[3] ``gnn`` (131072^2 power-law adjacency, N = 64) at full size:
    the permuted CSR and the GPU CSR->BCSR bit-exact against the oracle
    (host-engine permutation), Tier-1 C on sampled rows against fp64,
    spmm(2B) == 2 spmm(B), 100 Tier-1 calls on one BCSR matrix each equal to
    the first (the reference's amortisation story, README.md:127), and the
    prepared product equal to the pipeline.
  * configs[4] ``pruned`` with clustering on at full size: the clustered
    pipeline equals the unclustered one row for row, and sampled rows match
    fp64.
  * fully populated block grids whose blocks are not in the canonical layout
    (block columns permuted within rows, uneven rows, columns outside the
    grid): the GEMM-tiled kernel's tiles must notice and still give the
    tile-kernel product (reference src/common/spmm_math.hpp:68-114 sums a
    row's blocks in stored order).
  * dense operands the kernels cannot take (wrong device, shape, dtype, a
    transposed view, an fp16 B off a 16-byte boundary) are rejected before
    any kernel runs; a C that starts 4 bytes into its allocation is taken
    (the batch, GEMM-tiled, fp32 and pipeline paths store into it the same
    values as into an aligned C).
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


def rel_frob(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


def csr_rows_f64(rp, ci, vals, B, rows):
    """fp64 product rows A[rows, :] @ B of a host CSR matrix."""
    out = np.zeros((len(rows), B.shape[1]), np.float64)
    Bd = B.astype(np.float64)
    for i, r in enumerate(rows):
        a, b = int(rp[r]), int(rp[r + 1])
        out[i] = vals[a:b].astype(np.float64) @ Bd[ci[a:b]]
    return out


# ---------------------------------------------------------------------------
# cpu_ref
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_cpu_ref_tier1_whole_c(torch, itype):
    p = synth.cpu_ref()
    note(f"cpu_ref Tier-1 {itype.__name__}: M={p.M} K={p.K} N={p.N} nnz={p.nnz}")
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp.astype(itype), p.ci.astype(itype), p.vals)
    Bm = X.csr_to_bcsr(A)
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(Bm.row_ptr).astype(np.int64), brp)
    np.testing.assert_array_equal(host(Bm.col_ind).astype(np.int64), bci)
    assert host(Bm.values).tobytes() == bv.tobytes()
    C = torch.full((p.M, p.N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm(Bm, torch.as_tensor(p.B).cuda(), C)
    torch.cuda.synchronize()
    ref = oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, p.B)
    Ch = host(C)
    assert np.all(np.isfinite(Ch))
    e = rel_frob(Ch, ref)
    note(f"  rel_frob {e:.3e}")
    assert e <= 1e-5, e


@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("cluster", [False, True])
def test_cpu_ref_tier2_and_plan(torch, itype, cluster):
    p = synth.cpu_ref()
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp.astype(itype), p.ci.astype(itype), p.vals)
    B = torch.as_tensor(p.B).cuda()
    C, t = X.spmm_pipeline(A, B, optimize_pattern=cluster)
    plan = X.SpMMPlan(A, optimize_pattern=cluster)
    Cp = plan.execute(B)
    torch.cuda.synchronize()
    plan.close()
    note(f"cpu_ref Tier-2 {itype.__name__} cluster={cluster}: {t}")
    ref = oracle.csr_spmm_f64(p.M, p.N, p.rp, p.ci, p.vals, p.B)
    e = rel_frob(host(C), ref)
    assert e <= 1e-5, e
    assert torch.equal(C, Cp)


# ---------------------------------------------------------------------------
# gnn at full size
# ---------------------------------------------------------------------------

@pytest.fixture(scope="module")
def gnn(torch):
    p = synth.gnn()
    note(f"gnn: M={p.M} nnz={p.nnz} N={p.N}")
    perm = X.compute_1d_jaccard_clustering(p.M, p.K, p.rp, p.ci, 0.5, 16)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Ap = X.apply_permutation(A, torch.as_tensor(perm).cuda())
    Bm = X.csr_to_bcsr(Ap)
    B = torch.as_tensor(p.B).cuda()
    torch.cuda.synchronize()
    note(f"gnn: nnzb={Bm.num_blocks}")
    return dict(p=p, perm=perm, A=A, Ap=Ap, Bm=Bm, B=B)


def test_gnn_permutation_and_conversion_bit_exact(torch, gnn):
    p, perm, Ap, Bm = gnn["p"], gnn["perm"], gnn["Ap"], gnn["Bm"]
    assert np.array_equal(np.sort(perm), np.arange(p.M))
    nrp, nci, nv = oracle.apply_perm(p.M, p.rp, p.ci, p.vals, perm)
    np.testing.assert_array_equal(host(Ap.row_ptr).astype(np.int64), nrp)
    np.testing.assert_array_equal(host(Ap.col_ind).astype(np.int64), nci)
    assert np.array_equal(host(Ap.values).view(np.uint16), nv.view(np.uint16))
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, nrp, nci, nv)
    del nrp, nci, nv
    np.testing.assert_array_equal(host(Bm.row_ptr).astype(np.int64), brp)
    np.testing.assert_array_equal(host(Bm.col_ind).astype(np.int64), bci)
    assert np.array_equal(host(Bm.values).view(np.uint16), bv.view(np.uint16))
    note(f"gnn structure bit-exact: nnzb={len(bci)}")


def test_gnn_tier1_truth_and_scaling(torch, gnn):
    p, perm, Bm, B = gnn["p"], gnn["perm"], gnn["Bm"], gnn["B"]
    C = X.spmm(Bm, B)
    C2 = X.spmm(Bm, B * 2)
    torch.cuda.synchronize()
    assert torch.equal(C2, C * 2)
    rows = np.sort(np.random.default_rng(3).choice(p.M, size=512, replace=False))
    # C is in the permuted order: its row r is row perm[r] of A * B
    ref = csr_rows_f64(p.rp, p.ci, p.vals, p.B, perm[rows])
    e = rel_frob(host(C)[rows], ref)
    note(f"gnn Tier-1 sampled rel_frob {e:.3e}")
    assert e <= 1e-5, e
    # the longest block-rows are the ones split or reordered by the launcher
    L = np.diff(host(Bm.row_ptr).astype(np.int64))
    top = np.argsort(L)[-4:]
    trows = np.concatenate([np.arange(16 * b, 16 * b + 16) for b in top])
    ref = csr_rows_f64(p.rp, p.ci, p.vals, p.B, perm[trows])
    e = rel_frob(host(C)[trows], ref)
    note(f"gnn Tier-1 longest block-rows {L[top].tolist()} rel_frob {e:.3e}")
    assert e <= 1e-5, e


def test_gnn_tier1_100_calls_identical(torch, gnn):
    Bm, B = gnn["Bm"], gnn["B"]
    C0 = X.spmm(Bm, B)
    C = torch.empty_like(C0)
    same = 0
    for i in range(100):
        C.fill_(float("nan"))
        X.spmm(Bm, B, C)
        same += int(torch.equal(C, C0))
    torch.cuda.synchronize()
    note(f"gnn: {same}/100 Tier-1 calls equal to the first")
    assert same == 100


def test_gnn_plan_equals_pipeline(torch, gnn):
    p, A, B = gnn["p"], gnn["A"], gnn["B"]
    C_pipe, t = X.spmm_pipeline(A, B, optimize_pattern=True)
    plan = X.SpMMPlan(A)
    C_plan = plan.execute(B)
    C_again = plan.execute(B)
    torch.cuda.synchronize()
    note(f"gnn pipeline {t}; plan prep {plan.timings} packed={plan.packed_batches}")
    plan.close()
    assert torch.equal(C_pipe, C_plan)
    assert torch.equal(C_plan, C_again)
    rows = np.sort(np.random.default_rng(4).choice(p.M, size=512, replace=False))
    e = rel_frob(host(C_pipe)[rows], csr_rows_f64(p.rp, p.ci, p.vals, p.B, rows))
    assert e <= 1e-5, e


# ---------------------------------------------------------------------------
# pruned with clustering on, full size
# ---------------------------------------------------------------------------

def test_pruned_clustered_full_size(torch):
    p = synth.pruned()
    note(f"pruned: M={p.M} K={p.K} N={p.N} nnz={p.nnz}")
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    C_on, t_on = X.spmm_pipeline(A, B, optimize_pattern=True)
    C_off, t_off = X.spmm_pipeline(A, B, optimize_pattern=False)
    plan = X.SpMMPlan(A)
    C_plan = plan.execute(B)
    torch.cuda.synchronize()
    note(f"pruned clustered {t_on}; plain {t_off}; plan clustered={plan.clustered}")
    plan.close()
    # every row meets every block column: one cluster, the reversed order;
    # each C element accumulates the same products in the same K order
    assert torch.equal(C_on, C_off)
    assert torch.equal(C_plan, C_on)
    rows = np.sort(np.random.default_rng(5).choice(p.M, size=256, replace=False))
    e = rel_frob(host(C_on)[rows], csr_rows_f64(p.rp, p.ci, p.vals, p.B, rows))
    note(f"pruned clustered sampled rel_frob {e:.3e}")
    assert e <= 1e-5, e


# ---------------------------------------------------------------------------
# full block grids in a non-canonical layout (GEMM-tiled kernel's check)
# ---------------------------------------------------------------------------

def tile_product_f64(M, K, N, brp, bci, bv, B):
    """Reference tile product of an arbitrary BCSR matrix: each block-row
    sums its blocks in stored order; block columns outside [0, Kb) and B rows
    >= K contribute nothing."""
    Kb = (K + 15) // 16
    Bp = np.zeros((Kb * 16, N), np.float64)
    Bp[:K] = B.astype(np.float64)
    blocks = bv.astype(np.float64).reshape(-1, 16, 16)
    Mb = len(brp) - 1
    C = np.zeros((Mb * 16, N), np.float64)
    for br in range(Mb):
        for b in range(int(brp[br]), int(brp[br + 1])):
            c = int(bci[b])
            if 0 <= c < Kb:
                C[16 * br:16 * br + 16] += blocks[b] @ Bp[16 * c:16 * c + 16]
    return C[:M]


def full_grid(torch, M, K, N, itype, seed):
    rng = np.random.default_rng(seed)
    D = rng.standard_normal((M, K)).astype(np.float16)
    D[rng.random((M, K)) < 0.5] = 0
    for i in range(0, M, 16):
        for j in range(0, K, 16):
            D[i, j] = np.float16(1.0)
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum((D != 0).sum(axis=1))
    ci = np.nonzero(D)[1]
    A = X.CSRMatrix.from_host(M, K, rp.astype(itype), ci.astype(itype), D[D != 0])
    Bm = X.csr_to_bcsr(A)
    assert Bm.num_blocks == Bm.num_block_rows * Bm.num_block_cols
    B = rng.standard_normal((K, N)).astype(np.float16)
    return rng, Bm, B


def run_tier1(torch, Bm, brp, bci, bv, B, M, N):
    itype = Bm.row_ptr.dtype
    Bm.row_ptr = torch.as_tensor(brp).to("cuda", itype)
    Bm.col_ind = torch.as_tensor(bci).to("cuda", itype)
    Bm.values = torch.as_tensor(bv).cuda()
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm(Bm, torch.as_tensor(B).cuda(), C, N)
    torch.cuda.synchronize()
    return host(C)


FULL_SHAPES = [(130, 47, 72), (512, 256, 256), (1000, 96, 264)]


@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("shape", FULL_SHAPES, ids=[f"{m}x{k}xN{n}" for m, k, n in FULL_SHAPES])
def test_full_grid_permuted_block_columns(torch, shape, itype):
    M, K, N = shape
    rng, Bm, B = full_grid(torch, M, K, N, itype, M + K)
    brp = host(Bm.row_ptr).astype(np.int64)
    bci = host(Bm.col_ind).astype(np.int64)
    bv = host(Bm.values).reshape(-1, 256)
    # shuffle the blocks of every other block-row (block columns and values
    # together): the same matrix, stored in another order
    for br in range(0, Bm.num_block_rows, 2):
        a, b = brp[br], brp[br + 1]
        o = a + rng.permutation(b - a)
        bci[a:b], bv[a:b] = bci[o], bv[o]
    C = run_tier1(torch, Bm, brp, bci, bv.reshape(-1), B, M, N)
    ref = tile_product_f64(M, K, N, brp, bci, bv.reshape(-1), B)
    assert np.all(np.isfinite(C))
    e = rel_frob(C, ref)
    note(f"full grid {shape} permuted block columns: rel_frob {e:.3e}")
    assert e <= 1e-5, e


@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_full_grid_uneven_rows_and_outside_columns(torch, itype):
    M, K, N = 512, 256, 128
    rng, Bm, B = full_grid(torch, M, K, N, itype, 77)
    Kb = Bm.num_block_cols
    brp = host(Bm.row_ptr).astype(np.int64)
    bci = host(Bm.col_ind).astype(np.int64)
    bv = host(Bm.values)
    # block-row 3 gives its last block to block-row 2 (which then holds
    # column Kb - 1 twice), and some blocks of block-row 20 point outside
    # the grid: nnzb still equals Mb * Kb
    bci[3 * Kb] = bci[3 * Kb - 1]
    brp[3] += 1
    bad = np.arange(20 * Kb, 21 * Kb)[rng.random(Kb) < 0.3]
    bci[bad] = Kb + rng.integers(0, 100, size=len(bad))
    C = run_tier1(torch, Bm, brp, bci, bv, B, M, N)
    ref = tile_product_f64(M, K, N, brp, bci, bv, B)
    e = rel_frob(C, ref)
    note(f"full grid uneven rows / outside columns: rel_frob {e:.3e}")
    assert np.all(np.isfinite(C))
    assert e <= 1e-5, e


# ---------------------------------------------------------------------------
# operand checks of the Python view (no kernel may run)
# ---------------------------------------------------------------------------

def test_dense_operands_rejected_before_launch(torch):
    p = synth.random_csr(64, 48, 32, 0.2, seed=2)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bm = X.csr_to_bcsr(A)
    B = torch.as_tensor(p.B).cuda()
    sentinel = 12345.0
    C = torch.full((p.M, p.N), sentinel, dtype=torch.float32, device="cuda")
    bad_B = [
        (torch.as_tensor(p.B), ValueError),                       # host tensor
        (B.float(), TypeError),                                   # wrong dtype
        (B[:-1], ValueError),                                     # fewer than K rows
        (torch.as_tensor(p.B.T.copy()).cuda().t(), ValueError),  # transposed view
    ]
    if B.dtype == torch.float16:
        # a contiguous view that starts 2 bytes into its allocation: the
        # kernels read fp16 B rows 16 bytes at a time
        flat = torch.zeros(p.K * p.N + 8, dtype=torch.float16, device="cuda")
        off = flat[1:1 + p.K * p.N].view(p.K, p.N)
        off.copy_(B)
        assert off.is_contiguous() and off.data_ptr() % 16 == 2
        bad_B.append((off, ValueError))
    for b, err in bad_B:
        with pytest.raises(err):
            X.spmm(Bm, b, C, p.N)
        with pytest.raises(err):
            X.spmm_pipeline(A, b, C, p.N)
    bad_C = [
        (torch.zeros((p.M, p.N), dtype=torch.float32), ValueError),         # host
        (torch.zeros((p.M, p.N), dtype=torch.float16, device="cuda"), TypeError),
        (torch.zeros((p.M - 1, p.N), dtype=torch.float32, device="cuda"), ValueError),
        (torch.zeros((p.N, p.M), dtype=torch.float32, device="cuda").t(), ValueError),
    ]
    for c, err in bad_C:
        with pytest.raises(err):
            X.spmm(Bm, B, c, p.N)
        with pytest.raises(err):
            X.spmm_pipeline(A, B, c, p.N)
    plan = X.SpMMPlan(A)
    with pytest.raises(ValueError):
        plan.execute(B[:-1], C, p.N)
    if B.dtype == torch.float16:
        with pytest.raises(ValueError):
            plan.execute(off, C, p.N)
    with pytest.raises(ValueError):
        plan.execute(B, C[:, :-1], p.N)
    plan.close()
    with pytest.raises(ValueError):
        X.unpermute_dense_matrix(C, torch.arange(p.M, device="cuda"), C[:-1])
    with pytest.raises(ValueError):
        X.unpermute_dense_matrix(C, torch.arange(p.M - 1, device="cuda"))
    torch.cuda.synchronize()
    assert bool(torch.all(C == sentinel))


def c_view_off_by_one(torch, M, N):
    """A contiguous M x N fp32 C that starts 4 bytes into its allocation."""
    flat = torch.full((M * N + 4,), float("nan"), dtype=torch.float32, device="cuda")
    C = flat[1:1 + M * N].view(M, N)
    assert C.is_contiguous() and C.data_ptr() % 16 == 4
    return C


@pytest.mark.parametrize("path", ["batch", "dense", "fp32", "pipeline"])
def test_c_off_a_16_byte_boundary(torch, path):
    """C may be any contiguous view; its vector stores fall back to scalar ones
    when C does not start on a 16-byte boundary (same result as an aligned C)."""
    if path == "dense":
        M, K, N = 130, 47, 72
        _, Bm, Bh = full_grid(torch, M, K, N, np.int32, 5)
        A = None
    else:
        dtype = np.float32 if path == "fp32" else np.float16
        p = synth.random_csr(200, 144, 128, 0.05, seed=11, dtype=dtype)
        M, K, N, Bh = p.M, p.K, p.N, p.B
        A = X.CSRMatrix.from_host(M, K, p.rp, p.ci, p.vals)
        Bm = X.csr_to_bcsr(A)
    B = torch.as_tensor(Bh).cuda()
    Ca = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    Cm = c_view_off_by_one(torch, M, N)
    if path == "pipeline":
        X.spmm_pipeline(A, B, Ca, N, optimize_pattern=True, timings=False)
        X.spmm_pipeline(A, B, Cm, N, optimize_pattern=True, timings=False)
    else:
        X.spmm(Bm, B, Ca, N)
        X.spmm(Bm, B, Cm, N)
    torch.cuda.synchronize()
    note(f"C off a 16-byte boundary, {path}: M={M} N={N}")
    assert np.all(np.isfinite(host(Ca)))
    assert np.array_equal(host(Ca), host(Cm))
