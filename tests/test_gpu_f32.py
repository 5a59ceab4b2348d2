"""GPU: the fp32 Tier-1 and Tier-2 paths.

float is the only value type the reference exports
(src/xspmm.cpp:102-114, src/hip/unstructured_mtx_mul.hip:105-106) and every
reference benchmark runs in it, so a drop-in caller lands here.  Two fp32
kernels exist: the column-batch kernel (spmm_f32.hip; the default where
N % 4 == 0 and the grid has at least 512 workgroups) and the tile kernels
(spmm.hip: the short-grid kernel with B through a buffer resource, and with
XSPMM_F32_SHORT=off the one with 64-bit B addressing, which takes B beyond
1 GiB); XSPMM_F32_KERNEL=batch|tile forces a family.  The tests name the
64-bit form "tile64".  Bars:
  * C against the fp64 truth, relative Frobenius <= 1e-5 (the north-star
    tolerance of the fp32 path), for both kernels;
  * the examples/05 density sweep in fp32 (banded 16384^2, N = 128, B = ones):
    every C column equals the fp64 row sum, block count from the band's
    closed form, spmm(2B) == 2 spmm(B) exactly;
  * examples/02 at full size in fp32 (upper triangular 8192^2 at 1 %,
    N = 8192, Tier-2 with clustering on) and the headline templates matrix
    in fp32: sampled rows against fp64, and B = ones against every row sum.
"""
from __future__ import annotations

import contextlib
import os

import numpy as np
import pytest

import oracle
import xspmm_amd as X
from xspmm_amd import synth

pytestmark = pytest.mark.gpu

TOL = 1e-5


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X (torch.cuda.is_available() is False)")
    X.load()
    return torch


KERNEL_ENV = {
    "batch": {"XSPMM_F32_KERNEL": "batch"},
    "tile": {"XSPMM_F32_KERNEL": "tile"},
    "tile64": {"XSPMM_F32_KERNEL": "tile", "XSPMM_F32_SHORT": "off"},
}


@contextlib.contextmanager
def f32_kernel(name):
    env = KERNEL_ENV[name]
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        yield
    finally:
        for k, v in old.items():
            if v is None:
                del os.environ[k]
            else:
                os.environ[k] = v


def note(msg):
    print(msg, flush=True)


def sampled_rows_f64(p, rows, B=None):
    """fp64 product rows of the CSR (row r: sum of vals[j] * B[ci[j], :])."""
    B = p.B if B is None else B
    return np.stack([(p.vals[p.rp[r]:p.rp[r + 1]].astype(np.float64)[:, None]
                      * B[p.ci[p.rp[r]:p.rp[r + 1]]].astype(np.float64)).sum(axis=0)
                     for r in rows])


def run_tier1(torch, p, index=np.int32, kernel=None, B=None):
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp.astype(index), p.ci.astype(index), p.vals)
    Bm = X.csr_to_bcsr(A)
    Bt = torch.as_tensor(np.ascontiguousarray(p.B if B is None else B)).cuda()
    if kernel:
        with f32_kernel(kernel):
            C = X.spmm(Bm, Bt)
    else:
        C = X.spmm(Bm, Bt)
    torch.cuda.synchronize()
    return C.cpu().numpy(), Bm


def truth(p, B=None):
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    return oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, p.B if B is None else B)


# ---------------------------------------------------------------------------
# small shapes, both kernels
# ---------------------------------------------------------------------------

SHAPES = [
    # M, K, N, density, index, unsorted duplicates
    (200, 300, 4, 0.02, np.int32, False),
    (257, 129, 60, 0.05, np.int64, True),
    (512, 512, 64, 0.01, np.int32, False),
    (333, 700, 68, 0.03, np.int32, True),
    (1000, 800, 124, 0.004, np.int64, False),
    (640, 640, 128, 0.2, np.int32, False),
    (500, 1000, 132, 0.01, np.int32, False),
    (300, 260, 192, 0.6, np.int64, False),
    (160, 1600, 260, 0.002, np.int32, True),
]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}x{s[1]}n{s[2]}d{s[3]}" for s in SHAPES])
def test_both_kernels_against_fp64(torch, shape):
    M, K, N, dens, idx, dups = shape
    p = synth.random_csr(M, K, N, dens, seed=M + N, dtype=np.float32, unsorted=dups,
                         dup_frac=0.05 if dups else 0.0)
    ref = truth(p)
    out = {}
    for kern in ("batch", "tile", "tile64"):
        C, Bm = run_tier1(torch, p, idx, kern)
        e = oracle.errors(C, ref)
        note(f"{M}x{K} N={N} d={dens} {np.dtype(idx).name} {kern}: nnzb {Bm.num_blocks} "
             f"rel_frob {e['rel_frob']:.2e}")
        assert np.all(np.isfinite(C))
        assert e["rel_frob"] <= TOL, (kern, e)
        out[kern] = C
    assert oracle.errors(out["batch"], out["tile"])["rel_frob"] <= TOL
    assert oracle.errors(out["tile64"], out["tile"])["rel_frob"] <= TOL


@pytest.mark.parametrize("kern", ["tile", "tile64"])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_tile_invalid_block_columns_and_ragged_edges(torch, itype, kern):
    """Malformed BCSR for the tile kernels: block columns >= Kb (negative ones
    with int32 indices, ones with high bits set with int64) contribute
    nothing, where the reference would read B out of bounds; K = 250 and
    N = 37 leave ragged last block columns and column tiles.  C against the
    fp64 product of the same blocks without the bad ones."""
    p = synth.random_csr(300, 250, 37, 0.05, seed=21, dtype=np.float32)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp.astype(itype), p.ci.astype(itype), p.vals)
    Bm = X.csr_to_bcsr(A)
    bci = Bm.col_ind.cpu().numpy().copy()
    rng = np.random.default_rng(5)
    bad = rng.random(len(bci)) < 0.25
    Kb = Bm.num_block_cols
    bci_bad = bci.copy()
    bci_bad[bad] = Kb + rng.integers(0, 1000, size=int(bad.sum()))
    alt = bad & (rng.random(len(bci)) < 0.5)
    if itype == np.int32:
        bci_bad[alt] = -1 - rng.integers(0, 1 << 20, size=int(alt.sum()))
    else:
        bci_bad[alt] = (np.int64(1) << 40) + bci[alt]
    Bm.col_ind = torch.as_tensor(bci_bad.astype(itype)).cuda()
    with f32_kernel(kern):
        C = X.spmm(Bm, torch.as_tensor(p.B).cuda()).cpu().numpy()
    brp, bci_o, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    assert np.array_equal(bci_o, bci)
    bv = bv.reshape(-1, 256).copy()
    bv[bad] = 0
    ref = oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci_o, bv, p.B)
    e = oracle.errors(C, ref)
    note(f"tile {kern} {np.dtype(itype).name}: {int(bad.sum())} bad of {len(bci)} blocks, "
         f"rel_frob {e['rel_frob']:.2e}")
    assert np.all(np.isfinite(C))
    assert e["rel_frob"] <= TOL, e


def test_batch_is_deterministic_and_linear(torch):
    """Two calls give the same bits, and doubling B doubles C exactly."""
    p = synth.random_csr(700, 900, 128, 0.01, seed=5, dtype=np.float32)
    C1, _ = run_tier1(torch, p, kernel="batch")
    C2, _ = run_tier1(torch, p, kernel="batch")
    C3, _ = run_tier1(torch, p, kernel="batch", B=p.B * 2)
    assert C1.tobytes() == C2.tobytes()
    assert np.array_equal(C3, C1 * 2)


def mixed_blocks(seed=3, M=512, K=1024, N=128):
    """Rows of sparse entries with fully dense 16x16 blocks mixed in, a block
    holding only explicit zeros, and empty block-rows: the batch kernel's full
    blocks take its direct path between open batches."""
    rng = np.random.default_rng(seed)
    D = np.zeros((M, K), np.float32)
    mask = rng.random((M, K)) < 0.01
    D[mask] = rng.uniform(-1, 1, size=int(mask.sum()))
    Mb, Kb = M // 16, K // 16
    for _ in range(60):
        br, bc = int(rng.integers(0, Mb)), int(rng.integers(0, Kb))
        D[16 * br:16 * br + 16, 16 * bc:16 * bc + 16] = rng.uniform(0.5, 1.0, size=(16, 16))
    D[16 * 5:16 * 6, :] = 0.0            # an empty block-row
    D[16 * 7:16 * 8, 16 * 3:16 * 4] = 0.0
    rows, cols = np.nonzero(D)
    vals = D[rows, cols]
    # an all-zero block kept in the structure (explicit zeros)
    rows = np.concatenate([rows, np.arange(16 * 7, 16 * 8)])
    cols = np.concatenate([cols, np.full(16, 16 * 3 + 2)])
    vals = np.concatenate([vals, np.zeros(16, np.float32)])
    order = np.lexsort((cols, rows))
    rows, cols, vals = rows[order], cols[order], vals[order]
    rp = np.zeros(M + 1, np.int64)
    np.cumsum(np.bincount(rows, minlength=M), out=rp[1:])
    B = rng.uniform(-1, 1, size=(K, N)).astype(np.float32)
    return synth.Problem("mixed", M, K, N, rp.astype(np.int32), cols.astype(np.int32),
                         vals.astype(np.float32), B)


@pytest.mark.parametrize("N", [64, 128, 256])
def test_full_blocks_between_sparse_ones(torch, N):
    p = mixed_blocks(N=N)
    ref = truth(p)
    C, Bm = run_tier1(torch, p, kernel="batch")
    e = oracle.errors(C, ref)
    note(f"mixed N={N}: nnzb {Bm.num_blocks} rel_frob {e['rel_frob']:.2e}")
    assert np.all(np.isfinite(C))
    assert e["rel_frob"] <= TOL, e
    assert np.all(C[16 * 5:16 * 6] == 0.0)


def test_nonfinite_a_propagates(torch):
    """An Inf or NaN entry of A reaches its C row as in the fp64 product
    (its column is non-zero, so it is never skipped)."""
    p = synth.random_csr(256, 512, 64, 0.02, seed=11, dtype=np.float32)
    p.B[:] = np.where(p.B == 0, 0.5, p.B)
    p.vals[int(p.rp[10])] = np.inf
    p.vals[int(p.rp[40]) + 1] = np.nan
    ref = sampled_rows_f64(p, np.arange(p.M))
    for kern in ("batch", "tile", "tile64"):
        C, _ = run_tier1(torch, p, kernel=kern)
        assert np.array_equal(np.isnan(C), np.isnan(ref)), kern
        assert np.array_equal(np.isposinf(C), np.isposinf(ref)), kern
        fin = np.isfinite(ref)
        assert np.all(np.isfinite(C[fin])), kern


def zero_column_block(seed=2, M=256, K=512, N=64):
    """Block (0, 1) has non-zero entries in its columns 0..7 only; B row
    16 + 12 (column 12 of that block, all zero in A) is +Inf."""
    rng = np.random.default_rng(seed)
    D = np.zeros((M, K), np.float32)
    D[0:16, 16:24] = rng.uniform(0.5, 1.0, size=(16, 8))
    mask = rng.random((M, K)) < 0.01
    mask[:, 16:32] = False           # block column 1 only in block-row 0
    D[mask] = rng.uniform(-1, 1, size=int(mask.sum()))
    D[:, 28] = 0.0                     # column 28 is zero everywhere
    rows, cols = np.nonzero(D)
    rp = np.zeros(M + 1, np.int64)
    np.cumsum(np.bincount(rows, minlength=M), out=rp[1:])
    B = rng.uniform(-1, 1, size=(K, N)).astype(np.float32)
    Binf = B.copy()
    Binf[28, :] = np.inf
    p = synth.Problem("zerocol", M, K, N, rp.astype(np.int32), cols.astype(np.int32),
                      D[rows, cols].astype(np.float32), B)
    return p, Binf


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_nonfinite_b_in_a_zero_column(torch, dtype):
    """Documented divergence from the reference: the column-batch kernels skip
    block columns that are zero in all 16 rows, so an Inf in a B row that
    meets only such columns leaves C finite and equal to the product with
    that row zeroed; the reference (spmm_math.hpp:93-110) multiplies every
    block column and turns the 16 rows of that block-row into NaN.  The fp32
    tile kernels multiply every block column, as the reference does."""
    p, Binf = zero_column_block()
    if dtype == np.float16:
        p.vals = p.vals.astype(np.float16)
        p.B = p.B.astype(np.float16)
        Binf = Binf.astype(np.float16)
    Bzero = p.B.copy()
    Bzero[28, :] = 0
    C_inf, _ = run_tier1(torch, p, kernel="batch", B=Binf)
    C_zero, _ = run_tier1(torch, p, kernel="batch", B=Bzero)
    assert np.all(np.isfinite(C_inf))
    assert np.array_equal(C_inf, C_zero)
    if dtype == np.float32:
        for kern in ("tile", "tile64"):
            C_tile, _ = run_tier1(torch, p, kernel=kern, B=Binf)
            assert np.all(np.isnan(C_tile[0:16])), kern
            assert np.all(np.isfinite(C_tile[16:])), kern


# ---------------------------------------------------------------------------
# the reference's own fp32 workloads at full size
# ---------------------------------------------------------------------------

def band_blocks(M, bw):
    b = np.arange((M + 15) // 16)
    lo = np.maximum(0, 16 * b - bw) // 16
    hi = np.minimum(M - 1, 16 * b + 15 + bw) // 16
    return int((hi - lo + 1).sum())


@pytest.mark.parametrize("name", list(synth.SWEEP_DENSITIES))
def test_density_sweep_fp32(torch, name):
    """examples/05_core_spmm_benchmark.cpp:25, :57-77, :103-117 as the
    reference runs it: ValueType = float, banded 16384^2, N = 128, B = ones."""
    p = synth.CONFIGS[f"banded{name}_f32"]()
    assert p.vals.dtype == np.float32
    bw = p.meta["bandwidth"]
    note(f"banded {name} % fp32: bandwidth {bw}, nnz {p.nnz}")
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bm = X.csr_to_bcsr(A)
    assert Bm.num_blocks == band_blocks(p.M, bw)
    del A
    B = torch.ones((p.K, p.N), dtype=torch.float32, device="cuda")
    C = X.spmm(Bm, B)
    C2 = X.spmm(Bm, B * 2)
    torch.cuda.synchronize()
    assert torch.equal(C2, C * 2)
    rs = np.add.reduceat(p.vals.astype(np.float64), p.rp[:-1].astype(np.int64))
    Ch = C.cpu().numpy()
    assert np.all(np.isfinite(Ch))
    e = oracle.errors(Ch, np.repeat(rs[:, None], p.N, axis=1))
    note(f"  nnzb {Bm.num_blocks}: rel_frob {e['rel_frob']:.3e}")
    assert e["rel_frob"] <= TOL, e


def test_examples02_triangular_tier2_fp32(torch):
    """examples/02_spmm_benchmark.cpp:60-61, :121-124, :268-269: the Tier-2
    pipeline with clustering on, fp32, upper triangular 8192^2 at 1 %,
    N = 8192.  Sampled rows of C against fp64, and B = ones against every
    row sum."""
    p = synth.triangular(8192, 0.01)
    note(f"triangular 8192^2 1 %: nnz {p.nnz}, N {p.N}")
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    C, t = X.spmm_pipeline(A, B, optimize_pattern=True)
    torch.cuda.synchronize()
    note(f"  stages {t}")
    rows = np.random.default_rng(1).choice(p.M, size=256, replace=False)
    Cs = C[torch.as_tensor(rows).cuda()].cpu().numpy()
    e = oracle.errors(Cs, sampled_rows_f64(p, rows))
    note(f"  sampled rows rel_frob {e['rel_frob']:.2e}")
    assert np.all(np.isfinite(Cs))
    assert e["rel_frob"] <= TOL, e
    del B, C
    ones = torch.ones((p.K, 64), dtype=torch.float32, device="cuda")
    C1, _ = X.spmm_pipeline(A, ones, optimize_pattern=True, timings=False)
    torch.cuda.synchronize()
    rs = np.add.reduceat(p.vals.astype(np.float64), p.rp[:-1].astype(np.int64))
    e = oracle.errors(C1.cpu().numpy(), np.repeat(rs[:, None], 64, axis=1))
    note(f"  row sums rel_frob {e['rel_frob']:.2e}")
    assert e["rel_frob"] <= TOL, e


def test_templates_fp32_tier1_and_tier2(torch):
    """The headline matrix in fp32 (the reference's type): Tier-1 on the
    clustered BCSR and the Tier-2 pipeline, sampled rows against fp64.  The
    pipeline's BCSR form (XSPMM_PIPELINE_FORMAT=bcsr) multiplies the same
    BCSR and must agree exactly; its default packed fp32 form sums the same
    products in another order (relative difference <= 1e-6)."""
    p = synth.templates(dtype=np.float32)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()
    perm = X.compute_1d_jaccard_clustering(p.M, p.K, p.rp, p.ci, 0.5, 16)
    Ap = X.apply_permutation(A, torch.as_tensor(perm).cuda())
    Bm = X.csr_to_bcsr(Ap)
    C1 = X.spmm(Bm, B)
    Cp, _ = X.spmm_pipeline(A, B, optimize_pattern=True, timings=False)
    torch.cuda.synchronize()
    assert X.pipeline_last_packed()
    os.environ["XSPMM_PIPELINE_FORMAT"] = "bcsr"
    try:
        C2, _ = X.spmm_pipeline(A, B, optimize_pattern=True, timings=False)
        torch.cuda.synchronize()
    finally:
        del os.environ["XSPMM_PIPELINE_FORMAT"]
    d = float((Cp.double() - C2.double()).norm() / C2.double().norm())
    note(f"templates fp32: packed pipeline against the BCSR form, relative {d:.2e}")
    assert d <= 1e-6
    note(f"templates fp32: nnzb {Bm.num_blocks}")
    rows = np.random.default_rng(2).choice(p.M, size=512, replace=False)
    # C1 is in the permuted row order: its row r is row perm[r] of A * B
    e = oracle.errors(C1.cpu().numpy()[rows], sampled_rows_f64(p, perm[rows]))
    note(f"  Tier-1 sampled rows rel_frob {e['rel_frob']:.2e}")
    assert e["rel_frob"] <= TOL, e
    C1u = torch.empty_like(C1)
    C1u[torch.as_tensor(perm.astype(np.int64)).cuda()] = C1
    assert torch.equal(C1u, C2)
