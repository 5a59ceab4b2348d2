"""GPU parity: every HIP kernel against the oracle on the same seeded inputs.

Bars:
  * structure (BCSR row_ptr / col_ind / values, permuted CSR, permutations,
    un-permuted C) -- bit-exact;
  * C of the SpMM -- relative Frobenius error against the fp64 truth
    <= 2e-3 for fp16 inputs and <= 1e-5 for fp32 inputs (the stated
    tolerances), and additionally <= 1e-5 for fp16 (fp32 accumulation of
    exact fp16 products leaves far less than the stated bound).
All calls go through the C ABI of libxspmm.so (xspmm_amd is its ctypes view).
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
import xspmm_amd as X
from tests.helpers import dense_last_wins, golden_cases, widen
from xspmm_amd import synth

pytestmark = pytest.mark.gpu

TOL = {np.float16: 2e-3, np.float32: 1e-5}
TIGHT = 1e-5


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X (torch.cuda.is_available() is False)")
    X.load()
    return torch


def dev(torch, a):
    return torch.as_tensor(np.ascontiguousarray(a)).cuda()


def host(t):
    return t.detach().cpu().numpy()


def note(msg):
    print(msg, flush=True)


def check_c(C, ref, dtype):
    e = oracle.errors(C, ref)
    assert np.all(np.isfinite(C))
    assert e["rel_frob"] <= TOL[dtype], e
    assert e["rel_frob"] <= TIGHT, e
    return e


# ---------------------------------------------------------------------------
# CSR -> BCSR
# ---------------------------------------------------------------------------

CONV = golden_cases("conversion")


@pytest.mark.parametrize("case", CONV, ids=[c["name"] for c in CONV])
def test_conversion_golden(torch, case):
    M, K, rb, cb = int(case["M"]), int(case["K"]), int(case["rb"]), int(case["cb"])
    note(f"conversion golden {case['name']} M={M} K={K} r={rb} c={cb}")
    A = X.CSRMatrix.from_host(M, K, case["rp"], case["ci"], case["vals"])
    Bm = X.csr_to_bcsr(A, rb, cb)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(widen(host(Bm.row_ptr)), widen(case["brp"]))
    np.testing.assert_array_equal(widen(host(Bm.col_ind)), widen(case["bci"]))
    got = host(Bm.values).astype(np.float32)
    assert got.view(np.uint32).tobytes() == case["bvals"].astype(np.float32).view(np.uint32).tobytes()


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("seed", range(4))
def test_conversion_random(torch, dtype, itype, seed):
    rng = np.random.default_rng(seed)
    M, K = int(rng.integers(1, 400)), int(rng.integers(1, 3000))
    rb, cb = [(16, 16), (16, 16), (4, 8), (3, 5)][seed]
    p = synth.random_csr(M, K, 4, float(rng.uniform(0.002, 0.05)), seed=seed, dtype=dtype,
                         unsorted=seed >= 2, dup_frac=0.2 if seed == 3 else 0.0)
    note(f"conversion random seed={seed} {dtype.__name__} {itype.__name__} M={M} K={K}")
    rp, ci = p.rp.astype(itype), p.ci.astype(itype)
    A = X.CSRMatrix.from_host(M, K, rp, ci, p.vals)
    Bm = X.csr_to_bcsr(A, rb, cb)
    want = oracle.csr_to_bcsr(M, K, rp, ci, p.vals, rb, cb)
    torch.cuda.synchronize()
    assert Bm.row_ptr.dtype == A.row_ptr.dtype
    np.testing.assert_array_equal(widen(host(Bm.row_ptr)), want[0])
    np.testing.assert_array_equal(widen(host(Bm.col_ind)), want[1])
    assert host(Bm.values).tobytes() == want[2].tobytes()


def test_conversion_rejects_bad_columns(torch):
    A = X.CSRMatrix.from_host(2, 10, np.array([0, 1, 2], np.int32), np.array([3, 10], np.int32),
                              np.ones(2, np.float32))
    with pytest.raises(X.XspmmInvalidArgument):
        X.csr_to_bcsr(A)
    A = X.CSRMatrix.from_host(2, 10, np.array([0, 1, 2], np.int32), np.array([-1, 2], np.int32),
                              np.ones(2, np.float32))
    with pytest.raises(X.XspmmInvalidArgument):
        X.csr_to_bcsr(A)


# ---------------------------------------------------------------------------
# Tier-1 SpMM
# ---------------------------------------------------------------------------

SHAPES = [(16, 16, 16), (17, 33, 5), (100, 77, 31), (256, 512, 128), (1, 1, 1), (64, 40, 300),
          (300, 200, 64), (48, 48, 17)]


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("shape", SHAPES, ids=[f"{m}x{k}xN{n}" for m, k, n in SHAPES])
def test_spmm_tier1_random(torch, dtype, itype, shape):
    M, K, N = shape
    p = synth.random_csr(M, K, N, 0.05, seed=M * 7 + K + N, dtype=dtype, unsorted=True,
                         dup_frac=0.05)
    note(f"tier1 {dtype.__name__} {itype.__name__} M={M} K={K} N={N}")
    A = X.CSRMatrix.from_host(M, K, p.rp.astype(itype), p.ci.astype(itype), p.vals)
    Bm = X.csr_to_bcsr(A)
    Bd = dev(torch, p.B)
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm(Bm, Bd, C, N)
    torch.cuda.synchronize()
    brp, bci, bv = oracle.csr_to_bcsr(M, K, p.rp, p.ci, p.vals)
    ref = oracle.bcsr_spmm_f64(M, K, N, brp, bci, bv, p.B)
    check_c(host(C), ref, dtype)


@pytest.mark.parametrize("N", [1, 2, 4, 8, 17, 18, 24, 30, 31, 128])
def test_spmm_ragged_n_banded(torch, N):
    # examples/06_bad_col_lengths.cpp: banded matrix, B = ones, ragged N
    p = synth.banded(M=512, bandwidth=20, N=N, dtype=np.float32)
    for dtype in (np.float32, np.float16):
        note(f"ragged N={N} {dtype.__name__}")
        A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals.astype(dtype))
        Bm = X.csr_to_bcsr(A)
        C = X.spmm(Bm, dev(torch, p.B.astype(dtype)), N=N)
        torch.cuda.synchronize()
        rs = np.add.reduceat(p.vals.astype(dtype).astype(np.float64), p.rp[:-1])
        check_c(host(C), np.repeat(rs[:, None], N, axis=1), dtype)


# The launcher picks 14- or 16-block-row tiles by how the grid fills the CUs.
# On a 256-CU MI355X the small shapes (one round) take 14-row tiles; 16384 x 48
# x 2048 (1024 block-rows, 8 column groups: 512 tiles of 16 = two full rounds)
# takes 16-row tiles; 14300 x 40 x 2048 (894 block-rows: 448 tiles of 16 against
# 512 of 14) takes 14-row tiles with a ragged last row group (12 of 14 rows).
DENSE_SHAPES = [(16, 16, 8), (128, 64, 256), (130, 47, 72), (256, 512, 264), (300, 33, 520),
                (48, 160, 16), (16384, 48, 2048), (14300, 40, 2048)]


@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("shape", DENSE_SHAPES, ids=[f"{m}x{k}xN{n}" for m, k, n in DENSE_SHAPES])
def test_spmm_full_block_grid(torch, shape, itype):
    # every 16x16 block present (nnzb == Mb * Kb): the GEMM-tiled fp16 kernel;
    # ragged M and K, odd Kb, N not a multiple of the 256-column tile
    M, K, N = shape
    rng = np.random.default_rng(M + K + N)
    D = rng.standard_normal((M, K)).astype(np.float16)
    D[rng.random((M, K)) < 0.5] = 0
    for i in range(0, M, 16):                # at least one entry per block
        for j in range(0, K, 16):
            D[i, j] = np.float16(1.0)
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum((D != 0).sum(axis=1))
    ci = np.nonzero(D)[1].astype(itype)
    vals = D[D != 0]
    B = rng.standard_normal((K, N)).astype(np.float16)
    note(f"full block grid M={M} K={K} N={N} {itype.__name__}")
    A = X.CSRMatrix.from_host(M, K, rp.astype(itype), ci, vals)
    Bm = X.csr_to_bcsr(A)
    assert Bm.num_blocks == Bm.num_block_rows * Bm.num_block_cols
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm(Bm, dev(torch, B), C, N)
    torch.cuda.synchronize()
    check_c(host(C), D.astype(np.float64) @ B.astype(np.float64), np.float16)


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
def test_spmm_b_beyond_32_bit_offsets(torch, dtype):
    # B of more than 2^31 bytes (K * N * sizeof(T) > 2^31): the fp16
    # column-batch kernel's 32-bit byte offsets do not apply, and the launcher
    # must take a 64-bit path (fp16 panel kernel, fp32 kernel).  Rows touch
    # the first and the last column of K, so the largest offsets are read.
    K = 65536
    N = 16392 if dtype == np.float16 else 8200
    assert K * N * np.dtype(dtype).itemsize > 2 ** 31
    M = 40
    rng = np.random.default_rng(31)
    rows = []
    for r in range(M):
        c = rng.choice(K, size=6, replace=False)
        c = np.concatenate([c, [0, K - 1] if r % 3 == 0 else [K - 1 - r]])
        rows.append(np.unique(c))
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum([len(c) for c in rows])
    ci = np.concatenate(rows).astype(np.int32)
    vals = rng.uniform(-1, 1, len(ci)).astype(dtype)
    note(f"B beyond 2^31 bytes: K={K} N={N} {dtype.__name__}")
    A = X.CSRMatrix.from_host(M, K, rp.astype(np.int32), ci, vals)
    Bm = X.csr_to_bcsr(A)
    tdt = torch.float16 if dtype == np.float16 else torch.float32
    gen = torch.Generator(device="cuda").manual_seed(7)
    Bd = torch.randn(K, N, generator=gen, dtype=torch.float32, device="cuda").to(tdt)
    C = X.spmm(Bm, Bd, N=N)
    # the prepared product (clustered: the un-permuted store through a workspace)
    plan = X.SpMMPlan(A)
    Cp = plan.execute(Bd)
    torch.cuda.synchronize()
    plan.close()
    used, ci_sub = np.unique(ci, return_inverse=True)
    Bsub = host(Bd[torch.as_tensor(used).long().cuda()]).astype(np.float64)
    del Bd
    ref = oracle.csr_spmm_f64(M, N, rp, ci_sub.astype(np.int64), vals, Bsub)
    check_c(host(C), ref, dtype)
    check_c(host(Cp), ref, dtype)


@pytest.mark.parametrize("N", [64, 128])
def test_spmm_many_skewed_block_rows(torch, N):
    # Mb = 3000 > 2048 block-rows with power-law lengths: the launcher orders
    # rows longest-first before the column-batch kernel
    rng = np.random.default_rng(N)
    M, K = 48000, 4096
    deg = np.minimum((rng.pareto(1.2, M) + 1) * 3, K).astype(np.int64)
    rows = [np.sort(rng.choice(K, size=d, replace=False)) for d in deg]
    rp = np.zeros(M + 1, np.int64); rp[1:] = np.cumsum(deg)
    ci = np.concatenate(rows).astype(np.int32)
    vals = rng.uniform(-1, 1, len(ci)).astype(np.float16)
    B = rng.standard_normal((K, N)).astype(np.float16)
    note(f"skewed rows M={M} nnz={len(ci)} N={N}")
    A = X.CSRMatrix.from_host(M, K, rp.astype(np.int32), ci, vals)
    Bm = X.csr_to_bcsr(A)
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm(Bm, dev(torch, B), C, N)
    torch.cuda.synchronize()
    ref = oracle.csr_spmm_f64(M, N, rp, ci, vals, B)
    check_c(host(C), ref, np.float16)


def xcd_ranges(Mb):
    """Workgroup i -> block-row start[i % 8] + i / 8 (XCD x: a contiguous range)."""
    counts = np.array([(Mb - x + 7) // 8 for x in range(8)])
    start = np.concatenate([[0], np.cumsum(counts)])[:-1]
    i = np.arange(Mb)
    return start[i % 8] + i // 8


@pytest.mark.parametrize("case", ["band", "random_blocks", "long_rows", "short_grid"])
def test_spmm_locality_order(torch, case):
    """Grids of 256 .. 2048 block-rows: csr_to_bcsr keeps an order computed
    from the block columns -- contiguous block-row ranges per XCD for short,
    alike neighbouring rows (a narrow band) -- and none for unrelated
    neighbours (random dense blocks), long rows (a wide band) or fewer than
    256 block-rows.  C of the ordered call equals the unordered entry point's
    bit for bit; where the grid takes the band kernel (contiguous block-rows),
    the Python Tier-1 call equals the band entry point's C."""
    import ctypes as C
    if case == "band":
        p = synth.banded_sweep(0.01, M=8192, N=64)          # 512 block-rows, ~6 blocks each
        expect = "xcd"
    elif case == "random_blocks":
        p = synth.blocks(M=8192, N=64)                      # 512 block-rows of random blocks
        expect = "identity"
    elif case == "long_rows":
        p = synth.banded_sweep(0.5, M=8192, N=64)           # ~256 blocks per block-row
        expect = "identity"
    else:
        p = synth.banded_sweep(0.01, M=2048, N=64)          # 128 block-rows
        expect = None
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    Bm = X.csr_to_bcsr(A)
    Mb = Bm.num_block_rows
    order = Bm.dispatch_order()
    if expect == "xcd":
        o = host(order).astype(np.int64)
        assert np.array_equal(o, xcd_ranges(Mb)), (case, o[:16])
    else:
        assert order is None  # the identity (or a short grid): no order passed
    B = dev(torch, np.random.default_rng(3).uniform(-1, 1, (p.K, p.N)).astype(p.vals.dtype))
    L = X.load()
    ptr = lambda t: C.c_void_p(t.data_ptr())
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    C1 = torch.full((p.M, p.N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.xspmm_bcsr_spmm_ordered(X.vcode(Bm.values.dtype), X.icode(Bm.row_ptr.dtype), Bm.num_rows,
                                     Bm.num_cols, Mb, Bm.num_block_cols, Bm.num_blocks,
                                     ptr(Bm.row_ptr), ptr(Bm.col_ind), ptr(Bm.values), ptr(B), ptr(C1),
                                     p.N, ptr(order) if order is not None else None, stream) == X.OK
    if Bm.band_rows():
        C3 = torch.full((p.M, p.N), float("nan"), dtype=torch.float32, device="cuda")
        assert L.xspmm_bcsr_spmm_band(X.vcode(Bm.values.dtype), X.icode(Bm.row_ptr.dtype), Bm.num_rows,
                                      Bm.num_cols, Mb,
                                      Bm.num_block_cols, Bm.num_blocks, ptr(Bm.row_ptr),
                                      ptr(Bm.col_ind), ptr(Bm.values), ptr(B), ptr(C3), p.N,
                                      stream) == X.OK
        assert torch.equal(X.spmm(Bm, B), C3)
        check_c(host(C3), host(C1).astype(np.float64), np.float16)
    else:
        assert torch.equal(X.spmm(Bm, B), C1)
    C2 = torch.full((p.M, p.N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.xspmm_bcsr_spmm(X.vcode(Bm.values.dtype), X.icode(Bm.row_ptr.dtype), Bm.num_rows,
                             Bm.num_cols, Mb, Bm.num_block_cols, Bm.num_blocks, ptr(Bm.row_ptr),
                             ptr(Bm.col_ind), ptr(Bm.values), ptr(B), ptr(C2), p.N, stream) == X.OK
    torch.cuda.synchronize()
    assert torch.equal(C1, C2)


@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_spmm_cached_dispatch_order(torch, itype):
    # Mb = 3000 > 2048: csr_to_bcsr keeps the longest-first dispatch order and
    # Tier-1 passes it (xspmm_bcsr_spmm_ordered); C equals the C of the entry
    # point that orders the rows on every call, bit for bit.  An order whose
    # ids fall outside the grid skips those block-rows (their C rows stay as
    # they were), and an in-place change of row_ptr makes the view recompute it.
    import ctypes as C
    rng = np.random.default_rng(5)
    M, K, N = 48000, 4096, 64
    deg = np.minimum((rng.pareto(1.2, M) + 1) * 3, K).astype(np.int64)
    rows = [np.sort(rng.choice(K, size=d, replace=False)) for d in deg]
    rp = np.zeros(M + 1, np.int64); rp[1:] = np.cumsum(deg)
    ci = np.concatenate(rows)
    vals = rng.uniform(-1, 1, len(ci)).astype(np.float16)
    A = X.CSRMatrix.from_host(M, K, rp.astype(itype), ci.astype(itype), vals)
    Bm = X.csr_to_bcsr(A)
    order = Bm._order
    assert order is not None and order.dtype == torch.int32
    assert np.array_equal(np.sort(host(order)), np.arange(Bm.num_block_rows))
    B = dev(torch, rng.standard_normal((K, N)).astype(np.float16))
    C1 = X.spmm(Bm, B)
    L = X.load()
    ptr = lambda t: C.c_void_p(t.data_ptr())
    stream = C.c_void_p(torch.cuda.current_stream().cuda_stream)
    args = (X.vcode(Bm.values.dtype), X.icode(Bm.row_ptr.dtype), Bm.num_rows, Bm.num_cols,
            Bm.num_block_rows, Bm.num_block_cols, Bm.num_blocks, ptr(Bm.row_ptr),
            ptr(Bm.col_ind), ptr(Bm.values), ptr(B))
    C2 = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.xspmm_bcsr_spmm(*args, ptr(C2), N, stream) == X.OK
    torch.cuda.synchronize()
    assert torch.equal(C1, C2)
    # ids outside [0, Mb) are skipped
    bad = order.clone()
    skipped = host(bad[:5]).copy()
    bad[:5] = Bm.num_block_rows + 7
    C3 = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    assert L.xspmm_bcsr_spmm_ordered(*args, ptr(C3), N, ptr(bad), stream) == X.OK
    torch.cuda.synchronize()
    lost = np.zeros(M, bool)
    for br in skipped:
        lost[16 * br:16 * br + 16] = True
    C3h = host(C3)
    assert np.all(np.isnan(C3h[lost]))
    assert np.array_equal(C3h[~lost], host(C1)[~lost])
    # an in-place change of row_ptr: the cached order is recomputed
    key = Bm._order_key
    Bm.row_ptr.add_(0)
    assert Bm.dispatch_order() is not None and Bm._order_key != key
    C4 = X.spmm(Bm, B)
    torch.cuda.synchronize()
    assert torch.equal(C4, C1)
    ref = oracle.csr_spmm_f64(M, N, rp, ci, vals, host(B))
    check_c(host(C1), ref, np.float16)


def test_spmm_empty_and_odd_block_rows(torch):
    # block-rows with 0, 1, 2, 3 blocks; C must be overwritten (zeros where empty)
    rows = []
    for r in range(64):
        strip = r // 16
        rows.append(np.arange(strip) * 16 + (r % 16))  # strip s has s blocks
    lens = [len(x) for x in rows]
    rp = np.zeros(65, np.int32); rp[1:] = np.cumsum(lens)
    ci = np.concatenate(rows).astype(np.int32)
    vals = np.random.default_rng(0).uniform(-1, 1, len(ci)).astype(np.float16)
    B = np.random.default_rng(1).uniform(-1, 1, (64, 48)).astype(np.float16)
    A = X.CSRMatrix.from_host(64, 64, rp, ci, vals)
    Bm = X.csr_to_bcsr(A)
    assert list(host(Bm.row_ptr)) == [0, 0, 1, 3, 6]
    C = torch.full((64, 48), 7.0, dtype=torch.float32, device="cuda")
    X.spmm(Bm, dev(torch, B), C)
    torch.cuda.synchronize()
    Ch = host(C)
    assert np.all(Ch[:16] == 0)
    ref = dense_last_wins(64, 64, rp, ci, vals) @ B.astype(np.float64)
    check_c(Ch, ref, np.float16)


def test_spmm_no_blocks_gives_zeros(torch):
    A = X.CSRMatrix.from_host(40, 40, np.zeros(41, np.int32), np.zeros(0, np.int32),
                              np.zeros(0, np.float16))
    Bm = X.csr_to_bcsr(A)
    assert Bm.num_blocks == 0
    C = torch.full((40, 20), 3.0, dtype=torch.float32, device="cuda")
    X.spmm(Bm, dev(torch, np.ones((40, 20), np.float16)), C)
    torch.cuda.synchronize()
    assert np.all(host(C) == 0)


def test_spmm_checkers_closed_form(torch):
    # examples/01_uspmm_checkers.cpp: shuffled checkers, B = ones -> row sums
    for dtype in (np.float32, np.float16):
        p = synth.checkers(M=512, K=512, N=64, bs=4, dtype=dtype)
        note(f"checkers {dtype.__name__}")
        A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
        C = X.spmm(X.csr_to_bcsr(A), dev(torch, p.B))
        torch.cuda.synchronize()
        rs = np.add.reduceat(p.vals.astype(np.float64), p.rp[:-1])
        check_c(host(C), np.repeat(rs[:, None], p.N, axis=1), dtype)


# ---------------------------------------------------------------------------
# permutation / un-permutation
# ---------------------------------------------------------------------------

PERM = golden_cases("permutation")


@pytest.mark.parametrize("case", PERM, ids=[c["name"] for c in PERM])
def test_apply_permutation_golden(torch, case):
    M = int(case["M"])
    A = X.CSRMatrix.from_host(M, int(case["K"]), case["rp"], case["ci"], case["vals"])
    P = X.apply_permutation(A, dev(torch, case["perm"]))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(widen(host(P.row_ptr)), widen(case["nrp"]))
    np.testing.assert_array_equal(widen(host(P.col_ind)), widen(case["nci"]))
    np.testing.assert_array_equal(host(P.values), case["nvals"])


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("M", [1, 255, 256, 257, 5000])
def test_apply_permutation_random(torch, dtype, itype, M):
    p = synth.random_csr(M, 300, 4, 0.02, seed=M, dtype=dtype)
    perm = np.random.default_rng(M).permutation(M).astype(itype)
    A = X.CSRMatrix.from_host(M, 300, p.rp.astype(itype), p.ci.astype(itype), p.vals)
    P = X.apply_permutation(A, dev(torch, perm))
    want = oracle.apply_perm(M, p.rp, p.ci, p.vals, perm)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(widen(host(P.row_ptr)), want[0])
    np.testing.assert_array_equal(widen(host(P.col_ind)), want[1])
    assert host(P.values).tobytes() == want[2].tobytes()


@pytest.mark.parametrize("N", [1, 3, 4, 64, 128, 1000, 1028])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_unpermute(torch, N, itype):
    M = 333
    rng = np.random.default_rng(N)
    Xh = rng.standard_normal((M, N)).astype(np.float32)
    perm = rng.permutation(M).astype(itype)
    out = X.unpermute_dense_matrix(dev(torch, Xh), dev(torch, perm))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(host(out), oracle.unpermute(M, N, Xh, perm))


# ---------------------------------------------------------------------------
# Tier-2 pipeline
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("cluster", [True, False])
@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_pipeline_matches_oracle_chain(torch, cluster, dtype, itype):
    p = synth.templates(M=1024, n_templates=64, tcols=40, seed=3, N=96)
    vals = p.vals.astype(dtype)
    B = p.B.astype(dtype)
    note(f"pipeline cluster={cluster} {dtype.__name__} {itype.__name__}")
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp.astype(itype), p.ci.astype(itype), vals)
    C, t = X.spmm_pipeline(A, dev(torch, B), optimize_pattern=cluster)
    torch.cuda.synchronize()
    # oracle chain of the same stages
    if cluster:
        perm = oracle.jaccard(p.M, p.K, p.rp, p.ci, 0.5, 16)
        nrp, nci, nv = oracle.apply_perm(p.M, p.rp, p.ci, vals, perm)
    else:
        perm = np.arange(p.M)
        nrp, nci, nv = p.rp, p.ci, vals
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, nrp, nci, nv)
    Cp = oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, B)
    ref = np.zeros_like(Cp)
    ref[perm] = Cp
    check_c(host(C), ref, dtype)
    truth = oracle.csr_spmm_f64(p.M, p.N, p.rp, p.ci, vals, B)
    check_c(host(C), truth, dtype)
    assert t["total_pipeline_ms"] > 0 and t["spmm_ms"] > 0 and t["conversion_ms"] > 0
    if cluster:
        assert t["clustering_ms"] > 0 and t["permutation_ms"] > 0
    else:
        assert t["clustering_ms"] == 0 and t["permutation_ms"] == 0


def test_pipeline_checkers_clustered(torch):
    p = synth.checkers(M=1024, K=1024, N=128, bs=4, dtype=np.float32)
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp, p.ci, p.vals)
    C, _ = X.spmm_pipeline(A, dev(torch, p.B), optimize_pattern=True)
    torch.cuda.synchronize()
    rs = np.add.reduceat(p.vals.astype(np.float64), p.rp[:-1])
    Ch = host(C)
    assert np.max(np.abs(Ch - rs[:, None])) < 1e-3  # the reference example's abs tolerance
    check_c(Ch, np.repeat(rs[:, None], p.N, axis=1), np.float32)
