"""GPU parity of the band kernels (xspmm_bcsr_spmm_band: spmm_f16_band_kernel
and spmm_f32_band_kernel) and of the check that selects them
(xspmm_bcsr_band_rows).

The band kernels multiply grids whose block-rows are contiguous runs of block
columns, four neighbouring block-rows per workgroup sharing each B tile (fp16,
through LDS) or each B load (fp32, in registers); the density sweep of the
reference (examples/05_core_spmm_benchmark.cpp:56-77, banded matrices) is of
this shape.  Bars, for fp16 and fp32 values:
  * integer-valued A and B keep every fp32 partial sum exact, so C must equal
    the fp64 product bit for bit (a row, column or pair mix-up cannot hide in
    a tolerance);
  * random values: relative Frobenius error <= 1e-5 against the fp64 BCSR
    product of the oracle (oracle.bcsr_spmm_f64), on the same BCSR arrays;
  * shapes: ragged M, K and N, groups of four block-rows cut by the grid's
    end, empty block-rows and whole empty groups, single block-rows, int32
    and int64 indices, N from 8 to 264 (one to three 128-column chunks);
  * an Inf in B that meets a zero column of a present block gives NaN, as the
    reference's tile product (src/common/spmm_math.hpp:93-110) does, and
    never reaches a row that does not hold that block;
  * the selection: bands and shifted bands take the kernel (fp32 from 16
    blocks per block-row); a grid with a gap in a block-row, a random sparse
    grid and a fully populated grid do not.
All calls go through the C ABI.
"""
from __future__ import annotations

import ctypes

import numpy as np
import pytest

import oracle
import xspmm_amd as X

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


DTYPES = [np.float16, np.float32]


def band_csr(M, K, bw, shift=0, empty_every=0, rng=None, integer=False, dtype=np.float16):
    """Rows i: columns max(0, i + shift - bw) .. min(K - 1, i + shift + bw);
    block-rows b with b % empty_every == 1 left empty."""
    rows = []
    for i in range(M):
        if empty_every and (i // 16) % empty_every == 1:
            rows.append(np.zeros(0, np.int64))
            continue
        c = i + shift
        lo, hi = max(0, c - bw), min(K - 1, c + bw)
        rows.append(np.arange(lo, hi + 1) if hi >= lo else np.zeros(0, np.int64))
    lens = np.array([len(r) for r in rows], np.int64)
    rp = np.zeros(M + 1, np.int64)
    np.cumsum(lens, out=rp[1:])
    ci = np.concatenate(rows) if rp[-1] else np.zeros(0, np.int64)
    if integer:
        vals = rng.integers(-3, 4, size=len(ci)).astype(dtype)
    else:
        vals = rng.standard_normal(len(ci)).astype(dtype)
    return rp, ci, vals


def device_bcsr(torch, M, K, rp, ci, vals, itype):
    A = X.CSRMatrix.from_host(M, K, rp.astype(itype), ci.astype(itype), vals)
    return X.csr_to_bcsr(A)


def band_rows(Bm, nnz):
    band = ctypes.c_int(-1)
    X._check(X.load().xspmm_bcsr_band_rows(X.vcode(Bm.values.dtype), X.icode(Bm.row_ptr.dtype),
                                           Bm.num_rows, Bm.num_cols,
                                           Bm.num_block_rows, Bm.num_block_cols, nnz, Bm.num_blocks,
                                           X._ptr(Bm.row_ptr), X._ptr(Bm.col_ind), ctypes.byref(band),
                                           X._stream()))
    return band.value


def spmm_band(torch, Bm, B):
    N = int(B.shape[1])
    C = torch.full((Bm.num_rows, N), float("nan"), dtype=torch.float32, device="cuda")
    X._check(X.load().xspmm_bcsr_spmm_band(X.vcode(B.dtype), X.icode(Bm.row_ptr.dtype),
                                           Bm.num_rows, Bm.num_cols,
                                           Bm.num_block_rows, Bm.num_block_cols, Bm.num_blocks,
                                           X._ptr(Bm.row_ptr), X._ptr(Bm.col_ind), X._ptr(Bm.values),
                                           X._ptr(B), X._ptr(C), N, X._stream()))
    torch.cuda.synchronize()
    return C


def host_bcsr(Bm):
    return (Bm.row_ptr.cpu().numpy().astype(np.int64), Bm.col_ind.cpu().numpy().astype(np.int64),
            Bm.values.cpu().numpy())


# (M, K, bandwidth, shift, empty block-rows every, N, index type)
CASES = [
    (1000, 1100, 40, 0, 0, 8, np.int32),
    (1000, 1100, 40, 37, 0, 136, np.int64),
    (333, 2000, 17, 5, 0, 264, np.int32),
    (64, 64, 5, 0, 0, 72, np.int32),
    (80, 4000, 2000, 0, 0, 128, np.int32),
    (2048, 2048, 64, 0, 3, 256, np.int64),
    (16, 48, 100, 0, 0, 16, np.int32),       # one block-row
    (100, 1000, 3, 950, 0, 40, np.int32),    # rows past K: the last block-rows empty
    (4096, 4096, 1000, 0, 0, 128, np.int32),
    (1030, 1030, 30, 0, 4, 24, np.int64),    # whole groups of four empty, a cut last group
]


def case_id(c):
    M, K, bw, sh, ee, N, it = c
    return f"M{M}_K{K}_bw{bw}_s{sh}_e{ee}_N{N}_{np.dtype(it).name}"


@pytest.mark.parametrize("dtype", DTYPES, ids=["f16", "f32"])
@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_band_integer_exact(torch, case, dtype):
    M, K, bw, shift, ee, N, itype = case
    rng = np.random.default_rng(M + K + N)
    rp, ci, vals = band_csr(M, K, bw, shift, ee, rng, integer=True, dtype=dtype)
    note(f"band exact: {case_id(case)} {np.dtype(dtype).name}, nnz {len(ci)}")
    Bm = device_bcsr(torch, M, K, rp, ci, vals, itype)
    Bh = rng.integers(-4, 5, size=(K, N)).astype(dtype)
    C = spmm_band(torch, Bm, torch.as_tensor(Bh).cuda()).cpu().numpy()
    ref = oracle.csr_spmm_f64(M, N, rp, ci, vals, Bh)
    assert np.array_equal(C, ref.astype(np.float32))


@pytest.mark.parametrize("dtype", DTYPES, ids=["f16", "f32"])
@pytest.mark.parametrize("case", CASES, ids=[case_id(c) for c in CASES])
def test_band_random_against_oracle(torch, case, dtype):
    M, K, bw, shift, ee, N, itype = case
    rng = np.random.default_rng(7 * M + K + N)
    rp, ci, vals = band_csr(M, K, bw, shift, ee, rng, dtype=dtype)
    note(f"band random: {case_id(case)} {np.dtype(dtype).name}, nnz {len(ci)}")
    Bm = device_bcsr(torch, M, K, rp, ci, vals, itype)
    Bh = rng.standard_normal((K, N)).astype(dtype)
    Bd = torch.as_tensor(Bh).cuda()
    C = spmm_band(torch, Bm, Bd)
    C2 = spmm_band(torch, Bm, Bd)
    assert torch.equal(C, C2)  # the same summation order on every call
    brp, bci, bv = host_bcsr(Bm)
    ref = oracle.bcsr_spmm_f64(M, K, N, brp, bci, bv, Bh)
    e = oracle.errors(C.cpu().numpy(), ref)
    note(f"  rel_frob {e['rel_frob']:.2e}")
    assert np.all(np.isfinite(C.cpu().numpy()))
    assert e["rel_frob"] <= 1e-5, e
    # where the check selects it, the Python Tier-1 call takes the band
    # kernel: the same C bit for bit
    if Bm.band_rows():
        assert torch.equal(X.spmm(Bm, Bd), C)


@pytest.mark.parametrize("dtype", DTYPES, ids=["f16", "f32"])
def test_band_inf_meets_zero_column(torch, dtype):
    """B row k holds Inf; column k of A is zero in every row, but the blocks
    over it stay present: the reference multiplies each block a row holds
    whole, so 0 * Inf gives NaN in every row of the block-rows holding that
    block, and only there."""
    M = K = 256
    N = 32
    rng = np.random.default_rng(3)
    rp, ci, vals = band_csr(M, K, 20, 0, 0, rng, dtype=dtype)
    D = np.zeros((M, K), dtype)
    for i in range(M):
        D[i, ci[rp[i]:rp[i + 1]]] = vals[rp[i]:rp[i + 1]]
    k = 16 * 5 + 3
    D[:, k] = 0  # column k zero everywhere; blocks over it stay present
    nzr, nzc = np.nonzero(D)
    rp2 = np.zeros(M + 1, np.int64)
    np.add.at(rp2, nzr + 1, 1)
    rp2 = np.cumsum(rp2)
    Bm = device_bcsr(torch, M, K, rp2, nzc, D[nzr, nzc], np.int32)
    Bh = rng.standard_normal((K, N)).astype(dtype)
    Bh[k, 7] = np.inf
    C = spmm_band(torch, Bm, torch.as_tensor(Bh).cuda()).cpu().numpy()
    brp, bci, _ = host_bcsr(Bm)
    hit = np.zeros(M, bool)
    for b in range(Bm.num_block_rows):
        if (bci[brp[b]:brp[b + 1]] == k // 16).any():
            hit[16 * b:16 * b + 16] = True
    assert hit.any() and not hit.all()
    assert np.isnan(C[hit, 7]).all()
    assert np.isfinite(C[~hit]).all()
    assert np.isfinite(np.delete(C[hit], 7, axis=1)).all()


def test_band_selection(torch):
    rng = np.random.default_rng(11)
    # a band and a shifted band: contiguous, neighbours overlap
    for shift in (0, 300):
        rp, ci, vals = band_csr(4096, 4096, 700, shift, 0, rng)
        Bm = device_bcsr(torch, 4096, 4096, rp, ci, vals, np.int32)
        assert band_rows(Bm, len(ci)) == 1
        assert Bm.band_rows()
    # a gap inside one block-row: two bands far apart
    M = K = 2048
    rp, ci, vals = band_csr(M, K, 30, 0, 0, rng)
    rows = [ci[rp[i]:rp[i + 1]] for i in range(M)]
    rows[500] = np.union1d(rows[500], [1900])
    lens = np.array([len(r) for r in rows])
    rp2 = np.concatenate([[0], np.cumsum(lens)])
    ci2 = np.concatenate(rows)
    v2 = rng.standard_normal(len(ci2)).astype(np.float16)
    Bm = device_bcsr(torch, M, K, rp2, ci2, v2, np.int32)
    assert band_rows(Bm, len(ci2)) == 0
    assert not Bm.band_rows()
    # random sparse rows (no contiguous block-rows)
    from xspmm_amd import synth
    p = synth.random_csr(2048, 2048, 64, 0.005, seed=1)
    Bm = device_bcsr(torch, p.M, p.K, p.rp, p.ci, p.vals, np.int32)
    assert band_rows(Bm, p.nnz) == 0
    # every block present: the GEMM-tiled kernel's grid, not the band kernel
    D = rng.standard_normal((256, 256)).astype(np.float16)
    nzr, nzc = np.nonzero(D)
    rp3 = np.concatenate([[0], np.cumsum(np.bincount(nzr, minlength=256))])
    Bm = device_bcsr(torch, 256, 256, rp3, nzc, D[nzr, nzc], np.int32)
    assert band_rows(Bm, len(nzc)) == 0
    # fp32: a wide band (about 90 blocks per block-row) takes the fp32 band
    # kernel, a narrow one (about 5) keeps the column-batch kernel
    rp, ci, vals = band_csr(4096, 4096, 700, 0, 0, rng, dtype=np.float32)
    Bm = device_bcsr(torch, 4096, 4096, rp, ci, vals, np.int32)
    assert band_rows(Bm, len(ci)) == 1 and Bm.band_rows()
    rp, ci, vals = band_csr(4096, 4096, 30, 0, 0, rng, dtype=np.float32)
    Bm = device_bcsr(torch, 4096, 4096, rp, ci, vals, np.int32)
    assert band_rows(Bm, len(ci)) == 0 and not Bm.band_rows()


def block_band(Mb, Kb, wb):
    """Block-row b holds block columns max(0, b - wb) .. min(Kb - 1, b + wb)."""
    lo = np.maximum(0, np.arange(Mb) - wb)
    hi = np.minimum(Kb - 1, np.arange(Mb) + wb)
    lens = hi - lo + 1
    brp = np.zeros(Mb + 1, np.int64)
    np.cumsum(lens, out=brp[1:])
    bci = np.concatenate([np.arange(a, b + 1) for a, b in zip(lo, hi)])
    return brp, bci


def spmm_band_arrays(torch, M, K, Mb, Kb, brp, bci, vals, B):
    N = int(B.shape[1])
    C = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    X._check(X.load().xspmm_bcsr_spmm_band(X.vcode(B.dtype), X.icode(brp.dtype), M, K, Mb, Kb,
                                           int(bci.numel()), X._ptr(brp), X._ptr(bci), X._ptr(vals),
                                           X._ptr(B), X._ptr(C), N, X._stream()))
    torch.cuda.synchronize()
    return C


# (block-rows, block columns, half-width in blocks, ragged rows cut from M, N, index type)
SPLIT_CASES = [
    (1024, 1024, 460, 0, 128, np.int32),   # the examples/05 90 % band, 16384^2
    (1024, 1024, 460, 0, 64, np.int64),
    (256, 300, 120, 7, 132, np.int32),     # 64 groups on 256 CUs; ragged M, three chunks
    (1027, 1100, 60, 3, 8, np.int32),      # too little work: one group per workgroup either way
]


@pytest.mark.parametrize("case", SPLIT_CASES, ids=[f"Mb{c[0]}_Kb{c[1]}_w{c[2]}_N{c[4]}_{np.dtype(c[5]).name}"
                                                   for c in SPLIT_CASES])
def test_band_f32_balanced_launch(torch, case, monkeypatch):
    """The fp32 band kernel's balanced launch (a plan kernel, equal shares of
    the groups' blocks per workgroup, a group cut by a share border summed
    from its parts' partial tiles in part order) at full size: small-integer
    A and B keep every sum exact, so C equals the fp64 product on sampled
    block-rows and equals the one-group-per-workgroup launch
    (XSPMM_BAND_SPLIT=off) bit for bit; repeated calls give the same C."""
    Mb, Kb, wb, cut, N, itype = case
    M, K = 16 * Mb - cut, 16 * Kb
    brp_h, bci_h = block_band(Mb, Kb, wb)
    note(f"fp32 balanced band: Mb {Mb} Kb {Kb} half-width {wb} M {M} N {N} {np.dtype(itype).name}, "
         f"nnzb {len(bci_h)}")
    g = torch.Generator(device="cuda")
    g.manual_seed(Mb + N)
    brp = torch.as_tensor(brp_h.astype(itype)).cuda()
    bci = torch.as_tensor(bci_h.astype(itype)).cuda()
    vals = torch.randint(-2, 3, (len(bci_h), 16, 16), generator=g, device="cuda").to(torch.float32)
    # rows of the last block-row past M are padding: zero, as a conversion leaves them
    if cut:
        vals[int(brp_h[Mb - 1]):, 16 - cut:, :] = 0
    B = torch.randint(-3, 4, (K, N), generator=g, device="cuda").to(torch.float32)
    monkeypatch.delenv("XSPMM_BAND_SPLIT", raising=False)
    C = spmm_band_arrays(torch, M, K, Mb, Kb, brp, bci, vals, B)
    assert torch.equal(C, spmm_band_arrays(torch, M, K, Mb, Kb, brp, bci, vals, B))
    monkeypatch.setenv("XSPMM_BAND_SPLIT", "off")
    C_off = spmm_band_arrays(torch, M, K, Mb, Kb, brp, bci, vals, B)
    monkeypatch.delenv("XSPMM_BAND_SPLIT")
    assert torch.equal(C, C_off)
    Bh = B.cpu().numpy().astype(np.float64)
    Ch = C.cpu().numpy()
    for b in sorted({0, 1, Mb // 3, Mb // 2, Mb - 2, Mb - 1}):
        blocks = vals[int(brp_h[b]):int(brp_h[b + 1])].cpu().numpy().astype(np.float64)
        ref = np.zeros((16, N))
        for blk, c in zip(blocks, bci_h[brp_h[b]:brp_h[b + 1]]):
            ref += blk @ Bh[16 * c:16 * c + 16]
        rows = min(16, M - 16 * b)
        assert np.array_equal(Ch[16 * b:16 * b + rows], ref[:rows].astype(np.float32)), b


def test_band_f32_empty_grid(torch):
    """A grid of block-rows without blocks (nnzb = 0) through the band entry:
    few enough groups for the balanced launch, which an empty grid does not
    take (its plan would have no column index to read); C is all zeros."""
    Mb, Kb, N = 40, 30, 64
    brp = torch.zeros(Mb + 1, dtype=torch.int32, device="cuda")
    bci = torch.zeros(0, dtype=torch.int32, device="cuda")
    vals = torch.zeros(0, dtype=torch.float32, device="cuda")
    B = torch.ones((16 * Kb, N), dtype=torch.float32, device="cuda")
    note("fp32 band entry, empty grid")
    C = spmm_band_arrays(torch, 16 * Mb, 16 * Kb, Mb, Kb, brp, bci, vals, B)
    assert torch.count_nonzero(C).item() == 0


def test_band_f32_balanced_random_shapes(torch, monkeypatch):
    """24 seeded random band shapes through the fp32 band entry (ragged M, K
    and N, shifted bands, runs of empty block-rows, both index types), with
    the balanced launch forced (XSPMM_BAND_SPLIT=force; the launcher's rule
    leaves most of these small grids to one group per workgroup):
    small-integer products equal the fp64 product exactly and the
    one-group-per-workgroup launch bit for bit."""
    rng = np.random.default_rng(2024)
    for i in range(24):
        M = int(rng.integers(17, 2600))
        K = int(rng.integers(17, 2600))
        bw = int(rng.integers(1, max(2, K // 2)))
        shift = int(rng.integers(-K // 4, K // 4 + 1))
        ee = int(rng.choice([0, 0, 2, 3, 5]))
        N = 4 * int(rng.integers(1, 50))
        itype = np.int32 if i % 2 == 0 else np.int64
        note(f"random fp32 band {i}: M {M} K {K} bw {bw} shift {shift} empty every {ee} N {N} "
             f"{np.dtype(itype).name}")
        rp, ci, vals = band_csr(M, K, bw, shift, ee, rng, integer=True, dtype=np.float32)
        Bm = device_bcsr(torch, M, K, rp, ci, vals, itype)
        Bh = rng.integers(-3, 4, size=(K, N)).astype(np.float32)
        Bd = torch.as_tensor(Bh).cuda()
        monkeypatch.setenv("XSPMM_BAND_SPLIT", "force")
        C = spmm_band(torch, Bm, Bd)
        monkeypatch.setenv("XSPMM_BAND_SPLIT", "off")
        C_off = spmm_band(torch, Bm, Bd)
        monkeypatch.delenv("XSPMM_BAND_SPLIT")
        ref = oracle.csr_spmm_f64(M, N, rp, ci, vals, Bh)
        assert np.array_equal(C.cpu().numpy(), ref.astype(np.float32)), i
        assert torch.equal(C, C_off), i
