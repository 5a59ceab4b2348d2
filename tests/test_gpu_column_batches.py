"""GPU parity of the fp16 column-batch SpMM kernel (the Tier-1 default for
N % 8 == 0) on block contents chosen to drive its batch logic: pairs with 1,
8, 16, 17, 24, 25 and 32 non-zero columns, slot ranges that end exactly on
and straddle the 16-slot half, every pair a batch of its own, all-zero
blocks, odd block counts, and special values (-0.0, fp16 subnormals, large
magnitudes, an Inf).

Integer-valued A and B keep every fp32 partial sum exact, so C is compared
bit for bit with the fp64 product (a slot or column mix-up cannot hide in a
tolerance).  The prepared product, which stores the same batches in pack mode,
must give the same C.  All calls go through the C ABI.
"""
from __future__ import annotations

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


def host(t):
    return t.detach().cpu().numpy()


# block-rows given as the number of non-zero columns of each block, in order
COUNT_ROWS = [
    [16] * 20,                            # 32 columns per pair: every pair its own batch
    [8, 8] * 10,                          # 16 per pair: batches end exactly on the half
    [9, 8] * 10,                          # 17 per pair: slot ranges straddle the half
    [1] * 37,                             # one column per block, odd block count
    [15, 16, 1, 0, 3, 16, 12, 13] * 3,    # mixed, with an all-zero block
    [16, 16, 16],                         # odd count of full blocks
    list(range(17)),                      # 0 .. 16 columns
    [12, 12, 13, 12, 4, 4, 16, 9] * 4,    # 24, 25, 8, 25 per pair
    [],                                   # empty block-row
    [2, 0, 0, 2, 5],                      # zero-column pair in the middle
]


def to_csr(D, itype):
    nzr, nzc = np.nonzero(D)
    rp = np.zeros(D.shape[0] + 1, np.int64)
    np.add.at(rp, nzr + 1, 1)
    rp = np.cumsum(rp)
    return rp.astype(itype), nzc.astype(itype), D[nzr, nzc]


def bcsr_of_dense(torch, D, rows, rng_cols, itype):
    """Device BCSR of D with exactly the block structure of `rows` (zero blocks
    included), block columns as drawn by build()."""
    Mb = D.shape[0] // 16
    Kb = D.shape[1] // 16
    brp = [0]
    bci = []
    vals = []
    for i, counts in enumerate(rows):
        for c in rng_cols[i]:
            bci.append(c)
            vals.append(D[16 * i:16 * i + 16, 16 * c:16 * c + 16].reshape(-1))
        brp.append(len(bci))
    bv = np.concatenate(vals) if vals else np.zeros(0, np.float16)
    t = lambda a, dt: torch.as_tensor(np.asarray(a, dt)).cuda()
    return X.BCSRMatrix(Mb, Kb, 16, 16, D.shape[0], D.shape[1], t(brp, itype), t(bci, itype),
                        t(bv, np.float16))


def build(seed, value_fn, Kb=64):
    rng = np.random.default_rng(seed)
    Mb = len(COUNT_ROWS)
    D = np.zeros((16 * Mb, 16 * Kb), np.float16)
    cols_per_row = []
    for i, counts in enumerate(COUNT_ROWS):
        cols = np.sort(rng.choice(Kb, size=len(counts), replace=False))
        cols_per_row.append(cols)
        for c, n in zip(cols, counts):
            blk = np.zeros((16, 16), np.float16)
            for e in rng.choice(16, size=n, replace=False):
                rws = rng.random(16) < 0.4
                rws[rng.integers(16)] = True
                blk[rws, e] = value_fn(rng, int(rws.sum()))
            D[16 * i:16 * i + 16, 16 * c:16 * c + 16] = blk
    return rng, D, cols_per_row


def small_ints(rng, n):
    v = rng.integers(1, 4, size=n) * rng.choice([-1, 1], size=n)
    return v.astype(np.float16)


@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("N", [8, 64, 128, 136])
def test_batch_column_counts_exact(torch, itype, N):
    rng, D, cols = build(7, small_ints)
    B = rng.integers(-4, 5, size=(D.shape[1], N)).astype(np.float16)
    ref = D.astype(np.float64) @ B.astype(np.float64)
    note(f"column counts N={N} {itype.__name__}")
    Bm = bcsr_of_dense(torch, D, COUNT_ROWS, cols, itype)
    C = torch.full((D.shape[0], N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm(Bm, torch.as_tensor(B).cuda(), C, N)
    torch.cuda.synchronize()
    Ch = host(C)
    assert np.array_equal(Ch.astype(np.float64), ref)
    assert np.all(Ch[16 * COUNT_ROWS.index([]):][:16] == 0)


@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_batch_column_counts_prepared_product(torch, itype):
    # the prepared product packs the same batches (count and pack modes): its
    # C equals the pipeline's bit for bit and the exact product
    rng, D, _ = build(11, small_ints)
    rp, ci, vals = to_csr(D, itype)
    A = X.CSRMatrix.from_host(D.shape[0], D.shape[1], rp, ci, vals)
    for cluster in (False, True):
        plan = X.SpMMPlan(A, optimize_pattern=cluster)
        for N in (8, 64, 128):
            B = rng.integers(-4, 5, size=(D.shape[1], N)).astype(np.float16)
            Bd = torch.as_tensor(B).cuda()
            C1 = plan.execute(Bd)
            C2, _ = X.spmm_pipeline(A, Bd, optimize_pattern=cluster)
            torch.cuda.synchronize()
            note(f"prepared cluster={cluster} N={N} batches={plan.packed_batches}")
            assert torch.equal(C1, C2), (cluster, N)
            assert np.array_equal(host(C1).astype(np.float64),
                                  D.astype(np.float64) @ B.astype(np.float64))
        plan.close()


def special_values(rng, n):
    pool = np.array([-0.0, 2.0 ** -24, -(2.0 ** -24), 2.0 ** -15, 2.0 ** -14, 1.5, -3.0,
                     6.0e4, -6.0e4, 1.0 / 3.0], np.float64)
    return pool[rng.integers(len(pool), size=n)].astype(np.float16)


@pytest.mark.parametrize("N", [64, 128])
def test_batch_special_values(torch, N):
    # -0.0 entries (a column holding only -0.0 still takes a slot), fp16
    # subnormals and large magnitudes, against the fp64 product
    rng, D, cols = build(3, special_values)
    assert np.any(np.signbit(D) & (D == 0))
    B = (rng.choice([-2.0, -1.0, 0.5, 1.0, 2.0, 4.0], size=(D.shape[1], N))).astype(np.float16)
    Bm = bcsr_of_dense(torch, D, COUNT_ROWS, cols, np.int32)
    C = X.spmm(Bm, torch.as_tensor(B).cuda(), N=N)
    torch.cuda.synchronize()
    Ch = host(C)
    ref = D.astype(np.float64) @ B.astype(np.float64)
    assert np.all(np.isfinite(Ch))
    e = oracle.errors(Ch, ref)
    note(f"special values N={N}: {e}")
    assert e["rel_frob"] <= 1e-6, e
    # entries whose terms are all subnormal-scale stay exact: compare rows of
    # the all-subnormal case directly
    D2 = np.zeros_like(D)
    D2[D != 0] = np.float16(2.0 ** -24)
    Bm2 = bcsr_of_dense(torch, D2, COUNT_ROWS, cols, np.int32)
    C2 = X.spmm(Bm2, torch.as_tensor(B).cuda(), N=N)
    torch.cuda.synchronize()
    assert np.array_equal(host(C2).astype(np.float64), D2.astype(np.float64) @ B.astype(np.float64))


def test_batch_inf_stays_in_its_row(torch):
    # an Inf in A makes its C row non-finite (as the reference's 0 * Inf and
    # Inf * b do); every other row is exact
    rng, D, cols = build(5, small_ints)
    r, c = [(i, j) for i, j in zip(*np.nonzero(D)) if i // 16 == 4][0]
    D[r, c] = np.float16(np.inf)
    N = 64
    B = rng.integers(1, 5, size=(D.shape[1], N)).astype(np.float16)
    Bm = bcsr_of_dense(torch, D, COUNT_ROWS, cols, np.int32)
    C = host(X.spmm(Bm, torch.as_tensor(B).cuda(), N=N))
    torch.cuda.synchronize()
    assert not np.any(np.isfinite(C[r]))
    Df = D.astype(np.float64)
    Df[r] = 0
    ref = Df @ B.astype(np.float64)
    keep = np.arange(D.shape[0]) != r
    assert np.array_equal(C[keep].astype(np.float64), ref[keep])


@pytest.mark.parametrize("itype", [np.int32, np.int64])
def test_batch_invalid_block_columns_contribute_nothing(torch, itype):
    # malformed BCSR: block columns >= Kb (and, for int64, with high bits set)
    # are masked out; the reference would read B out of bounds
    rng, D, cols = build(9, small_ints)
    Bm = bcsr_of_dense(torch, D, COUNT_ROWS, cols, itype)
    bci = host(Bm.col_ind).copy()
    bad = rng.random(len(bci)) < 0.25
    Kb = Bm.num_block_cols
    bci_bad = bci.copy()
    bci_bad[bad] = Kb + rng.integers(0, 1000, size=int(bad.sum()))
    if itype == np.int64:
        hi = bad & (rng.random(len(bci)) < 0.5)
        bci_bad[hi] = (np.int64(1) << 40) + bci[hi]
    Bm.col_ind = torch.as_tensor(bci_bad).cuda()
    N = 64
    B = rng.integers(-4, 5, size=(D.shape[1], N)).astype(np.float16)
    C = host(X.spmm(Bm, torch.as_tensor(B).cuda(), N=N))
    torch.cuda.synchronize()
    # reference: the same blocks without the bad ones
    Dg = D.astype(np.float64).copy()
    brp = host(Bm.row_ptr)
    for i in range(len(COUNT_ROWS)):
        for k in range(brp[i], brp[i + 1]):
            if bad[k]:
                c = bci[k]
                Dg[16 * i:16 * i + 16, 16 * c:16 * c + 16] = 0
    assert np.array_equal(C.astype(np.float64), Dg @ B.astype(np.float64))


XCD_CHILD = r"""
import hashlib, json, sys
import numpy as np, torch
sys.path.insert(0, sys.argv[1])
import xspmm_amd as X
out = {}
for Mb, N in ((64, 256), (64, 200), (66, 256)):
    rng = np.random.default_rng(Mb + N)
    Kb = 96
    D = np.zeros((16 * Mb, 16 * Kb), np.float16)
    for b in range(Mb):
        for c in np.nonzero(rng.random(Kb) < 0.2)[0]:
            D[16 * b:16 * b + 16, 16 * c:16 * c + 16] = rng.integers(-3, 4, size=(16, 16))
    nzr, nzc = np.nonzero(D)
    rp = np.concatenate([[0], np.cumsum(np.bincount(nzr, minlength=16 * Mb))]).astype(np.int32)
    A = X.CSRMatrix.from_host(16 * Mb, 16 * Kb, rp, nzc.astype(np.int32), D[nzr, nzc])
    Bm = X.csr_to_bcsr(A)
    B = rng.integers(-4, 5, size=(16 * Kb, N)).astype(np.float16)
    C = X.spmm(Bm, torch.as_tensor(B).cuda(), N=N).cpu().numpy()
    ref = D.astype(np.float64) @ B.astype(np.float64)
    out[f"{Mb}x{N}"] = {"exact": bool(np.array_equal(C.astype(np.float64), ref)),
                        "sha256": hashlib.sha256(C.tobytes()).hexdigest()}
print(json.dumps(out))
"""


def test_batch_two_chunks_on_xcd_halves():
    """Grids of two 128-column chunks with Mb % 4 == 0 (configs[1]'s shape)
    put each chunk on its own half of the XCDs (workgroup l runs chunk
    (l / 4) % 2 of block-row 4 (l / 8) + l % 4).  Exact small-integer products
    with the mapping (default) and without it (XSPMM_BATCH_XCD=off, read once
    per process, so each runs in its own process), bit-identical C; Mb = 66
    keeps the plain grid either way."""
    import json
    import os
    import subprocess
    import sys
    root = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
    res = {}
    for mode in ("on", "off"):
        env = dict(os.environ)
        env.pop("XSPMM_BATCH_XCD", None)
        if mode == "off":
            env["XSPMM_BATCH_XCD"] = "off"
        note(f"two-chunk grids, XCD halves {mode}")
        r = subprocess.run([sys.executable, "-c", XCD_CHILD, root], env=env, capture_output=True,
                           text=True, timeout=180)
        assert r.returncode == 0, r.stderr[-2000:]
        res[mode] = json.loads(r.stdout.strip().splitlines()[-1])
    for k in res["on"]:
        assert res["on"][k]["exact"] and res["off"][k]["exact"], k
        assert res["on"][k]["sha256"] == res["off"][k]["sha256"], k
