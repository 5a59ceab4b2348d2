"""CPU: pins the oracle (oracle/oracle.c) before anything is checked against it.

Every oracle function is checked against
  * the golden vectors written by tests/golden/make_golden.py from the
    reference's own CPU code (oracle/_ref, compiled from /root/reference);
  * the compiled reference directly on further seeded inputs, when it is
    present in this container;
  * closed forms and invariants chosen so that a plausible mistake (dropped
    term, wrong index, transposed block, first-wins duplicates, wrong scan
    direction in the clustering) fails one of them.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from tests.helpers import dense_from_bcsr, dense_last_wins, golden_cases, widen
from xspmm_amd import synth

CONV = golden_cases("conversion")
JAC = golden_cases("jaccard")
PERM = golden_cases("permutation")


def test_golden_present():
    assert len(CONV) >= 20 and len(JAC) >= 20 and len(PERM) >= 6


# ---------------------------------------------------------------------------
# csr_to_bcsr
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", CONV, ids=[c["name"] for c in CONV])
def test_conversion_matches_golden(case):
    M, K, rb, cb = int(case["M"]), int(case["K"]), int(case["rb"]), int(case["cb"])
    brp, bci, bv = oracle.csr_to_bcsr(M, K, case["rp"], case["ci"], case["vals"], rb, cb)
    np.testing.assert_array_equal(brp, widen(case["brp"]))
    np.testing.assert_array_equal(bci, widen(case["bci"]))
    assert bv.view(np.uint32).tobytes() == case["bvals"].astype(np.float32).view(np.uint32).tobytes()


@pytest.mark.parametrize("case", CONV, ids=[c["name"] for c in CONV])
def test_conversion_dense_invariant(case):
    M, K, rb, cb = int(case["M"]), int(case["K"]), int(case["rb"]), int(case["cb"])
    brp, bci, bv = oracle.csr_to_bcsr(M, K, case["rp"], case["ci"], case["vals"], rb, cb)
    D = dense_last_wins(M, K, case["rp"], case["ci"], case["vals"])
    np.testing.assert_array_equal(dense_from_bcsr(M, K, rb, cb, brp, bci, bv), D)
    # block columns strictly ascending inside every block-row
    for br in range(len(brp) - 1):
        seg = bci[brp[br]:brp[br + 1]]
        assert np.all(np.diff(seg) > 0)


def test_conversion_last_duplicate_wins():
    # one row, the same column three times: the last value must survive
    rp = np.array([0, 3]); ci = np.array([5, 5, 5]); v = np.array([1.0, 2.0, 3.0], np.float32)
    brp, bci, bv = oracle.csr_to_bcsr(1, 16, rp, ci, v)
    assert list(brp) == [0, 1] and list(bci) == [0]
    assert bv[5] == 3.0 and np.count_nonzero(bv) == 1


def test_conversion_fp16_bits_preserved():
    rng = np.random.default_rng(3)
    p = synth.random_csr(40, 50, 5, 0.1, seed=4, dtype=np.float16, unsorted=True, dup_frac=0.2)
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    b2, c2, v2 = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals.astype(np.float32))
    np.testing.assert_array_equal(brp, b2)
    np.testing.assert_array_equal(bci, c2)
    assert bv.dtype == np.float16
    np.testing.assert_array_equal(bv.astype(np.float32), v2)
    del rng


def test_conversion_rejects_bad_column():
    with pytest.raises(ValueError):
        oracle.csr_to_bcsr(1, 10, np.array([0, 1]), np.array([10]), np.ones(1, np.float32))


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no /root/reference)")
@pytest.mark.parametrize("seed", range(6))
def test_conversion_matches_reference_random(seed):
    rng = np.random.default_rng(100 + seed)
    M, K = int(rng.integers(1, 90)), int(rng.integers(1, 300))
    rb, cb = [(16, 16), (4, 4), (8, 16), (5, 3), (16, 2), (1, 1)][seed]
    p = synth.random_csr(M, K, 4, float(rng.uniform(0.01, 0.2)), seed=seed, dtype=np.float32,
                         unsorted=bool(seed % 2), dup_frac=0.15 * (seed % 3))
    a = oracle.csr_to_bcsr(M, K, p.rp, p.ci, p.vals, rb, cb)
    b = oracle.ref_csr_to_bcsr(M, K, p.rp, p.ci, p.vals, rb, cb, index_dtype=np.int64)
    for x, y in zip(a, b):
        np.testing.assert_array_equal(np.asarray(x, np.float64), np.asarray(y, np.float64))


# ---------------------------------------------------------------------------
# Jaccard clustering
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", JAC, ids=[c["name"] for c in JAC])
def test_jaccard_matches_golden(case):
    perm = oracle.jaccard(int(case["M"]), int(case["K"]), case["rp"], case["ci"],
                          float(case["thresh"]), int(case["bw"]))
    np.testing.assert_array_equal(perm, widen(case["perm"]))


def _csr(rows):
    rp = np.zeros(len(rows) + 1, np.int64)
    rp[1:] = np.cumsum([len(r) for r in rows])
    ci = np.concatenate([np.asarray(r, np.int64) for r in rows]) if rows else np.zeros(0, np.int64)
    return rp, ci


def test_jaccard_hand_case():
    # blocks of width 16: row0={0}, row1={0,1}, row2={2}, row3={0}.
    # seed 3 (p={0}); cand 2: d=1 -> no; cand 1: d=1-1/2=0.5 -> join, p={0,1};
    # cand 0: d=0.5 -> join.  Then seed 2 alone.  perm = [3, 1, 0, 2].
    rp, ci = _csr([[1], [2, 20], [40], [3]])
    assert list(oracle.jaccard(4, 48, rp, ci, 0.5, 16)) == [3, 1, 0, 2]
    # just below the tie only identical patterns join: seed 3 takes row 0
    # (d=0; row 2 moves into slot 0), then seed 1 (now last) and seed 2 alone.
    assert list(oracle.jaccard(4, 48, rp, ci, 0.49, 16)) == [3, 0, 1, 2]


def test_jaccard_swap_remove_order():
    # rows 0..4 all identical -> one cluster; visiting order is seed 4 then
    # positions 3,2,1,0 -> perm = reversed.
    rp, ci = _csr([[0]] * 5)
    assert list(oracle.jaccard(5, 16, rp, ci, 0.5, 16)) == [4, 3, 2, 1, 0]
    # joins move the last element into the freed slot; it is not revisited:
    # blocks row0={1}, row1={0}, row2={5}, row3={0}: seed 3 joins row1 at pos 1
    # (d=0); row2 (last) moves into pos 1, then pos 0 (row0, d=1) -> no.
    rp, ci = _csr([[16], [0], [80], [1]])
    assert list(oracle.jaccard(4, 96, rp, ci, 0.5, 16)) == [3, 1, 2, 0]


def test_jaccard_closed_forms():
    # disjoint blocks: no joins -> perm = [M-1, ..., 0]
    rp, ci = _csr([[16 * i] for i in range(20)])
    assert list(oracle.jaccard(20, 320, rp, ci, 0.5, 16)) == list(range(19, -1, -1))
    # all rows empty -> one cluster in scan order -> reversed
    rp, ci = _csr([[] for _ in range(7)])
    assert list(oracle.jaccard(7, 32, rp, ci, 0.5, 16)) == list(range(6, -1, -1))
    # threshold >= 1: everything joins the first seed -> reversed
    p = synth.random_csr(50, 200, 4, 0.05, seed=1)
    assert list(oracle.jaccard(50, 200, p.rp, p.ci, 1.0, 16)) == list(range(49, -1, -1))


def test_jaccard_is_permutation_on_config_like_input():
    p = synth.random_csr(400, 1024, 4, 0.01, seed=7)
    perm = oracle.jaccard(p.M, p.K, p.rp, p.ci)
    assert sorted(perm) == list(range(p.M))


@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no /root/reference)")
@pytest.mark.parametrize("seed", range(5))
def test_jaccard_matches_reference_random(seed):
    rng = np.random.default_rng(200 + seed)
    M, K = int(rng.integers(2, 300)), int(rng.integers(16, 400))
    thr = float([0.5, 0.5, 0.33, 0.6, 0.2][seed])
    bw = [16, 8, 16, 4, 16][seed]
    p = synth.random_csr(M, K, 4, float(rng.uniform(0.005, 0.08)), seed=seed)
    np.testing.assert_array_equal(oracle.jaccard(M, K, p.rp, p.ci, thr, bw),
                                  oracle.ref_jaccard(M, K, p.rp, p.ci, thr, bw))


# ---------------------------------------------------------------------------
# permutation / unpermutation
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("case", PERM, ids=[c["name"] for c in PERM])
def test_permutation_matches_golden(case):
    M = int(case["M"])
    nrp, nci, nv = oracle.apply_perm(M, case["rp"], case["ci"], case["vals"], case["perm"])
    np.testing.assert_array_equal(nrp, widen(case["nrp"]))
    np.testing.assert_array_equal(nci, widen(case["nci"]))
    np.testing.assert_array_equal(nv, case["nvals"])


def test_permutation_roundtrip():
    p = synth.random_csr(64, 64, 4, 0.1, seed=2, dtype=np.float32)
    perm = np.random.default_rng(0).permutation(p.M)
    nrp, nci, nv = oracle.apply_perm(p.M, p.rp, p.ci, p.vals, perm)
    inv = np.argsort(perm)
    brp, bci, bv = oracle.apply_perm(p.M, nrp, nci, nv, inv)
    np.testing.assert_array_equal(brp, widen(p.rp))
    np.testing.assert_array_equal(bci, widen(p.ci))
    np.testing.assert_array_equal(bv, p.vals)


def test_unpermute_is_scatter():
    rng = np.random.default_rng(5)
    X = rng.standard_normal((30, 7)).astype(np.float32)
    perm = rng.permutation(30)
    out = oracle.unpermute(30, 7, X, perm)
    np.testing.assert_array_equal(out[perm], X)


# ---------------------------------------------------------------------------
# SpMM
# ---------------------------------------------------------------------------

def test_spmm_checkers_times_ones_is_row_sums():
    # closed form behind examples/01_uspmm_checkers.cpp: C[i, :] = sum_j A[i, j]
    p = synth.checkers(M=96, K=80, N=12, bs=4, dtype=np.float32)
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    C = oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, p.B)
    rs = np.add.reduceat(p.vals.astype(np.float64), p.rp[:-1]) if p.nnz else np.zeros(p.M)
    rs[np.diff(p.rp) == 0] = 0
    np.testing.assert_allclose(C, np.repeat(rs[:, None], p.N, axis=1), rtol=1e-12, atol=1e-12)


def test_spmm_identity_blocks_copy_B():
    # A = identity (ragged 40 x 40): C must equal B exactly, also in fp32 accumulation
    M = 40
    rp = np.arange(M + 1); ci = np.arange(M); v = np.ones(M, np.float32)
    B = np.random.default_rng(1).standard_normal((M, 9)).astype(np.float32)
    brp, bci, bv = oracle.csr_to_bcsr(M, M, rp, ci, v)
    np.testing.assert_array_equal(oracle.bcsr_spmm_f64(M, M, 9, brp, bci, bv, B), B)
    np.testing.assert_array_equal(oracle.bcsr_spmm_f32(M, M, 9, brp, bci, bv, B), B)


def test_spmm_matches_dense_numpy():
    for dtype in (np.float16, np.float32):
        p = synth.random_csr(70, 45, 19, 0.08, seed=11, dtype=dtype, unsorted=True)
        brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
        D = dense_last_wins(p.M, p.K, p.rp, p.ci, p.vals.astype(np.float64))
        ref = D @ p.B.astype(np.float64)
        np.testing.assert_allclose(oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, p.B), ref,
                                   rtol=1e-12, atol=1e-12)
        c32 = oracle.bcsr_spmm_f32(p.M, p.K, p.N, brp, bci, bv, p.B, nthreads=3)
        assert oracle.errors(c32, ref)["rel_frob"] < 1e-6


def test_spmm_fp16_widening_all_finite_patterns():
    # identity block times B holding every finite fp16 bit pattern: the fp32
    # accumulation path must reproduce numpy's exact fp16 -> fp32 widening.
    bits = np.arange(65536, dtype=np.uint16)
    h = bits.view(np.float16)
    h = h[np.isfinite(h)]
    n = 16 * ((len(h) + 15) // 16)
    Bv = np.zeros(n, np.float16); Bv[:len(h)] = h
    B = Bv.reshape(16, -1)
    rp = np.arange(17); ci = np.arange(16); v = np.ones(16, np.float16)
    brp, bci, bv = oracle.csr_to_bcsr(16, 16, rp, ci, v)
    C = oracle.bcsr_spmm_f32(16, 16, B.shape[1], brp, bci, bv, B)
    want = B.astype(np.float32)
    want[want == 0] = 0.0  # accumulation starts at +0, and +0 + (-0) = +0
    np.testing.assert_array_equal(C.view(np.uint32), want.view(np.uint32))


def test_csr_spmm_truth_and_errors():
    p = synth.cpu_ref()
    ref = oracle.csr_spmm_f64(p.M, p.N, p.rp, p.ci, p.vals, p.B)
    D = dense_last_wins(p.M, p.K, p.rp, p.ci, p.vals)
    np.testing.assert_allclose(ref, D @ p.B.astype(np.float64), rtol=1e-12, atol=1e-12)
    e = oracle.errors(ref.astype(np.float32) * 1.0, ref)
    assert e["rel_frob"] < 1e-7
    e = oracle.errors(np.zeros_like(ref, np.float32), ref)
    assert abs(e["rel_frob"] - 1.0) < 1e-12 and abs(e["max_rel"] - 1.0) < 1e-12
