"""GPU parity of the device Jaccard clustering (xspmm_jaccard_clustering).

The permutation must equal the reference's bit for bit:
  * against the golden permutations written by the compiled reference
    (ties inter/union = 1/2, thresholds 0 / 0.3 / 0.75 / 1 / negative, block
    widths 1 and 4, more than one bitmap word per row), with each engine
    forced and with the automatic choice;
  * against the oracle's greedy on seeded random, template-like, skewed and
    empty-row inputs, int32 and int64, both engines;
  * both with the partner lists (all pairs on the int8 matrix cores by
    default, or by VALU popcounts with XSPMM_CLUSTER_PARTNERS=popcount) and
    without them (XSPMM_CLUSTER_PARTNERS=off), and with both partner passes
    at row bitmaps of 1 to 32 words;
  * runs of joins that leave the pattern as it is (committed in one step),
    and rows with more partners than their lists hold;
  * at the headline size (templates, 16384 rows) against the oracle, and on
    the 131072-row power-law graph against the product's host engine (the
    oracle's scan would take minutes there; the host engine is pinned to the
    reference by the CPU tests).
All calls go through the C ABI of libxspmm.so.
"""
from __future__ import annotations

import os

import numpy as np
import pytest

import oracle
import xspmm_amd as X
from tests.helpers import golden_cases, nested_csr, widen
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


def csr(torch, M, K, rp, ci, itype=None):
    it = itype or np.asarray(rp).dtype
    rp = np.ascontiguousarray(rp).astype(it)
    ci = np.ascontiguousarray(ci).astype(it)
    t = torch.int32 if np.dtype(it) == np.int32 else torch.int64
    return X.CSRMatrix(int(M), int(K), torch.as_tensor(rp).cuda().to(t),
                       torch.as_tensor(ci).cuda().to(t),
                       torch.zeros(max(len(ci), 0), dtype=torch.float16, device="cuda"))


def gpu_perm(torch, M, K, rp, ci, thr=0.5, bw=16, itype=None):
    A = csr(torch, M, K, rp, ci, itype)
    perm, engine = X.jaccard_clustering(A, thr, bw, return_engine=True)
    torch.cuda.synchronize()
    return perm.cpu().numpy(), engine


def expected_engine(forced, thr):
    if not (0.0 <= thr < 1.0):  # NaN too
        return "closed-form"
    return forced


JAC = golden_cases("jaccard")


@pytest.mark.parametrize("partners", ["on", "popcount", "off"])
@pytest.mark.parametrize("engine", ["scan", "index", "auto"])
@pytest.mark.parametrize("case", JAC, ids=[c["name"] for c in JAC])
def test_gpu_clustering_matches_reference_golden(torch, case, engine, partners, monkeypatch):
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", engine)
    monkeypatch.setenv("XSPMM_CLUSTER_PARTNERS", partners)
    thr = float(case["thresh"])
    note(f"golden {case['name']} engine={engine} partners={partners} M={int(case['M'])} thr={thr}")
    perm, used = gpu_perm(torch, int(case["M"]), int(case["K"]), case["rp"], case["ci"], thr,
                          int(case["bw"]))
    assert perm.dtype == case["rp"].dtype
    np.testing.assert_array_equal(widen(perm), widen(case["perm"]))
    if engine != "auto":
        assert used == expected_engine(engine, thr)


def skewed_csr(rng, M, K):
    rows = []
    for r in range(M):
        kind = rng.integers(0, 10)
        if kind == 0:
            rows.append(np.zeros(0, np.int64))  # empty row
        elif kind == 1:
            rows.append(rng.integers(0, K, size=int(rng.integers(50, 400))))  # long row
        else:
            rows.append(rng.integers(0, K, size=int(rng.integers(1, 12))))
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum([len(x) for x in rows])
    ci = np.concatenate(rows) if rp[-1] else np.zeros(0, np.int64)
    return rp, ci


@pytest.mark.parametrize("partners", ["on", "popcount", "off"])
@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("engine", ["scan", "index"])
@pytest.mark.parametrize("seed", range(8))
def test_gpu_clustering_matches_oracle_random(torch, seed, engine, itype, partners, monkeypatch):
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", engine)
    monkeypatch.setenv("XSPMM_CLUSTER_PARTNERS", partners)
    rng = np.random.default_rng(900 + seed)
    thr = [0.5, 0.4, 0.0, 0.5, 0.25, 0.7, 0.75, 0.6][seed]
    bw = [16, 8, 16, 3, 16, 1, 16, 32][seed]
    if seed >= 6:
        # many joins: rows drawn from a few patterns with small perturbations
        M, K = 3000, 2048 if seed == 6 else 9000
        base = [rng.choice(K, size=int(rng.integers(5, 40)), replace=False) for _ in range(40)]
        rows = []
        for r in range(M):
            b = base[int(rng.integers(0, len(base)))]
            keep = b[rng.random(len(b)) < 0.9]
            rows.append(np.concatenate([keep, rng.integers(0, K, size=int(rng.integers(0, 3)))]))
        rp = np.zeros(M + 1, np.int64)
        rp[1:] = np.cumsum([len(x) for x in rows])
        ci = np.concatenate(rows).astype(np.int64)
    elif seed % 3 == 0:
        M, K = int(rng.integers(100, 3000)), int(rng.integers(64, 5000))
        p = synth.random_csr(M, K, 4, float(rng.uniform(0.001, 0.02)), seed=seed,
                             dtype=np.float32, unsorted=bool(seed % 2))
        rp, ci = p.rp, p.ci
    elif seed % 3 == 1:
        p = synth.templates(M=1024 + 512 * seed, n_templates=64, seed=seed)
        M, K, rp, ci = p.M, p.K, p.rp, p.ci
    else:
        M, K = int(rng.integers(500, 2500)), int(rng.integers(100, 3000))
        rp, ci = skewed_csr(rng, M, K)
    note(f"random seed={seed} engine={engine} partners={partners} itype={np.dtype(itype).name} "
         f"M={M} K={K} thr={thr} bw={bw}")
    want = oracle.jaccard(M, K, rp, ci, thr, bw)
    got, used = gpu_perm(torch, M, K, rp, ci, thr, bw, itype)
    assert got.dtype == itype
    np.testing.assert_array_equal(widen(got), want)
    assert used == engine


@pytest.mark.parametrize("thr", [-0.25, 1.0, 1.5, float("nan")])
def test_gpu_clustering_thresholds_outside_unit_interval(torch, thr):
    # d <= thr never holds (thr < 0, NaN) or always holds (thr >= 1)
    rng = np.random.default_rng(5)
    rp, ci = skewed_csr(rng, 700, 900)
    want = oracle.jaccard(700, 900, rp, ci, thr, 16)
    got, used = gpu_perm(torch, 700, 900, rp, ci, thr)
    np.testing.assert_array_equal(widen(got), want)
    np.testing.assert_array_equal(widen(got), np.arange(699, -1, -1))
    assert used == "closed-form"


@pytest.mark.parametrize("engine", ["scan", "index"])
def test_gpu_clustering_degenerate_shapes(torch, engine, monkeypatch):
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", engine)
    # one row
    got, _ = gpu_perm(torch, 1, 16, np.array([0, 2]), np.array([3, 9]))
    np.testing.assert_array_equal(got, [0])
    # no column at all (K = 0): every row is empty
    got, _ = gpu_perm(torch, 37, 0, np.zeros(38, np.int64), np.zeros(0, np.int64))
    np.testing.assert_array_equal(widen(got), oracle.jaccard(37, 0, np.zeros(38, np.int64),
                                                             np.zeros(0, np.int64)))
    # only empty rows but K > 0, and a mix of identical rows
    rp = np.array([0, 0, 0, 2, 2, 4, 4], np.int64)
    ci = np.array([5, 40, 5, 40], np.int64)
    got, _ = gpu_perm(torch, 6, 64, rp, ci)
    np.testing.assert_array_equal(widen(got), oracle.jaccard(6, 64, rp, ci))
    # more than 1024 rows join the first cluster (several 1024-position steps)
    M = 5000
    rp = np.arange(M + 1, dtype=np.int64)
    ci = np.full(M, 7, np.int64)
    got, _ = gpu_perm(torch, M, 32, rp, ci)
    np.testing.assert_array_equal(widen(got), oracle.jaccard(M, 32, rp, ci))


def test_gpu_clustering_rejects_bad_input(torch):
    with pytest.raises(X.XspmmInvalidArgument):
        gpu_perm(torch, 2, 16, np.array([0, 1, 2]), np.array([0, 99]))
    with pytest.raises(X.XspmmInvalidArgument):
        gpu_perm(torch, 2, 16, np.array([0, 1, 2]), np.array([0, -1]))
    with pytest.raises(X.XspmmInvalidArgument):
        gpu_perm(torch, 1, 16, np.array([0, 1]), np.array([0]), bw=0)


def test_gpu_clustering_headline_size_matches_oracle(torch):
    p = synth.templates()
    note(f"templates M={p.M} nnz={int(p.rp[-1])}")
    want = oracle.jaccard(p.M, p.K, p.rp, p.ci)
    for engine, partners in (("auto", "on"), ("scan", "on"), ("index", "on"), ("auto", "popcount")):
        os.environ["XSPMM_CLUSTER_ENGINE"] = engine
        os.environ["XSPMM_CLUSTER_PARTNERS"] = partners
        try:
            got, used = gpu_perm(torch, p.M, p.K, p.rp, p.ci)
        finally:
            del os.environ["XSPMM_CLUSTER_ENGINE"]
            del os.environ["XSPMM_CLUSTER_PARTNERS"]
        note(f"templates engine={engine} partners={partners} ran={used}")
        np.testing.assert_array_equal(widen(got), want)


def test_gpu_clustering_power_law_graph_matches_host_engine(torch):
    p = synth.gnn()
    note(f"gnn M={p.M} nnz={int(p.rp[-1])}")
    want = X.compute_1d_jaccard_clustering(p.M, p.K, p.rp, p.ci)
    got, used = gpu_perm(torch, p.M, p.K, p.rp, p.ci)
    note(f"gnn engine={used}")
    np.testing.assert_array_equal(widen(got), widen(want))


def many_joins_csr(rng, M, K, n_patterns=40):
    base = [rng.choice(K, size=int(rng.integers(5, 40)), replace=False) for _ in range(n_patterns)]
    rows = []
    for _ in range(M):
        b = base[int(rng.integers(0, len(base)))]
        keep = b[rng.random(len(b)) < 0.9]
        rows.append(np.concatenate([keep, rng.integers(0, K, size=int(rng.integers(0, 3)))]))
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum([len(x) for x in rows])
    return rp, np.concatenate(rows).astype(np.int64)


@pytest.mark.parametrize("W", [1, 4, 5, 8, 9, 16, 17, 28, 32])
def test_gpu_partner_passes_across_bitmap_widths(torch, W, monkeypatch):
    # The matrix-core partner pass stages W words per row (1, 2, 4 or 8 word
    # quads by W) and the popcount pass one of three register widths: both
    # must give the oracle's permutation at every width, for thresholds that
    # make its candidate bound tight (0) or loose (0.8); 700 rows is six
    # 128-row tiles, the last one ragged.
    rng = np.random.default_rng(500 + W)
    M, bw = 700, 16
    K = bw * (64 * (W - 1) + 33)  # Kb = 64 (W - 1) + 33 blocks: W words per row
    rp, ci = many_joins_csr(rng, M, K)
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", "scan")
    for thr in (0.0, 0.3, 0.5, 0.8):
        want = oracle.jaccard(M, K, rp, ci, thr, bw)
        for partners in ("on", "popcount"):
            monkeypatch.setenv("XSPMM_CLUSTER_PARTNERS", partners)
            note(f"bitmap width W={W} thr={thr} partners={partners}")
            got, _ = gpu_perm(torch, M, K, rp, ci, thr, bw)
            np.testing.assert_array_equal(widen(got), want)


@pytest.mark.parametrize("partners", ["on", "popcount", "off"])
def test_gpu_clustering_joins_inside_the_pattern(torch, partners, monkeypatch):
    # The scan engine commits a run of joiners whose rows lie inside the
    # pattern in one step (they leave it as it is), and the all-pairs
    # partner passes stop adding to lists already past their cap: dense
    # pruned-like rows (every pair close, every row joins the first cluster)
    # and nested subsets with some rows that grow the pattern, against the
    # oracle.
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", "scan")
    monkeypatch.setenv("XSPMM_CLUSTER_PARTNERS", partners)
    p = synth.pruned(M=3000, K=1024, N=16, seed=3)
    cases = [(p.M, p.K, p.rp.astype(np.int64), p.ci.astype(np.int64), 0.5, 16)]
    rng = np.random.default_rng(78)
    for thr, bw in ((0.3, 4), (0.5, 8), (0.7, 16)):
        rp, ci = nested_csr(rng, 2500, 2000)
        cases.append((2500, 2000, rp, ci, thr, bw))
    for M, K, rp, ci, thr, bw in cases:
        note(f"inside-pattern joins M={M} thr={thr} bw={bw} partners={partners}")
        want = oracle.jaccard(M, K, rp, ci, thr, bw)
        got, used = gpu_perm(torch, M, K, rp, ci, thr, bw)
        assert used == "scan"
        np.testing.assert_array_equal(widen(got), want)


@pytest.mark.parametrize("itype", [np.int32, np.int64])
@pytest.mark.parametrize("vdtype", [np.float16, np.float32])
def test_pipeline_gpu_clustering_equals_host_clustering(torch, itype, vdtype, monkeypatch):
    # XSPMM_CLUSTER_DEVICE=gpu only moves the clustering stage: C is identical
    rng = np.random.default_rng(41)
    M, K, N = 4000, 3000, 64
    rp, ci = many_joins_csr(rng, M, K)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(vdtype)
    A = X.CSRMatrix.from_host(M, K, rp.astype(itype), ci.astype(itype), vals)
    B = torch.as_tensor(rng.uniform(-1, 1, size=(K, N)).astype(vdtype)).cuda()
    monkeypatch.delenv("XSPMM_CLUSTER_DEVICE", raising=False)
    C_host, _ = X.spmm_pipeline(A, B, optimize_pattern=True)
    monkeypatch.setenv("XSPMM_CLUSTER_DEVICE", "gpu")
    C_gpu, st = X.spmm_pipeline(A, B, optimize_pattern=True)
    torch.cuda.synchronize()
    assert torch.equal(C_host, C_gpu)
    assert st["clustering_ms"] >= 0.0
    perm_host = oracle.jaccard(M, K, rp, ci)
    assert not np.array_equal(perm_host, np.arange(M - 1, -1, -1))  # the clustering joins rows

