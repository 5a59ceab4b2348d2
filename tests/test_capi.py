"""CPU: the C-ABI library loads, exports what include/xspmm_capi.h declares,
rejects bad arguments before touching the GPU, and its host clustering (the
product's, not the oracle's) reproduces the reference's permutations."""
from __future__ import annotations

import ctypes as C
import os
import re

import numpy as np
import pytest

import oracle
import xspmm_amd as X
from tests.helpers import golden_cases, nested_csr, widen
from xspmm_amd import synth

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
HEADER = os.path.join(ROOT, "include", "xspmm_capi.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xspmm_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    L = X.load()
    syms = declared_symbols()
    assert len(syms) >= 9
    for s in syms:
        assert hasattr(L, s), s
    assert L.xspmm_abi_version() == 4
    assert L.xspmm_last_error() == b""


def test_bad_type_codes_are_rejected_without_gpu():
    L = X.load()
    rc = L.xspmm_bcsr_spmm(7, X.I32, 16, 16, 1, 1, 0, None, None, None, None, None, 16, None)
    assert rc == X.ERR_INVALID and b"value type" in L.xspmm_last_error()
    rc = L.xspmm_bcsr_spmm(X.F16, 9, 16, 16, 1, 1, 0, None, None, None, None, None, 16, None)
    assert rc == X.ERR_INVALID and b"index type" in L.xspmm_last_error()
    rc = L.xspmm_unpermute_dense(5, None, None, None, 4, 4, None)
    assert rc == X.ERR_INVALID


def test_negative_and_inconsistent_sizes_are_rejected_without_gpu():
    L = X.load()
    assert L.xspmm_bcsr_spmm(X.F16, X.I32, -1, 16, 1, 1, 0, None, None, None, None, None, 16,
                             None) == X.ERR_INVALID
    # element shape larger than the block grid
    assert L.xspmm_bcsr_spmm(X.F16, X.I32, 33, 16, 2, 1, 0, None, None, None, None, None, 16,
                             None) == X.ERR_INVALID
    n = C.c_int64(0)
    assert L.xspmm_csr_to_bcsr_count(X.I32, 4, 4, 0, None, None, 0, 16, None, C.byref(n),
                                     None) == X.ERR_INVALID
    assert L.xspmm_csr_to_bcsr_count(X.I32, 4, 4, 0, None, None, 2000, 16, None, C.byref(n),
                                     None) == X.ERR_INVALID
    assert L.xspmm_csr_to_bcsr_count(X.I32, 4, 4, 0, None, None, 16, 16, None, None,
                                     None) == X.ERR_INVALID
    assert L.xspmm_spmm_pipeline(X.F16, X.I32, 4, 4, 0, None, None, None, None, None, 4, 8, 1,
                                 None, None) == X.ERR_INVALID
    assert b"hw_block_size" in L.xspmm_last_error()


def test_misaligned_operands_are_rejected_without_gpu():
    # the kernels read the block values (and fp16 B) 16 bytes at a time; a
    # pointer off a 16-byte boundary is refused before anything is launched
    # (the addresses below are never dereferenced)
    L = X.load()
    L.xspmm_bcsr_spmm_noalloc.restype = C.c_int
    L.xspmm_bcsr_spmm_noalloc.argtypes = L.xspmm_bcsr_spmm.argtypes
    for entry in (L.xspmm_bcsr_spmm, L.xspmm_bcsr_spmm_noalloc):
        for vt in (X.F16, X.F32):
            rc = entry(vt, X.I32, 16, 16, 1, 1, 1, 0x1000, 0x2000, 0x3008, 0x4000, 0x5000, 16, None)
            assert rc == X.ERR_INVALID, (entry, vt)
            assert b"block values must be 16-byte aligned" in L.xspmm_last_error()
        rc = entry(X.F16, X.I64, 16, 16, 1, 1, 1, 0x1000, 0x2000, 0x3000, 0x4002, 0x5000, 16, None)
        assert rc == X.ERR_INVALID and b"fp16 B must be 16-byte aligned" in L.xspmm_last_error()
    rc = L.xspmm_bcsr_spmm_ordered(X.F16, X.I32, 16, 16, 1, 1, 1, 0x1000, 0x2000, 0x3000, 0x4008,
                                   0x5000, 16, None, None)
    assert rc == X.ERR_INVALID and b"fp16 B must be 16-byte aligned" in L.xspmm_last_error()


def test_noalloc_entry_point_argument_errors_without_gpu():
    # type codes and sizes are checked before the scratch array is looked up
    L = X.load()
    L.xspmm_bcsr_spmm_noalloc.restype = C.c_int
    L.xspmm_bcsr_spmm_noalloc.argtypes = L.xspmm_bcsr_spmm.argtypes
    L.xspmm_noalloc_scratch_bytes.restype = C.c_int64
    assert L.xspmm_noalloc_scratch_bytes() == 8 << 20
    rc = L.xspmm_bcsr_spmm_noalloc(7, X.I32, 16, 16, 1, 1, 0, None, None, None, None, None, 16,
                                   None)
    assert rc == X.ERR_INVALID and b"value type" in L.xspmm_last_error()
    assert L.xspmm_bcsr_spmm_noalloc(X.F16, X.I32, -1, 16, 1, 1, 0, None, None, None, None, None,
                                     16, None) == X.ERR_INVALID
    assert L.xspmm_bcsr_spmm_noalloc(X.F16, X.I32, 33, 16, 2, 1, 0, None, None, None, None, None,
                                     16, None) == X.ERR_INVALID


def test_host_clustering_error_paths():
    with pytest.raises(X.XspmmInvalidArgument):
        X.compute_1d_jaccard_clustering(2, 16, np.array([0, 1, 2], np.int32),
                                        np.array([0, 99], np.int32))
    with pytest.raises(X.XspmmInvalidArgument):
        X.compute_1d_jaccard_clustering(1, 16, np.array([0, 1], np.int32),
                                        np.array([0], np.int32), block_width=0)
    assert len(X.compute_1d_jaccard_clustering(0, 16, np.array([0], np.int32),
                                               np.zeros(0, np.int32))) == 0


def test_device_clustering_argument_errors_without_gpu():
    L = X.load()
    f = L.xspmm_jaccard_clustering
    assert f(X.I32, -1, 16, 0, None, None, 0.5, 16, None, None, None) == X.ERR_INVALID
    assert f(X.I32, 4, -16, 0, None, None, 0.5, 16, None, None, None) == X.ERR_INVALID
    assert f(X.I32, 1, 16, 0, None, None, 0.5, 0, None, None, None) == X.ERR_INVALID
    assert b"block_width" in L.xspmm_last_error()
    assert f(9, 1, 16, 0, None, None, 0.5, 16, None, None, None) == X.ERR_INVALID
    # M = 0: nothing to cluster, no device work
    assert f(X.I64, 0, 16, 0, None, None, 0.5, 16, None, None, None) == X.OK


def test_plan_argument_errors_without_gpu():
    L = X.load()
    h = C.c_void_p()
    create = L.xspmm_plan_create
    assert create(X.F16, X.I32, 4, 4, 0, None, None, None, 16, 1, None, None, None) == X.ERR_INVALID
    assert b"plan_out" in L.xspmm_last_error()
    assert create(X.F16, X.I32, 4, 4, 0, None, None, None, 8, 1, None, None,
                  C.byref(h)) == X.ERR_INVALID
    assert b"hw_block_size" in L.xspmm_last_error() and h.value is None
    assert create(X.F16, X.I32, -4, 4, 0, None, None, None, 16, 1, None, None,
                  C.byref(h)) == X.ERR_INVALID
    assert create(5, X.I32, 4, 4, 0, None, None, None, 16, 1, None, None,
                  C.byref(h)) == X.ERR_INVALID
    assert L.xspmm_plan_execute(None, None, None, 8, None) == X.ERR_INVALID
    assert L.xspmm_plan_info(None, None, None, None, None) == X.ERR_INVALID
    assert L.xspmm_plan_destroy(None) == X.OK


JAC = golden_cases("jaccard")


@pytest.mark.parametrize("engine", ["scan", "index", "auto"])
@pytest.mark.parametrize("case", JAC, ids=[c["name"] for c in JAC])
def test_product_clustering_matches_reference_golden(case, engine, monkeypatch):
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", engine)
    for nthreads in (1, 4):
        perm = X.compute_1d_jaccard_clustering(int(case["M"]), int(case["K"]), case["rp"],
                                               case["ci"], float(case["thresh"]),
                                               int(case["bw"]), nthreads=nthreads)
        assert perm.dtype == case["rp"].dtype
        np.testing.assert_array_equal(widen(perm), widen(case["perm"]))


@pytest.mark.parametrize("engine", ["scan", "index"])
@pytest.mark.parametrize("seed", range(8))
def test_product_clustering_matches_oracle_random(seed, engine, monkeypatch):
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", engine)
    rng = np.random.default_rng(300 + seed)
    M, K = int(rng.integers(1, 2500)), int(rng.integers(16, 3000))
    thr = float([0.5, 0.5, 0.4, 0.5, 0.25, 0.7, 0.5, 0.5][seed])
    bw = [16, 16, 8, 4, 16, 16, 2, 16][seed]
    p = synth.random_csr(M, K, 4, float(rng.uniform(0.001, 0.03)), seed=seed,
                         dtype=np.float32, unsorted=bool(seed % 2))
    want = oracle.jaccard(M, K, p.rp, p.ci, thr, bw)
    got = X.compute_1d_jaccard_clustering(M, K, p.rp, p.ci, thr, bw, nthreads=1 + seed % 4)
    np.testing.assert_array_equal(widen(got), want)


def test_product_clustering_templates_like_input():
    # a scaled-down version of the headline configuration (same generator)
    p = synth.templates(M=2048, n_templates=128, seed=5)
    want = oracle.jaccard(p.M, p.K, p.rp, p.ci)
    for engine in ("scan", "index"):
        os.environ["XSPMM_CLUSTER_ENGINE"] = engine
        try:
            got = X.compute_1d_jaccard_clustering(p.M, p.K, p.rp, p.ci, nthreads=4)
        finally:
            del os.environ["XSPMM_CLUSTER_ENGINE"]
        np.testing.assert_array_equal(widen(got), want)


@pytest.mark.parametrize("n_templates,keep", [(16, 1.0), (64, 1.0), (64, 0.85), (63, 0.85)])
def test_product_clustering_index_partner_lists(n_templates, keep, monkeypatch):
    # the index engine's partner lists (at most 32 per row): 128 identical
    # rows per template overflow them; 32 or 33 rows per template put the
    # partner count at and just past the cap; keep < 1 makes the partners
    # near-duplicates whose joins change the pattern
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", "index")
    p = synth.templates(M=2048, n_templates=n_templates, keep=keep, seed=n_templates)
    want = oracle.jaccard(p.M, p.K, p.rp, p.ci)
    for nthreads in (1, 5):
        got = X.compute_1d_jaccard_clustering(p.M, p.K, p.rp, p.ci, nthreads=nthreads)
        np.testing.assert_array_equal(widen(got), want)


@pytest.mark.parametrize("engine", ["scan", "index"])
def test_product_clustering_joins_inside_the_pattern(engine, monkeypatch):
    # Runs of joiners whose rows lie inside the pattern are committed in one
    # step by the scan engine (they leave the pattern as it is); the
    # permutation must stay the reference's: dense pruned-like rows (every
    # row joins the first cluster) and nested subsets with some rows that
    # grow the pattern, one and four threads, both search forms.
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", engine)
    p = synth.pruned(M=3000, K=1024, N=16, seed=3)
    cases = [(p.M, p.K, p.rp.astype(np.int64), p.ci.astype(np.int64), 0.5, 16)]
    rng = np.random.default_rng(77)
    for thr, bw in ((0.3, 4), (0.5, 8), (0.7, 16)):
        rp, ci = nested_csr(rng, 2500, 2000)
        cases.append((2500, 2000, rp, ci, thr, bw))
    for M, K, rp, ci, thr, bw in cases:
        want = oracle.jaccard(M, K, rp, ci, thr, bw)
        for simd in ("scalar", "auto"):
            monkeypatch.setenv("XSPMM_CLUSTER_SIMD", simd)
            for nthreads in (1, 4):
                got = X.compute_1d_jaccard_clustering(M, K, rp, ci, thr, bw, nthreads=nthreads)
                np.testing.assert_array_equal(widen(got), want)


@pytest.mark.parametrize("simd", ["scalar", "auto"])
def test_product_clustering_scan_search_forms(simd, monkeypatch):
    # the scan engine's search has a scalar and an AVX-512 (vpopcntq) form,
    # picked by the host CPU; both give the reference's permutation (8-word
    # vector steps and a scalar tail)
    monkeypatch.setenv("XSPMM_CLUSTER_ENGINE", "scan")
    monkeypatch.setenv("XSPMM_CLUSTER_SIMD", simd)
    for M, seed in ((1024, 1), (8192, 2), (9216, 3)):  # bitmaps of 1, 8 and 9 words
        p = synth.templates(M=M, n_templates=M // 16, seed=seed)
        want = oracle.jaccard(p.M, p.K, p.rp, p.ci)
        got = X.compute_1d_jaccard_clustering(p.M, p.K, p.rp, p.ci, nthreads=3)
        np.testing.assert_array_equal(widen(got), want)
