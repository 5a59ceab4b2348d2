"""GPU: the Tier-2 pipeline's packed form against its BCSR form.

For fp16 products that the packed kernel covers, the pipeline converts the
(permuted) CSR straight into the column batches that the BCSR column-batch
kernel forms (csr_pack_analyse / csr_pack_emit in convert.hip) and multiplies
them with spmm_f16_packed_kernel, whose store un-permutes.  The batches must
be the BCSR path's byte for byte, so C must equal the pipeline's BCSR form
(XSPMM_PIPELINE_FORMAT=bcsr, the reference's stage sequence
src/hip/unstructured_mtx_mul.hip:31-100) bit for bit.  Inputs outside the
packed form's scope (unsorted or duplicate columns, Inf or NaN values, fully
populated grids, dense blocks) take the BCSR form.

fp32 products take packed batches of four non-zero columns
(spmm_f32_packed_kernel in spmm_f32.hip): the same products summed in
another order, so C is checked against the fp64 product (relative Frobenius
error <= 1e-5, the fp32 bar of the other tests) and against the BCSR form
(<= 1e-6).  Inf and NaN in A stay in the packed form and give the BCSR
form's non-finite entries.
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


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X (torch.cuda.is_available() is False)")
    X.load()
    return torch


@contextlib.contextmanager
def env(name, value):
    old = os.environ.get(name)
    os.environ[name] = value
    try:
        yield
    finally:
        if old is None:
            del os.environ[name]
        else:
            os.environ[name] = old


def both_forms(torch, p, cluster, index=np.int32):
    """C from the packed form and from the BCSR form, and which form ran."""
    A = X.CSRMatrix.from_host(p.M, p.K, p.rp.astype(index), p.ci.astype(index), p.vals)
    B = torch.as_tensor(np.ascontiguousarray(p.B)).cuda()
    C1 = torch.full((p.M, p.N), float("nan"), dtype=torch.float32, device="cuda")
    C0 = torch.full((p.M, p.N), float("nan"), dtype=torch.float32, device="cuda")
    X.spmm_pipeline(A, B, C1, optimize_pattern=cluster, timings=False)
    torch.cuda.synchronize()
    packed = X.pipeline_last_packed()
    with env("XSPMM_PIPELINE_FORMAT", "bcsr"):
        X.spmm_pipeline(A, B, C0, optimize_pattern=cluster, timings=False)
        torch.cuda.synchronize()
        assert not X.pipeline_last_packed()
    return C1.cpu().numpy(), C0.cpu().numpy(), packed


def truth(p):
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    return oracle.bcsr_spmm_f64(p.M, p.K, p.N, brp, bci, bv, p.B)


SHAPES = [
    # M, K, N, density, index, clustering
    (200, 3000, 8, 0.01, np.int32, False),
    (257, 1290, 64, 0.02, np.int64, True),
    (1000, 800, 128, 0.004, np.int32, True),
    (1000, 800, 16, 0.004, np.int32, False),
    (333, 2000, 24, 0.01, np.int64, False),
    (3000, 4096, 256, 0.003, np.int32, True),
    (4100, 4100, 136, 0.002, np.int32, False),
    (600, 5000, 40, 0.02, np.int32, True),
]


@pytest.mark.parametrize("shape", SHAPES, ids=[f"{s[0]}x{s[1]}n{s[2]}d{s[3]}c{int(s[5])}" for s in SHAPES])
def test_packed_form_equals_bcsr_form(torch, shape):
    M, K, N, dens, idx, cluster = shape
    p = synth.random_csr(M, K, N, dens, seed=M + K + N, dtype=np.float16)
    C1, C0, packed = both_forms(torch, p, cluster, idx)
    print(f"{M}x{K} N={N} d={dens} cluster={cluster}: packed form {packed}", flush=True)
    assert packed
    assert np.all(np.isfinite(C1))
    assert C1.tobytes() == C0.tobytes()
    e = oracle.errors(C1, truth(p))
    assert e["rel_frob"] <= 2e-3, e


def special_values(seed=7, M=600, K=900, N=64):
    """Explicit zeros, -0.0 entries, an all-zero block kept in the structure,
    fp16 subnormals and large magnitudes, empty rows and a ragged last strip."""
    rng = np.random.default_rng(seed)
    rows = []
    for r in range(M):
        if r % 37 == 0:
            rows.append(np.zeros(0, np.int64))
            continue
        k = rng.binomial(K, 0.01)
        rows.append(np.sort(rng.choice(K, size=k, replace=False)))
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum([len(r) for r in rows])
    ci = np.concatenate(rows).astype(np.int32)
    vals = rng.uniform(-1, 1, len(ci)).astype(np.float16)
    vals[::11] = np.float16(0.0)
    vals[5::13] = np.float16(-0.0)
    vals[7::17] = np.float16(6.0e-8)      # subnormal
    vals[3::19] = np.float16(-6.0e4)
    # rows 40..55 (strip 2 and 3): columns 480..487 only, all explicit zeros
    for r in range(40, 56):
        s, e = rp[r], rp[r + 1]
        sel = (ci[s:e] >= 480) & (ci[s:e] < 496)
        vals[s:e][sel] = np.float16(0.0)
    B = rng.uniform(-1, 1, size=(K, N)).astype(np.float16)
    return synth.Problem("special", M, K, N, rp.astype(np.int32), ci, vals, B)


@pytest.mark.parametrize("cluster", [False, True])
def test_packed_form_special_values(torch, cluster):
    p = special_values()
    C1, C0, packed = both_forms(torch, p, cluster)
    assert packed
    assert C1.tobytes() == C0.tobytes()
    assert np.all(C1[::37] == 0.0)


def test_unsorted_or_duplicate_columns_take_bcsr(torch):
    p = synth.random_csr(500, 700, 64, 0.02, seed=3, dtype=np.float16, unsorted=True,
                         dup_frac=0.05)
    C1, C0, packed = both_forms(torch, p, True)
    assert not packed
    assert C1.tobytes() == C0.tobytes()


def test_nonfinite_values_take_bcsr(torch):
    p = synth.random_csr(500, 700, 64, 0.02, seed=4, dtype=np.float16)
    p.vals[int(p.rp[10])] = np.float16(np.inf)
    C1, C0, packed = both_forms(torch, p, False)
    assert not packed
    assert C1.tobytes() == C0.tobytes()


def test_dense_blocks_take_bcsr(torch):
    """configs[1]-like dense blocks: batches would not save a quarter of the
    block bytes, so the BCSR kernels run."""
    p = synth.blocks(M=1024, N=64)
    C1, C0, packed = both_forms(torch, p, False)
    assert not packed
    assert C1.tobytes() == C0.tobytes()


@pytest.mark.slow
def test_templates_full_size(torch):
    p = synth.templates()
    with env("XSPMM_CLUSTER_DEVICE", "gpu"):
        C1, C0, packed = both_forms(torch, p, True)
    assert packed
    assert C1.tobytes() == C0.tobytes()


@pytest.mark.slow
def test_gnn_full_size(torch):
    """131072 rows, more than 2048 block-rows: the packed product takes the
    dispatch order, and long rows make long per-wave batch chains."""
    p = synth.gnn()
    with env("XSPMM_CLUSTER_DEVICE", "gpu"):
        C1, C0, packed = both_forms(torch, p, True)
    assert packed
    assert C1.tobytes() == C0.tobytes()


F32_SHAPES = [
    # M, K, N, density, index, clustering
    (200, 3000, 8, 0.01, np.int32, False),
    (257, 1290, 64, 0.02, np.int64, True),
    (1000, 800, 128, 0.004, np.int32, True),
    (333, 2000, 20, 0.01, np.int64, False),
    (3000, 4096, 256, 0.003, np.int32, True),
    (600, 5000, 44, 0.02, np.int32, True),
    (4100, 4100, 132, 0.002, np.int32, False),
]


def rel(a, b):
    a = a.astype(np.float64)
    b = b.astype(np.float64)
    return float(np.linalg.norm(a - b) / max(np.linalg.norm(b), 1e-300))


@pytest.mark.parametrize("shape", F32_SHAPES,
                         ids=[f"{s[0]}x{s[1]}n{s[2]}d{s[3]}c{int(s[5])}" for s in F32_SHAPES])
def test_fp32_packed_form(torch, shape):
    M, K, N, dens, idx, cluster = shape
    p = synth.random_csr(M, K, N, dens, seed=M + K + N + 1, dtype=np.float32)
    C1, C0, packed = both_forms(torch, p, cluster, idx)
    print(f"fp32 {M}x{K} N={N} d={dens} cluster={cluster}: packed form {packed}", flush=True)
    assert packed
    assert np.all(np.isfinite(C1))
    e = oracle.errors(C1, truth(p))
    assert e["rel_frob"] <= 1e-5, e
    assert rel(C1, C0) <= 1e-6


def fp32_special_values(seed=8, M=600, K=900, N=64):
    """fp32: explicit +-0 entries, an all-zero block, subnormals, large
    magnitudes, empty rows and a ragged last strip."""
    rng = np.random.default_rng(seed)
    p = special_values(seed, M, K, N)
    vals = rng.uniform(-1, 1, p.nnz).astype(np.float32)
    vals[::11] = np.float32(0.0)
    vals[5::13] = np.float32(-0.0)
    vals[7::17] = np.float32(1e-40)  # subnormal
    vals[3::19] = np.float32(-3e30)
    for r in range(40, 56):
        s, e = p.rp[r], p.rp[r + 1]
        sel = (p.ci[s:e] >= 480) & (p.ci[s:e] < 496)
        vals[s:e][sel] = np.float32(0.0)
    B = rng.uniform(-1, 1, size=(K, N)).astype(np.float32)
    return synth.Problem("special32", M, K, N, p.rp, p.ci, vals, B)


@pytest.mark.parametrize("cluster", [False, True])
def test_fp32_packed_form_special_values(torch, cluster):
    p = fp32_special_values()
    C1, C0, packed = both_forms(torch, p, cluster)
    assert packed
    assert np.all(C1[::37] == 0.0)
    assert oracle.errors(C1, truth(p))["rel_frob"] <= 1e-5
    assert rel(C1, C0) <= 1e-6


def test_fp32_nonfinite_a_stays_packed(torch):
    """Inf and NaN in A: the packed form runs and gives the BCSR form's
    non-finite entries; the finite entries agree."""
    p = synth.random_csr(500, 700, 64, 0.02, seed=9, dtype=np.float32)
    p.vals[int(p.rp[10])] = np.float32(np.inf)
    p.vals[int(p.rp[200]) + 1] = np.float32(np.nan)
    C1, C0, packed = both_forms(torch, p, False)
    assert packed
    fin1, fin0 = np.isfinite(C1), np.isfinite(C0)
    assert np.array_equal(fin1, fin0)
    assert np.array_equal(np.isnan(C1), np.isnan(C0))
    assert np.array_equal(np.isposinf(C1), np.isposinf(C0))
    assert not fin1.all()
    assert rel(np.where(fin1, C1, 0), np.where(fin0, C0, 0)) <= 1e-6


def test_fp32_unsorted_columns_take_bcsr(torch):
    p = synth.random_csr(500, 700, 64, 0.02, seed=10, dtype=np.float32, unsorted=True,
                         dup_frac=0.05)
    C1, C0, packed = both_forms(torch, p, True)
    assert not packed
    assert C1.tobytes() == C0.tobytes()


def test_fp32_dense_blocks_take_bcsr(torch):
    """Full blocks make 4 batches (1088 B) per block (1024 B): the BCSR form
    runs."""
    p = synth.blocks(M=1024, N=64, dtype=np.float32)
    C1, C0, packed = both_forms(torch, p, False)
    assert not packed
    assert C1.tobytes() == C0.tobytes()


@pytest.mark.slow
def test_fp32_templates_full_size(torch):
    p = synth.templates(dtype=np.float32)
    with env("XSPMM_CLUSTER_DEVICE", "gpu"):
        C1, C0, packed = both_forms(torch, p, True)
    assert packed
    assert rel(C1, C0) <= 1e-6


def heavy_strips(dtype, seed=11, M=2000, K=40000, N=64):
    """Strips of more than 1024 column blocks (the emit kernels' heavy
    launch): 24 rows of 1800 random columns among sparse ones, on a grid of
    2500 column blocks."""
    rng = np.random.default_rng(seed)
    heavy = set(rng.choice(M, size=24, replace=False).tolist())
    rows = []
    for r in range(M):
        k = 1800 if r in heavy else rng.binomial(K, 0.0008)
        rows.append(np.sort(rng.choice(K, size=k, replace=False)))
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum([len(x) for x in rows])
    ci = np.concatenate(rows).astype(np.int32)
    vals = rng.uniform(-1, 1, len(ci)).astype(dtype)
    B = rng.uniform(-1, 1, size=(K, N)).astype(dtype)
    return synth.Problem("heavy", M, K, N, rp.astype(np.int32), ci, vals, B)


@pytest.mark.parametrize("dtype", [np.float16, np.float32])
@pytest.mark.parametrize("cluster", [False, True])
def test_heavy_strips(torch, dtype, cluster):
    p = heavy_strips(dtype)
    brp, _, _ = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    assert np.diff(brp).max() > 1024
    C1, C0, packed = both_forms(torch, p, cluster)
    assert packed
    if dtype == np.float16:
        assert C1.tobytes() == C0.tobytes()
    else:
        assert rel(C1, C0) <= 1e-6
    assert oracle.errors(C1, truth(p))["rel_frob"] <= (2e-3 if dtype == np.float16 else 1e-5)
