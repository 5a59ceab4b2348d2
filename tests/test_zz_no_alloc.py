"""The allocation-free Tier-1 entry point (xspmm_bcsr_spmm_noalloc) against
the allocating one (xspmm_bcsr_spmm), both called through the C ABI.

The two share their kernels, so C must be identical bit for bit.  Every case
makes two calls in a row on the same GPU, the second with a smaller input, so
the shared scratch array keeps the first call's contents when the second one
runs.  Cases cover each path that uses scratch (the dispatch order of a grid
of more than 2048 block-rows; the repacked B panels of N % 8 != 0) and paths
that use none (the GEMM-tiled kernel of a full grid, fp32).  A product that
needs more scratch than the array holds is rejected before anything runs.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

import xspmm_amd as X
from xspmm_amd import synth

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X (torch.cuda.is_available() is False)")
    return torch


@pytest.fixture(scope="module")
def lib(torch):
    L = X.load()
    p, i64, i32 = C.c_void_p, C.c_int64, C.c_int
    L.xspmm_bcsr_spmm_noalloc.restype = i32
    L.xspmm_bcsr_spmm_noalloc.argtypes = [i32, i32, i64, i64, i64, i64, i64, p, p, p, p, p, i64, p]
    L.xspmm_noalloc_scratch_bytes.restype = i64
    L.xspmm_noalloc_scratch_bytes.argtypes = []
    return L


def call(L, fn, Bm, B, Cout, N, torch):
    ptr = lambda t: C.c_void_p(t.data_ptr()) if t.numel() else C.c_void_p(0)
    rc = getattr(L, fn)(X.vcode(Bm.values.dtype), X.icode(Bm.row_ptr.dtype), Bm.num_rows,
                        Bm.num_cols, Bm.num_block_rows, Bm.num_block_cols, Bm.num_blocks,
                        ptr(Bm.row_ptr), ptr(Bm.col_ind), ptr(Bm.values), ptr(B), ptr(Cout), N,
                        C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == X.OK, L.xspmm_last_error().decode()


def both(L, Bm, B, N, torch):
    C1 = torch.full((Bm.num_rows, N), float("nan"), dtype=torch.float32, device="cuda")
    C2 = torch.full((Bm.num_rows, N), float("nan"), dtype=torch.float32, device="cuda")
    call(L, "xspmm_bcsr_spmm", Bm, B, C1, N, torch)
    call(L, "xspmm_bcsr_spmm_noalloc", Bm, B, C2, N, torch)
    torch.cuda.synchronize()
    assert bool(torch.isfinite(C1).all())
    return C1, C2


def skewed(M, K, N, seed, dtype=np.float16, itype=np.int32):
    rng = np.random.default_rng(seed)
    deg = np.minimum((rng.pareto(1.2, M) + 1) * 3, K).astype(np.int64)
    rows = [np.sort(rng.choice(K, size=d, replace=False)) for d in deg]
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum(deg)
    ci = np.concatenate(rows)
    vals = rng.uniform(-1, 1, len(ci)).astype(dtype)
    B = rng.standard_normal((K, N)).astype(dtype)
    return X.CSRMatrix.from_host(M, K, rp.astype(itype), ci.astype(itype), vals), B


CASES = [
    # (description, first (M, K, N), second (M, K, N), value dtype, index dtype)
    ("dispatch order", (48000, 4096, 64), (36000, 2048, 64), np.float16, np.int32),
    ("dispatch order int64", (40000, 4096, 128), (33000, 4096, 128), np.float16, np.int64),
    ("panels N % 8 != 0", (3000, 4096, 20), (1000, 512, 12), np.float16, np.int32),
    ("fp32", (5000, 3000, 64), (700, 300, 40), np.float32, np.int32),
    ("fp32 column batches, dispatch order", (40000, 4096, 128), (36000, 2048, 64), np.float32,
     np.int32),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_noalloc_equals_allocating_entry_point(torch, lib, case):
    name, first, second, dtype, itype = case
    for i, (M, K, N) in enumerate((first, second)):
        print(f"noalloc {name} call {i}: M={M} K={K} N={N}", flush=True)
        A, B = skewed(M, K, N, seed=17 + i, dtype=dtype, itype=itype)
        Bm = X.csr_to_bcsr(A)
        Bd = torch.as_tensor(B).cuda()
        C1, C2 = both(lib, Bm, Bd, N, torch)
        assert torch.equal(C1, C2), f"{name} call {i}"


def test_noalloc_full_grid(torch, lib):
    # the GEMM-tiled kernel uses no scratch; two calls, the second smaller
    for i, (M, K, N) in enumerate(((1000, 96, 264), (300, 33, 72))):
        rng = np.random.default_rng(i)
        D = rng.standard_normal((M, K)).astype(np.float16)
        for r in range(0, M, 16):
            for c in range(0, K, 16):
                D[r, c] = np.float16(1.0)
        rp = np.zeros(M + 1, np.int64)
        rp[1:] = np.cumsum((D != 0).sum(axis=1))
        A = X.CSRMatrix.from_host(M, K, rp.astype(np.int32), np.nonzero(D)[1].astype(np.int32),
                                  D[D != 0])
        Bm = X.csr_to_bcsr(A)
        assert Bm.num_blocks == Bm.num_block_rows * Bm.num_block_cols
        Bd = torch.as_tensor(rng.standard_normal((K, N)).astype(np.float16)).cuda()
        C1, C2 = both(lib, Bm, Bd, N, torch)
        assert torch.equal(C1, C2)


def test_noalloc_rejects_products_beyond_its_scratch(torch, lib):
    cap = lib.xspmm_noalloc_scratch_bytes()
    assert cap == 8 << 20
    # a grid of more block-rows than the dispatch order fits: 4 bytes each.
    # Rejected before any launch.  The arrays are real and describe a valid
    # product of empty block-rows (a launch would stay in bounds and write
    # zeros), so C still holding its NaNs shows that nothing ran.
    Mb = cap // 4 + 1
    M, K, N = 16 * Mb, 16, 8
    brp = torch.zeros(Mb + 1, dtype=torch.int32, device="cuda")
    bci = torch.zeros(1, dtype=torch.int32, device="cuda")
    bvals = torch.zeros(256, dtype=torch.float16, device="cuda")
    B = torch.zeros((K, N), dtype=torch.float16, device="cuda")
    Cout = torch.full((M, N), float("nan"), dtype=torch.float32, device="cuda")
    torch.cuda.synchronize()
    vp = lambda t: C.c_void_p(t.data_ptr())
    rc = lib.xspmm_bcsr_spmm_noalloc(X.F16, X.I32, M, K, Mb, 1, 0, vp(brp), vp(bci), vp(bvals),
                                     vp(B), vp(Cout), N,
                                     C.c_void_p(torch.cuda.current_stream().cuda_stream))
    assert rc == X.ERR_INVALID
    assert "scratch" in lib.xspmm_last_error().decode()
    torch.cuda.synchronize()
    assert bool(torch.isnan(Cout).all())
    del Cout
    # the allocation-free path still works afterwards
    A, B = skewed(40000, 1024, 64, seed=5)
    Bm = X.csr_to_bcsr(A)
    C1, C2 = both(lib, Bm, torch.as_tensor(B).cuda(), 64, torch)
    assert torch.equal(C1, C2)


HIP_MEMPOOL_USED_MEM_CURRENT = 0x7   # hipMemPoolAttrUsedMemCurrent
HIP_MEMPOOL_USED_MEM_HIGH = 0x8      # hipMemPoolAttrUsedMemHigh


def test_noalloc_takes_nothing_from_the_pool(torch, lib):
    """The library's temporaries come from the device's default memory pool
    (hipMallocAsync).  Its high-water mark must not rise during
    allocation-free calls on paths that use scratch (dispatch order, B panels,
    fp32 column batches), and must rise during the allocating entry point's
    call on the same product (the positive control)."""
    hip = C.CDLL("libamdhip64.so.7")
    pool = C.c_void_p()
    assert hip.hipDeviceGetDefaultMemPool(C.byref(pool), torch.cuda.current_device()) == 0

    def attr(a):
        v = C.c_uint64(0)
        assert hip.hipMemPoolGetAttribute(pool, a, C.byref(v)) == 0
        return v.value

    def reset_high():
        v = C.c_uint64(0)
        assert hip.hipMemPoolSetAttribute(pool, HIP_MEMPOOL_USED_MEM_HIGH, C.byref(v)) == 0

    for name, (M, K, N), dtype in (("dispatch order", (48000, 4096, 64), np.float16),
                                   ("panels N % 8 != 0", (3000, 4096, 20), np.float16),
                                   ("fp32 dispatch order", (40000, 4096, 128), np.float32)):
        A, B = skewed(M, K, N, seed=3, dtype=dtype)
        Bm = X.csr_to_bcsr(A)
        Bd = torch.as_tensor(B).cuda()
        C1 = torch.empty((M, N), dtype=torch.float32, device="cuda")
        C2 = torch.empty((M, N), dtype=torch.float32, device="cuda")
        torch.cuda.synchronize()
        base = attr(HIP_MEMPOOL_USED_MEM_CURRENT)
        reset_high()
        call(lib, "xspmm_bcsr_spmm_noalloc", Bm, Bd, C2, N, torch)
        call(lib, "xspmm_bcsr_spmm_noalloc", Bm, Bd, C2, N, torch)
        torch.cuda.synchronize()
        high_noalloc = attr(HIP_MEMPOOL_USED_MEM_HIGH)
        reset_high()
        call(lib, "xspmm_bcsr_spmm", Bm, Bd, C1, N, torch)
        torch.cuda.synchronize()
        high_alloc = attr(HIP_MEMPOOL_USED_MEM_HIGH)
        print(f"{name}: pool in use {base} B; high water {high_noalloc} B (allocation-free), "
              f"{high_alloc} B (allocating)", flush=True)
        assert high_noalloc <= base, name
        assert high_alloc > base, name
        assert torch.equal(C1, C2), name
