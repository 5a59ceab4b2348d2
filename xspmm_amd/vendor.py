"""Vendor-library answers to the same products (libxspmm_vendor.so), for the
benchmark's comparison columns -- the reference's examples time rocSPARSE and
rocBLAS beside xSpMM (examples/04_real_matrices_benchmark.cpp:199-260).

Each function computes C[M x N] fp32 = A * B (fp16 or fp32 inputs, fp32
accumulation, row-major dense operands, int32 indices) on torch's device,
returns (C, mean milliseconds per call over `iters` calls after `warmup`):
  csr_spmm    rocsparse_spmm on the CSR matrix
  bsr_spmm    rocsparse_spmm on the BCSR matrix (16x16 row-major blocks)
  dense_gemm  rocblas_gemm_ex on a dense A
The product library libxspmm.so does not depend on these libraries.
"""
from __future__ import annotations

import ctypes as C
import os

from xspmm_amd import HERE, BCSRMatrix, CSRMatrix, _ptr

VENDOR_PATH = os.path.join(HERE, "libxspmm_vendor.so")
_v = None


def load():
    global _v
    if _v is None:
        if not os.path.exists(VENDOR_PATH):
            raise RuntimeError(f"{VENDOR_PATH} is not built (make -C xspmm_amd/csrc vendor)")
        L = C.CDLL(VENDOR_PATH)
        p, i64, i32 = C.c_void_p, C.c_int64, C.c_int
        L.xv_last_error.restype = C.c_char_p
        L.xv_csr_spmm.restype = i32
        L.xv_csr_spmm.argtypes = [i32, i64, i64, i64, i64, p, p, p, p, p, i32, i32,
                                  C.POINTER(C.c_float)]
        L.xv_bsr_spmm.restype = i32
        L.xv_bsr_spmm.argtypes = [i32, i64, i64, i64, p, p, p, i64, p, p, i32, i32,
                                  C.POINTER(C.c_float)]
        L.xv_dense_gemm.restype = i32
        L.xv_dense_gemm.argtypes = [i32, i64, i64, i64, p, p, p, i32, i32, C.POINTER(C.c_float)]
        _v = L
    return _v


def _vt(dtype):
    import torch
    if dtype == torch.float16:
        return 1
    if dtype == torch.float32:
        return 0
    raise TypeError(f"unsupported value dtype {dtype}")


def _check(rc):
    if rc != 0:
        raise RuntimeError(load().xv_last_error().decode(errors="replace"))


def _out(M, N, like):
    import torch
    return torch.empty((M, N), dtype=torch.float32, device=like.device)


def csr_spmm(A: CSRMatrix, B, warmup=3, iters=20):
    import torch
    if A.row_ptr.dtype != torch.int32:
        raise TypeError("rocSPARSE comparison uses int32 indices")
    N = int(B.shape[1])
    Cm = _out(A.num_rows, N, B)
    ms = C.c_float()
    _check(load().xv_csr_spmm(_vt(A.values.dtype), A.num_rows, A.num_cols, N, A.nnz,
                              _ptr(A.row_ptr), _ptr(A.col_ind), _ptr(A.values), _ptr(B), _ptr(Cm),
                              warmup, iters, C.byref(ms)))
    return Cm, ms.value


def bsr_spmm(Ab: BCSRMatrix, B, warmup=3, iters=20):
    import torch
    if Ab.row_ptr.dtype != torch.int32 or Ab.r_block != 16 or Ab.c_block != 16:
        raise TypeError("rocSPARSE BSR comparison uses int32 indices and 16x16 blocks")
    N = int(B.shape[1])
    if int(B.shape[0]) != Ab.num_block_cols * 16:
        raise ValueError("B must have num_block_cols * 16 rows (pad K to the block grid)")
    Cm = _out(Ab.num_block_rows * 16, N, B)
    ms = C.c_float()
    _check(load().xv_bsr_spmm(_vt(Ab.values.dtype), Ab.num_block_rows, Ab.num_block_cols,
                              Ab.num_blocks, _ptr(Ab.row_ptr), _ptr(Ab.col_ind), _ptr(Ab.values),
                              N, _ptr(B), _ptr(Cm), warmup, iters, C.byref(ms)))
    return Cm[: Ab.num_rows], ms.value


def dense_gemm(A_dense, B, warmup=3, iters=20):
    M, K = int(A_dense.shape[0]), int(A_dense.shape[1])
    N = int(B.shape[1])
    Cm = _out(M, N, B)
    ms = C.c_float()
    _check(load().xv_dense_gemm(_vt(A_dense.dtype), M, K, N, _ptr(A_dense), _ptr(B), _ptr(Cm),
                                warmup, iters, C.byref(ms)))
    return Cm, ms.value
