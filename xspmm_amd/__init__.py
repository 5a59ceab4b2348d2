"""xspmm_amd -- MI355X-native xSpMM SpMM hot path.

The product is ``libxspmm.so`` (built from ``xspmm_amd/csrc`` with hipcc for
gfx950): hand-written HIP kernels behind the reference's C++ API
(``include/xspmm/*.hpp``) and a flat C ABI (``include/xspmm_capi.h``).

This module is the Python view of that C ABI.  It mirrors the reference's
operator interface -- ``CSRMatrix``, ``BCSRMatrix``, ``csr_to_bcsr``,
``compute_1d_jaccard_clustering``, ``apply_permutation``, Tier-1 ``spmm``,
the Tier-2 pipeline ``spmm_pipeline`` and ``unpermute_dense_matrix`` -- with
torch tensors as device buffers.  Every call goes to the HIP library; there
is no CPU fallback, and importing the library fails loudly when it has not
been built.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass, field

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
# XSPMM_LIBRARY selects another build of the library (same C ABI).
LIB_PATH = os.environ.get("XSPMM_LIBRARY") or os.path.join(HERE, "libxspmm.so")

F32, F16 = 0, 1
I32, I64 = 0, 1
OK, ERR_INVALID, ERR_HIP, ERR_UNSUPPORTED, ERR_IO = 0, 1, 2, 3, 4

TIMING_FIELDS = ("clustering_ms", "permutation_ms", "conversion_ms", "spmm_ms",
                 "unpermutation_ms", "total_pipeline_ms")

_lib = None


class XspmmError(RuntimeError):
    """A HIP or unsupported-operation failure reported by libxspmm."""

    def __init__(self, code: int, msg: str):
        super().__init__(msg)
        self.code = code


class XspmmInvalidArgument(XspmmError, ValueError):
    """std::invalid_argument in the C++ API."""


def load():
    """Load libxspmm.so (raises if it was not built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() "
                           "(make -C xspmm_amd/csrc)")
    L = C.CDLL(LIB_PATH)
    p, i64, i32 = C.c_void_p, C.c_int64, C.c_int
    L.xspmm_last_error.restype = C.c_char_p
    L.xspmm_last_error.argtypes = []
    L.xspmm_abi_version.restype = i32
    L.xspmm_abi_version.argtypes = []
    L.xspmm_bcsr_spmm.restype = i32
    L.xspmm_bcsr_spmm.argtypes = [i32, i32, i64, i64, i64, i64, i64, p, p, p, p, p, i64, p]
    L.xspmm_bcsr_spmm_ordered.restype = i32
    L.xspmm_bcsr_spmm_ordered.argtypes = [i32, i32, i64, i64, i64, i64, i64, p, p, p, p, p, i64,
                                          p, p]
    L.xspmm_bcsr_dispatch_order.restype = i32
    L.xspmm_bcsr_dispatch_order.argtypes = [i32, i64, p, p, C.POINTER(C.c_int), p]
    L.xspmm_bcsr_band_rows.restype = i32
    L.xspmm_bcsr_band_rows.argtypes = [i32, i32, i64, i64, i64, i64, i64, i64, p, p, C.POINTER(C.c_int), p]
    L.xspmm_bcsr_spmm_band.restype = i32
    L.xspmm_bcsr_spmm_band.argtypes = [i32, i32, i64, i64, i64, i64, i64, p, p, p, p, p, i64, p]
    L.xspmm_bcsr_dispatch_order_cols.restype = i32
    L.xspmm_bcsr_dispatch_order_cols.argtypes = [i32, i64, p, p, p, C.POINTER(C.c_int), p]
    L.xspmm_csr_to_bcsr_count.restype = i32
    L.xspmm_csr_to_bcsr_count.argtypes = [i32, i64, i64, i64, p, p, i64, i64, p,
                                          C.POINTER(C.c_int64), p]
    L.xspmm_csr_to_bcsr_fill.restype = i32
    L.xspmm_csr_to_bcsr_fill.argtypes = [i32, i32, i64, i64, i64, p, p, p, i64, i64, p, p, p, p]
    L.xspmm_apply_permutation.restype = i32
    L.xspmm_apply_permutation.argtypes = [i32, i32, i64, i64, p, p, p, p, p, p, p, p]
    L.xspmm_unpermute_dense.restype = i32
    L.xspmm_unpermute_dense.argtypes = [i32, p, p, p, i64, i64, p]
    L.xspmm_jaccard_clustering_host.restype = i32
    L.xspmm_jaccard_clustering_host.argtypes = [i32, i64, i64, p, p, C.c_float, i64, p, i32]
    L.xspmm_jaccard_clustering.restype = i32
    L.xspmm_jaccard_clustering.argtypes = [i32, i64, i64, i64, p, p, C.c_float, i64, p,
                                           C.POINTER(C.c_int), p]
    L.xspmm_plan_create.restype = i32
    L.xspmm_plan_create.argtypes = [i32, i32, i64, i64, i64, p, p, p, i64, i32,
                                    C.POINTER(C.c_double), p, C.POINTER(C.c_void_p)]
    L.xspmm_plan_execute.restype = i32
    L.xspmm_plan_execute.argtypes = [p, p, p, i64, p]
    L.xspmm_plan_info.restype = i32
    L.xspmm_plan_info.argtypes = [p, C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                  C.POINTER(C.c_int), C.POINTER(C.c_void_p)]
    L.xspmm_plan_packed_batches.restype = i32
    L.xspmm_plan_packed_batches.argtypes = [p, C.POINTER(C.c_int64)]
    L.xspmm_plan_destroy.restype = i32
    L.xspmm_plan_destroy.argtypes = [p]
    L.xspmm_mtx_read.restype = i32
    L.xspmm_mtx_read.argtypes = [C.c_char_p, C.POINTER(C.c_void_p)]
    L.xspmm_mtx_info.restype = i32
    L.xspmm_mtx_info.argtypes = [p, C.POINTER(C.c_int64), C.POINTER(C.c_int64),
                                 C.POINTER(C.c_int64)]
    L.xspmm_mtx_export.restype = i32
    L.xspmm_mtx_export.argtypes = [p, i32, i32, p, p, p]
    L.xspmm_mtx_free.restype = i32
    L.xspmm_mtx_free.argtypes = [p]
    L.xspmm_pipeline_last_form.restype = i32
    L.xspmm_pipeline_last_form.argtypes = [C.POINTER(C.c_int)]
    L.xspmm_pipeline_temp_bytes.restype = i32
    L.xspmm_pipeline_temp_bytes.argtypes = [C.POINTER(C.c_int64)]
    L.xspmm_spmm_pipeline.restype = i32
    L.xspmm_spmm_pipeline.argtypes = [i32, i32, i64, i64, i64, p, p, p, p, p, i64, i64, i32,
                                      C.POINTER(C.c_double), p]
    _lib = L
    return L


def _check(rc: int):
    if rc == OK:
        return
    msg = load().xspmm_last_error().decode(errors="replace")
    if rc == ERR_INVALID:
        raise XspmmInvalidArgument(rc, msg)
    raise XspmmError(rc, msg)


# ---------------------------------------------------------------------------
# type codes / pointers
# ---------------------------------------------------------------------------

def _torch():
    import torch
    return torch


def vcode(dtype) -> int:
    torch = _torch()
    if dtype in (torch.float16, np.float16):
        return F16
    if dtype in (torch.float32, np.float32):
        return F32
    raise TypeError(f"unsupported value dtype {dtype}")


def icode(dtype) -> int:
    torch = _torch()
    if dtype in (torch.int32, np.int32):
        return I32
    if dtype in (torch.int64, np.int64):
        return I64
    raise TypeError(f"unsupported index dtype {dtype}")


def _ptr(t):
    return C.c_void_p(t.data_ptr()) if t is not None and t.numel() > 0 else C.c_void_p(0)


def _stream():
    torch = _torch()
    return C.c_void_p(torch.cuda.current_stream().cuda_stream)


def _device(dev=None):
    torch = _torch()
    if dev is None:
        dev = torch.device("cuda", torch.cuda.current_device())
    return torch.device(dev)


def _check_dense(t, name, rows, cols, dtype, device):
    """Reject a dense operand the kernels cannot take as given: the kernels
    read `rows` x `cols` elements row-major (ld = cols) from t.data_ptr() on
    `device`, and read fp16 B with 16-byte vector loads, so an fp16 B must
    start on a 16-byte boundary.  Raised before any kernel is launched."""
    torch = _torch()
    if not torch.is_tensor(t):
        raise TypeError(f"{name} must be a torch tensor")
    if t.dtype != dtype:
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if t.device != torch.device(device):
        raise ValueError(f"{name} is on {t.device}, the matrix is on {device}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous (row-major, ld = number of columns)")
    shape = tuple(t.shape)
    if t.dim() == 2:
        ok = shape == (rows, cols)
    else:
        ok = t.dim() == 1 and t.numel() == rows * cols
    if not ok:
        raise ValueError(f"{name} has shape {shape}, expected ({rows}, {cols})")
    if name == "B" and dtype == torch.float16 and t.data_ptr() % 16 != 0:
        raise ValueError(f"{name} must start on a 16-byte boundary (fp16 rows are read 16 bytes at a time)")


# ---------------------------------------------------------------------------
# matrices
# ---------------------------------------------------------------------------

@dataclass
class CSRMatrix:
    """Device CSR matrix (reference include/xspmm/matrix/csr.hpp:12-71)."""
    num_rows: int
    num_cols: int
    row_ptr: object   # torch int32/int64 [M+1]
    col_ind: object   # [nnz]
    values: object    # torch float16/float32 [nnz]

    @property
    def nnz(self) -> int:
        return int(self.col_ind.numel())

    @classmethod
    def from_host(cls, M, K, rp, ci, vals, device=None, index_dtype=None):
        torch = _torch()
        dev = _device(device)
        rp = np.asarray(rp)
        idt = index_dtype or rp.dtype
        it = torch.int32 if np.dtype(idt) == np.int32 else torch.int64
        return cls(int(M), int(K),
                   torch.as_tensor(np.ascontiguousarray(rp)).to(dev, it),
                   torch.as_tensor(np.ascontiguousarray(ci)).to(dev, it),
                   torch.as_tensor(np.ascontiguousarray(vals)).to(dev))


@dataclass
class BCSRMatrix:
    """Device BCSR matrix (reference include/xspmm/matrix/bcsr.hpp:12-116),
    plus the element shape num_rows x num_cols."""
    num_block_rows: int
    num_block_cols: int
    r_block: int
    c_block: int
    num_rows: int
    num_cols: int
    row_ptr: object   # [Mb+1]
    col_ind: object   # [nnzb]
    values: object    # [nnzb * r * c]
    # The Tier-1 column-batch kernels' dispatch order (block-row ids: longest
    # rows first above 2048 block-rows, else a contiguous range of block-rows
    # per XCD for short, alike neighbouring rows, or the identity; see
    # xspmm_bcsr_dispatch_order_cols), computed once for grids of at least
    # 256 block-rows and kept with the row_ptr and col_ind tensors it came
    # from (their identities and versions).
    _order: object = field(default=None, repr=False, compare=False)
    _order_key: object = field(default=None, repr=False, compare=False)
    # Whether Tier-1 takes a band kernel (every block-row a contiguous run of
    # block columns, see xspmm_bcsr_band_rows), decided once for the same
    # tensors as the order; _nnz: CSR entries behind the grid (0: not known),
    # which csr_to_bcsr records.
    _band: object = field(default=None, repr=False, compare=False)
    _band_key: object = field(default=None, repr=False, compare=False)
    _nnz: int = field(default=0, repr=False, compare=False)

    @property
    def num_blocks(self) -> int:
        return int(self.col_ind.numel())

    def dispatch_order(self):
        """The cached dispatch order for the current row_ptr (computed on
        first use), or None when Tier-1 does not order this grid."""
        key = (id(self.row_ptr), self.row_ptr.data_ptr(), self.row_ptr._version,
               id(self.col_ind), self.col_ind.data_ptr(), self.col_ind._version,
               int(self.num_block_rows))
        if self._order_key != key:
            torch = _torch()
            order = torch.empty(int(self.num_block_rows) + 1, dtype=torch.int32,
                                device=self.row_ptr.device)
            written = C.c_int(0)
            _check(load().xspmm_bcsr_dispatch_order_cols(icode(self.row_ptr.dtype),
                                                         int(self.num_block_rows), _ptr(self.row_ptr),
                                                         _ptr(self.col_ind), _ptr(order),
                                                         C.byref(written), _stream()))
            self._order = order[:int(self.num_block_rows)] if written.value else None
            self._order_key = key
        return self._order

    def band_rows(self) -> bool:
        """Whether Tier-1 multiplies this grid with a band kernel (decided on
        first use for the current row_ptr and col_ind)."""
        key = (id(self.row_ptr), self.row_ptr.data_ptr(), self.row_ptr._version,
               id(self.col_ind), self.col_ind.data_ptr(), self.col_ind._version,
               int(self.num_block_rows))
        if self._band_key != key:
            band = C.c_int(0)
            if self.r_block == 16 and self.c_block == 16:
                _check(load().xspmm_bcsr_band_rows(vcode(self.values.dtype), icode(self.row_ptr.dtype),
                                                   int(self.num_rows),
                                                   int(self.num_cols), int(self.num_block_rows),
                                                   int(self.num_block_cols), int(self._nnz),
                                                   self.num_blocks, _ptr(self.row_ptr),
                                                   _ptr(self.col_ind), C.byref(band), _stream()))
            self._band = bool(band.value)
            self._band_key = key
        return self._band


# ---------------------------------------------------------------------------
# operations
# ---------------------------------------------------------------------------

def csr_to_bcsr(A: CSRMatrix, r_block: int = 16, c_block: int = 16) -> BCSRMatrix:
    """GPU CSR -> BCSR (reference include/xspmm/matrix/conversion.hpp:19-22)."""
    torch = _torch()
    L = load()
    dev = A.row_ptr.device
    it = A.row_ptr.dtype
    Mb = (A.num_rows + r_block - 1) // r_block
    Kb = (A.num_cols + c_block - 1) // c_block
    brp = torch.empty(Mb + 1, dtype=it, device=dev)
    nnzb = C.c_int64(0)
    _check(L.xspmm_csr_to_bcsr_count(icode(it), A.num_rows, A.num_cols, A.nnz, _ptr(A.row_ptr),
                                     _ptr(A.col_ind), r_block, c_block, _ptr(brp),
                                     C.byref(nnzb), _stream()))
    n = nnzb.value
    bci = torch.empty(max(n, 0), dtype=it, device=dev)
    bv = torch.empty(max(n, 0) * r_block * c_block, dtype=A.values.dtype, device=dev)
    _check(L.xspmm_csr_to_bcsr_fill(vcode(A.values.dtype), icode(it), A.num_rows, A.num_cols,
                                    A.nnz, _ptr(A.row_ptr), _ptr(A.col_ind), _ptr(A.values),
                                    r_block, c_block, _ptr(brp), _ptr(bci), _ptr(bv), _stream()))
    out = BCSRMatrix(Mb, Kb, r_block, c_block, A.num_rows, A.num_cols, brp, bci, bv)
    out._nnz = int(A.nnz)
    if r_block == 16 and c_block == 16:
        out.dispatch_order()  # once here rather than in every Tier-1 call
        out.band_rows()
    return out


def spmm(A: BCSRMatrix, B, C_out=None, N: int | None = None):
    """Tier-1 C = A * B (reference include/xspmm/xspmm.hpp:14-18).  B is
    K x N row-major on the device; returns C (M x N fp32)."""
    torch = _torch()
    L = load()
    if N is None:
        N = int(B.shape[1]) if B.dim() == 2 else int(B.numel() // max(A.num_cols, 1))
    dev = A.row_ptr.device
    if C_out is None:
        C_out = torch.empty((A.num_rows, N), dtype=torch.float32, device=dev)
    _check_dense(B, "B", A.num_cols, N, A.values.dtype, dev)
    _check_dense(C_out, "C_out", A.num_rows, N, torch.float32, dev)
    if A.band_rows():
        _check(L.xspmm_bcsr_spmm_band(vcode(B.dtype), icode(A.row_ptr.dtype), A.num_rows, A.num_cols,
                                      A.num_block_rows, A.num_block_cols, A.num_blocks,
                                      _ptr(A.row_ptr), _ptr(A.col_ind), _ptr(A.values), _ptr(B),
                                      _ptr(C_out), N, _stream()))
        return C_out
    order = A.dispatch_order()
    _check(L.xspmm_bcsr_spmm_ordered(vcode(B.dtype), icode(A.row_ptr.dtype), A.num_rows,
                                     A.num_cols, A.num_block_rows, A.num_block_cols, A.num_blocks,
                                     _ptr(A.row_ptr), _ptr(A.col_ind), _ptr(A.values), _ptr(B),
                                     _ptr(C_out), N, _ptr(order) if order is not None else None,
                                     _stream()))
    return C_out


def compute_1d_jaccard_clustering(M, K, rp, ci, dist_thresh=0.5, block_width=16, nthreads=0):
    """Host Jaccard clustering on host arrays -> perm (numpy, same dtype as rp)
    (reference include/xspmm/clustering.hpp:19-25)."""
    L = load()
    rp = np.ascontiguousarray(rp)
    ci = np.ascontiguousarray(ci, dtype=rp.dtype)
    perm = np.zeros(max(int(M), 1), dtype=rp.dtype)
    _check(L.xspmm_jaccard_clustering_host(icode(rp.dtype), int(M), int(K),
                                           rp.ctypes.data_as(C.c_void_p),
                                           ci.ctypes.data_as(C.c_void_p) if ci.size else None,
                                           C.c_float(dist_thresh), int(block_width),
                                           perm.ctypes.data_as(C.c_void_p), int(nthreads)))
    return perm[: int(M)]


CLUSTER_ENGINES = {0: "closed-form", 1: "scan", 2: "index"}


def jaccard_clustering(A: CSRMatrix, dist_thresh=0.5, block_width=16, return_engine=False):
    """GPU Jaccard clustering of a device CSR matrix -> device perm tensor
    (perm[new] = old), the same permutation as the host greedy
    (reference include/xspmm/clustering.hpp:19-25, src/cpu/clustering_sylos_labini.cpp:51-120).
    Synchronizes torch's current stream.  With return_engine, also returns
    the engine that ran ("closed-form", "scan" or "index")."""
    torch = _torch()
    L = load()
    M = int(A.num_rows)
    perm = torch.empty(max(M, 1), dtype=A.row_ptr.dtype, device=A.row_ptr.device)
    used = C.c_int(-1)
    _check(L.xspmm_jaccard_clustering(icode(A.row_ptr.dtype), M, int(A.num_cols), A.nnz,
                                      _ptr(A.row_ptr), _ptr(A.col_ind) if A.nnz else None,
                                      C.c_float(dist_thresh), int(block_width), _ptr(perm),
                                      C.byref(used), _stream()))
    perm = perm[:M]
    if return_engine:
        return perm, CLUSTER_ENGINES.get(used.value, "none")
    return perm


def read_mtx(path, index_dtype=np.int32, value_dtype=np.float32):
    """MatrixMarket coordinate file -> (M, K, row_ptr, col_ind, values) as
    host numpy arrays, the matrix the reference's reader gives
    (utils/matrix_io.hpp:27-98).  Raises XspmmError (code ERR_IO) with the
    reference's message when the file cannot be opened or parsed."""
    L = load()
    h = C.c_void_p()
    _check(L.xspmm_mtx_read(os.fsencode(os.fspath(path)), C.byref(h)))
    try:
        M, K, n = C.c_int64(), C.c_int64(), C.c_int64()
        _check(L.xspmm_mtx_info(h, C.byref(M), C.byref(K), C.byref(n)))
        nnz = n.value
        rp = np.zeros(max(M.value, 0) + 1, index_dtype)
        ci = np.zeros(max(nnz, 1), index_dtype)
        vals = np.zeros(max(nnz, 1), value_dtype)
        _check(L.xspmm_mtx_export(h, icode(rp.dtype), vcode(vals.dtype),
                                  rp.ctypes.data_as(C.c_void_p), ci.ctypes.data_as(C.c_void_p),
                                  vals.ctypes.data_as(C.c_void_p)))
    finally:
        L.xspmm_mtx_free(h)
    return M.value, K.value, rp, ci[:nnz], vals[:nnz]


def apply_permutation(A: CSRMatrix, perm) -> CSRMatrix:
    """GPU row permutation (reference include/xspmm/clustering.hpp:34-38)."""
    torch = _torch()
    L = load()
    dev = A.row_ptr.device
    it = A.row_ptr.dtype
    perm_t = torch.as_tensor(perm).to(dev, it) if not torch.is_tensor(perm) else perm.to(dev, it)
    nrp = torch.empty(A.num_rows + 1, dtype=it, device=dev)
    nci = torch.empty_like(A.col_ind)
    nv = torch.empty_like(A.values)
    _check(L.xspmm_apply_permutation(vcode(A.values.dtype), icode(it), A.num_rows, A.nnz,
                                     _ptr(A.row_ptr), _ptr(A.col_ind), _ptr(A.values),
                                     _ptr(perm_t), _ptr(nrp), _ptr(nci), _ptr(nv), _stream()))
    return CSRMatrix(A.num_rows, A.num_cols, nrp, nci, nv)


def unpermute_dense_matrix(C_in, perm, out=None):
    """out[perm[r], :] = C_in[r, :] (reference include/xspmm/xspmm.hpp:35-40)."""
    torch = _torch()
    L = load()
    M, N = int(C_in.shape[0]), int(C_in.shape[1])
    if out is None:
        out = torch.empty_like(C_in)
    _check_dense(C_in, "C_in", M, N, torch.float32, C_in.device)
    _check_dense(out, "out", M, N, torch.float32, C_in.device)
    perm_t = perm if torch.is_tensor(perm) else torch.as_tensor(np.asarray(perm)).to(C_in.device)
    if perm_t.device != C_in.device or perm_t.dim() != 1 or perm_t.numel() != M:
        raise ValueError(f"perm must be a 1-D tensor of {M} entries on {C_in.device}")
    perm_t = perm_t.contiguous()
    _check(L.xspmm_unpermute_dense(icode(perm_t.dtype), _ptr(C_in), _ptr(out), _ptr(perm_t), M, N,
                                   _stream()))
    return out


def spmm_pipeline(A: CSRMatrix, B, C_out=None, N: int | None = None, hw_block_size: int = 16,
                  optimize_pattern: bool = True, timings: bool = True):
    """Tier-2 pipeline (reference include/xspmm/xspmm.hpp:24-32).
    Returns (C, timings dict or None)."""
    torch = _torch()
    L = load()
    if N is None:
        N = int(B.shape[1])
    dev = A.row_ptr.device
    if C_out is None:
        C_out = torch.empty((A.num_rows, N), dtype=torch.float32, device=dev)
    _check_dense(B, "B", A.num_cols, N, A.values.dtype, dev)
    _check_dense(C_out, "C_out", A.num_rows, N, torch.float32, dev)
    t = (C.c_double * 6)() if timings else None
    _check(L.xspmm_spmm_pipeline(vcode(A.values.dtype), icode(A.row_ptr.dtype), A.num_rows,
                                 A.num_cols, A.nnz, _ptr(A.row_ptr), _ptr(A.col_ind),
                                 _ptr(A.values), _ptr(B), _ptr(C_out), N, hw_block_size,
                                 1 if optimize_pattern else 0,
                                 C.cast(t, C.POINTER(C.c_double)) if t is not None else None,
                                 _stream()))
    return C_out, (dict(zip(TIMING_FIELDS, list(t))) if t is not None else None)


def pipeline_temp_bytes() -> int:
    """Device bytes of the temporaries the last spmm_pipeline call on this
    thread took (C ABI xspmm_pipeline_temp_bytes)."""
    out = C.c_int64(0)
    _check(load().xspmm_pipeline_temp_bytes(C.byref(out)))
    return int(out.value)


def pipeline_last_packed() -> bool:
    """Whether the last spmm_pipeline call on this thread multiplied packed
    column batches (C ABI xspmm_pipeline_last_form)."""
    out = C.c_int(0)
    _check(load().xspmm_pipeline_last_form(C.byref(out)))
    return bool(out.value)


class SpMMPlan:
    """Prepared Tier-2 product (C ABI xspmm_plan_*): the pipeline's clustering,
    permutation and CSR->BCSR stages run once here; execute() multiplies with
    the Tier-1 SpMM alone (un-permutation fused into the fp16 kernel's store)
    and returns the same C as spmm_pipeline(A, B, ...).  `timings` holds the
    preparation stage times.  No counterpart in the reference."""

    def __init__(self, A: CSRMatrix, hw_block_size: int = 16, optimize_pattern: bool = True):
        L = load()
        self._L = L
        self._h = None
        self.num_rows, self.num_cols = A.num_rows, A.num_cols
        self.value_dtype = A.values.dtype
        self.device = A.row_ptr.device
        t = (C.c_double * 6)()
        h = C.c_void_p()
        _check(L.xspmm_plan_create(vcode(A.values.dtype), icode(A.row_ptr.dtype), A.num_rows,
                                   A.num_cols, A.nnz, _ptr(A.row_ptr), _ptr(A.col_ind),
                                   _ptr(A.values), hw_block_size, 1 if optimize_pattern else 0,
                                   C.cast(t, C.POINTER(C.c_double)), _stream(), C.byref(h)))
        self._h = h
        self.timings = {k: v for k, v in zip(TIMING_FIELDS, list(t))
                        if k in ("clustering_ms", "permutation_ms", "conversion_ms",
                                 "total_pipeline_ms")}
        nb, nbr, cl = C.c_int64(), C.c_int64(), C.c_int()
        _check(L.xspmm_plan_info(h, C.byref(nb), C.byref(nbr), C.byref(cl), None))
        self.num_blocks, self.num_block_rows, self.clustered = nb.value, nbr.value, bool(cl.value)
        pb = C.c_int64()
        _check(L.xspmm_plan_packed_batches(h, C.byref(pb)))
        self.packed_batches = pb.value  # -1: multiplies the BCSR matrix itself

    def execute(self, B, C_out=None, N: int | None = None):
        torch = _torch()
        if self._h is None:
            raise RuntimeError("SpMMPlan is closed")
        if N is None:
            N = int(B.shape[1])
        if C_out is None:
            C_out = torch.empty((self.num_rows, N), dtype=torch.float32, device=self.device)
        _check_dense(B, "B", self.num_cols, N, self.value_dtype, self.device)
        _check_dense(C_out, "C_out", self.num_rows, N, torch.float32, self.device)
        _check(self._L.xspmm_plan_execute(self._h, _ptr(B), _ptr(C_out), N, _stream()))
        return C_out

    def close(self):
        if self._h is not None:
            self._L.xspmm_plan_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

