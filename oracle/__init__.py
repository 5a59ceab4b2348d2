"""ctypes view of the CPU oracle (oracle.c) and of the compiled reference.

TEST INFRASTRUCTURE ONLY.  Only tests/, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker (or as the timed CPU baseline).  The product package ``xspmm_amd``
never imports it.

All functions take and return numpy arrays.  Index arrays may be int32 or
int64; they are widened to int64 before crossing into C.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libxspmm_ref.so")

_lib = None
_ref = None

_p = C.c_void_p
_i64 = C.c_int64


def build(quiet: bool = True) -> None:
    """Compile liboracle.so (and oracle/_ref when the reference is present)."""
    out = subprocess.run(["make", "-C", HERE, "all"], capture_output=True, text=True)
    if out.returncode != 0:
        raise RuntimeError("oracle build failed:\n" + out.stdout + out.stderr)
    if not quiet:
        print(out.stdout)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = C.CDLL(LIB_PATH)
        L.xo_bcsr_count.restype = _i64
        L.xo_bcsr_count.argtypes = [_i64, _i64, _i64, _i64, _p, _p, _p]
        L.xo_bcsr_fill.restype = None
        L.xo_bcsr_fill.argtypes = [_i64, _i64, _i64, _i64, _p, _p, _p, C.c_int, _p, _p, _p]
        L.xo_jaccard.restype = None
        L.xo_jaccard.argtypes = [_i64, _i64, _p, _p, C.c_float, _i64, _p]
        L.xo_apply_perm.restype = None
        L.xo_apply_perm.argtypes = [_i64, _p, _p, _p, C.c_int, _p, _p, _p, _p]
        L.xo_unpermute.restype = None
        L.xo_unpermute.argtypes = [_i64, _i64, _p, _p, _p]
        L.xo_bcsr_spmm_f64.restype = None
        L.xo_bcsr_spmm_f64.argtypes = [_i64, _i64, _i64, _i64, _p, _p, _p, _p, _p]
        L.xo_bcsr_spmm_f32.restype = None
        L.xo_bcsr_spmm_f32.argtypes = [_i64, _i64, _i64, _i64, _p, _p, _p, _p, C.c_int, _p, C.c_int]
        L.xo_csr_spmm_f64.restype = None
        L.xo_csr_spmm_f64.argtypes = [_i64, _i64, _p, _p, _p, _p, _p]
        L.xo_errors.restype = None
        L.xo_errors.argtypes = [_i64, _p, _p, _p]
        L.xo_max_threads.restype = C.c_int
        L.xo_max_threads.argtypes = []
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref():
    """The reference's own CPU code (oracle/_ref), or None when not built."""
    global _ref
    if _ref is None and ref_available():
        R = C.CDLL(REF_PATH)
        for it, ct in (("i32", C.c_int32), ("i64", C.c_int64)):
            f = getattr(R, "ref_csr_to_bcsr_" + it)
            f.restype = _i64
            f.argtypes = [ct, ct, ct, _p, _p, _p, ct, ct, _p, _p, _p, _i64]
            f = getattr(R, "ref_jaccard_" + it)
            f.restype = None
            f.argtypes = [ct, ct, ct, _p, _p, C.c_float, ct, _p]
            f = getattr(R, "ref_apply_perm_" + it)
            f.restype = None
            f.argtypes = [ct, ct, ct, _p, _p, _p, _p, _p, _p, _p]
        _ref = R
    return _ref


def _ptr(a: np.ndarray):
    return a.ctypes.data_as(_p)


def _i64a(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a), dtype=np.int64)


# ---------------------------------------------------------------------------
# restatement
# ---------------------------------------------------------------------------

def csr_to_bcsr(M, K, rp, ci, vals, rb=16, cb=16):
    """-> (bcsr_row_ptr int64[Mb+1], bcsr_col_ind int64[nnzb], values[nnzb*rb*cb])."""
    rp, ci = _i64a(rp), _i64a(ci)
    vals = np.ascontiguousarray(vals)
    Mb = (M + rb - 1) // rb
    brp = np.zeros(Mb + 1, np.int64)
    nnzb = lib().xo_bcsr_count(M, K, rb, cb, _ptr(rp), _ptr(ci), _ptr(brp))
    if nnzb < 0:
        raise ValueError("column index out of range" if nnzb == -1 else "bad block size")
    bci = np.zeros(max(nnzb, 1), np.int64)
    bv = np.zeros(max(nnzb * rb * cb, 1), vals.dtype)
    lib().xo_bcsr_fill(M, K, rb, cb, _ptr(rp), _ptr(ci), _ptr(vals), vals.itemsize,
                       _ptr(brp), _ptr(bci), _ptr(bv))
    return brp, bci[:nnzb], bv[: nnzb * rb * cb]


def jaccard(M, K, rp, ci, dist_thresh=0.5, block_width=16):
    rp, ci = _i64a(rp), _i64a(ci)
    perm = np.zeros(max(M, 1), np.int64)
    lib().xo_jaccard(M, K, _ptr(rp), _ptr(ci), C.c_float(dist_thresh), block_width, _ptr(perm))
    return perm[:M]


def apply_perm(M, rp, ci, vals, perm):
    rp, ci, perm = _i64a(rp), _i64a(ci), _i64a(perm)
    vals = np.ascontiguousarray(vals)
    nnz = int(rp[M])
    nrp = np.zeros(M + 1, np.int64)
    nci = np.zeros(max(nnz, 1), np.int64)
    nv = np.zeros(max(nnz, 1), vals.dtype)
    lib().xo_apply_perm(M, _ptr(rp), _ptr(ci), _ptr(vals), vals.itemsize, _ptr(perm),
                        _ptr(nrp), _ptr(nci), _ptr(nv))
    return nrp, nci[:nnz], nv[:nnz]


def unpermute(M, N, x, perm):
    x = np.ascontiguousarray(x, np.float32)
    perm = _i64a(perm)
    out = np.zeros((M, N), np.float32)
    lib().xo_unpermute(M, N, _ptr(x), _ptr(out), _ptr(perm))
    return out


def bcsr_spmm_f64(M, K, N, brp, bci, bvals, B):
    """fp64 truth of the tile-kernel product; bvals/B any float dtype."""
    brp, bci = _i64a(brp), _i64a(bci)
    bv = np.ascontiguousarray(bvals, np.float32)
    Bf = np.ascontiguousarray(B, np.float32)
    Mb = len(brp) - 1
    out = np.zeros((M, N), np.float64)
    lib().xo_bcsr_spmm_f64(M, K, N, Mb, _ptr(brp), _ptr(bci), _ptr(bv), _ptr(Bf), _ptr(out))
    return out


def bcsr_spmm_f32(M, K, N, brp, bci, bvals, B, nthreads=1):
    """fp32-accumulated tile product (also the CPU baseline kernel)."""
    brp, bci = _i64a(brp), _i64a(bci)
    bv = np.ascontiguousarray(bvals)
    Bc = np.ascontiguousarray(B)
    assert bv.dtype == Bc.dtype and bv.dtype in (np.float16, np.float32)
    Mb = len(brp) - 1
    out = np.zeros((M, N), np.float32)
    lib().xo_bcsr_spmm_f32(M, K, N, Mb, _ptr(brp), _ptr(bci), _ptr(bv), _ptr(Bc),
                           bv.itemsize, _ptr(out), nthreads)
    return out


def csr_spmm_f64(M, N, rp, ci, vals, B):
    rp, ci = _i64a(rp), _i64a(ci)
    v = np.ascontiguousarray(vals, np.float32)
    Bf = np.ascontiguousarray(B, np.float32)
    out = np.zeros((M, N), np.float64)
    lib().xo_csr_spmm_f64(M, N, _ptr(rp), _ptr(ci), _ptr(v), _ptr(Bf), _ptr(out))
    return out


def errors(actual, expected):
    """{max_abs, max_rel, frob, rel_frob} as in utils/matrix_compare.hpp:23-65."""
    a = np.ascontiguousarray(actual, np.float32).ravel()
    e = np.ascontiguousarray(expected, np.float64).ravel()
    assert a.size == e.size
    out = np.zeros(4, np.float64)
    lib().xo_errors(a.size, _ptr(a), _ptr(e), _ptr(out))
    return dict(max_abs=out[0], max_rel=out[1], frob=out[2], rel_frob=out[3])


def max_threads() -> int:
    return int(lib().xo_max_threads())


# ---------------------------------------------------------------------------
# compiled reference (oracle/_ref), float values only
# ---------------------------------------------------------------------------

def _it(index_dtype):
    return ("i32", np.int32) if np.dtype(index_dtype) == np.int32 else ("i64", np.int64)


def ref_csr_to_bcsr(M, K, rp, ci, vals, rb=16, cb=16, index_dtype=np.int64):
    R = ref()
    name, dt = _it(index_dtype)
    rp = np.ascontiguousarray(rp, dt)
    ci = np.ascontiguousarray(ci, dt) if len(ci) else np.zeros(1, dt)
    v = np.ascontiguousarray(vals, np.float32) if len(vals) else np.zeros(1, np.float32)
    nnz = int(rp[M])
    f = getattr(R, "ref_csr_to_bcsr_" + name)
    Mb = (M + rb - 1) // rb
    brp = np.zeros(Mb + 1, dt)
    nnzb = f(M, K, nnz, _ptr(rp), _ptr(ci), _ptr(v), rb, cb, _ptr(brp), None, None, 0)
    bci = np.zeros(max(nnzb, 1), dt)
    bv = np.zeros(max(nnzb * rb * cb, 1), np.float32)
    f(M, K, nnz, _ptr(rp), _ptr(ci), _ptr(v), rb, cb, _ptr(brp), _ptr(bci), _ptr(bv), nnzb)
    return brp, bci[:nnzb], bv[: nnzb * rb * cb]


def ref_jaccard(M, K, rp, ci, dist_thresh=0.5, block_width=16, index_dtype=np.int64):
    R = ref()
    name, dt = _it(index_dtype)
    rp = np.ascontiguousarray(rp, dt)
    ci = np.ascontiguousarray(ci, dt) if len(ci) else np.zeros(1, dt)
    perm = np.full(max(M, 1), -1, dt)
    getattr(R, "ref_jaccard_" + name)(M, K, int(rp[M]), _ptr(rp), _ptr(ci),
                                      C.c_float(dist_thresh), block_width, _ptr(perm))
    return perm[:M]


def ref_apply_perm(M, K, rp, ci, vals, perm, index_dtype=np.int64):
    R = ref()
    name, dt = _it(index_dtype)
    rp = np.ascontiguousarray(rp, dt)
    nnz = int(rp[M])
    ci = np.ascontiguousarray(ci, dt) if nnz else np.zeros(1, dt)
    v = np.ascontiguousarray(vals, np.float32) if nnz else np.zeros(1, np.float32)
    perm = np.ascontiguousarray(perm, dt)
    nrp = np.zeros(M + 1, dt)
    nci = np.zeros(max(nnz, 1), dt)
    nv = np.zeros(max(nnz, 1), np.float32)
    getattr(R, "ref_apply_perm_" + name)(M, K, nnz, _ptr(rp), _ptr(ci), _ptr(v), _ptr(perm),
                                         _ptr(nrp), _ptr(nci), _ptr(nv))
    return nrp, nci[:nnz], nv[:nnz]


# ---------------------------------------------------------------------------
# MatrixMarket reader: restatement of the reference's utils/matrix_io.hpp:27-98
# (matrix_utils::io::read_mtx<float>), plain Python.  The reference extracts
# tokens with std::istringstream; the helpers below restate libstdc++'s
# extraction rules for int and float (skip whitespace, the numeric grammar,
# strtof on the accepted characters, failure on overflow) and use libc's
# strtof for the rounding, as libstdc++ does.
# ---------------------------------------------------------------------------

_WS = b" \t\n\v\f\r"
_libc = None


def _strtof(tok: bytes):
    """libc strtof on tok; None unless the whole token converts to a finite float."""
    global _libc
    if _libc is None:
        _libc = C.CDLL(None)
        _libc.strtof.restype = C.c_float
        _libc.strtof.argtypes = [C.c_char_p, C.POINTER(C.c_char_p)]
    buf = C.create_string_buffer(tok)
    end = C.c_char_p()
    v = _libc.strtof(buf, C.byref(end))
    consumed = C.cast(end, C.c_void_p).value - C.cast(buf, C.c_void_p).value
    if len(tok) == 0 or consumed != len(tok) or v in (float("inf"), float("-inf")):
        return None
    return np.float32(v)


def _skip_ws(s: bytes, i: int) -> int:
    while i < len(s) and s[i] in _WS:
        i += 1
    return i


def _extract_int(s: bytes, i: int):
    """`iss >> int`: optional sign, decimal digits, must fit int32."""
    i = _skip_ws(s, i)
    j = i
    if j < len(s) and s[j] in b"+-":
        j += 1
    k = j
    while k < len(s) and 48 <= s[k] <= 57:
        k += 1
    if k == j:
        return None, k
    v = int(s[i:k])
    if not (-2**31 <= v < 2**31):
        return None, k
    return v, k


def _extract_float(s: bytes, i: int):
    """`iss >> float`: sign, digits, one '.', an exponent after a digit."""
    i = _skip_ws(s, i)
    j = i
    if j < len(s) and s[j] in b"+-":
        j += 1
    mant = dot = sci = False
    while j < len(s):
        c = s[j]
        if 48 <= c <= 57:
            mant = True
        elif c == 46 and not dot and not sci:
            dot = True
        elif c in b"eE" and not sci and mant:
            sci = True
            if j + 1 < len(s) and s[j + 1] in b"+-":
                j += 1
        else:
            break
        j += 1
    return _strtof(s[i:j]), j


def read_mtx(path):
    """(M, K, rp int32, ci int32, vals float32) as the reference reads `path`:
    lines that are empty or start with '%' are skipped; the first other line
    gives rows, cols, nnz; each entry line gives 1-based row and column and a
    value (1.0 when absent or unreadable); entries outside the matrix and
    unreadable lines are dropped; entries are sorted by (row, column), equal
    keys in file order (the reference's std::sort leaves them in file order for
    the small duplicate cases tested); duplicates are kept."""
    data = open(path, "rb").read()
    lines = data.split(b"\n")
    if lines and lines[-1] == b"":
        lines.pop()
    rows = cols = 0
    k = 0
    while k < len(lines):
        line = lines[k]
        k += 1
        if not line or line[:1] == b"%":
            continue
        r, i = _extract_int(line, 0)
        c, i = _extract_int(line, i) if r is not None else (None, i)
        n, i = _extract_int(line, i) if c is not None else (None, i)
        if n is None:
            raise RuntimeError("Failed to parse MTX dimensions.")
        rows, cols = r, c
        break
    el = []
    for line in lines[k:]:
        if not line or line[:1] == b"%":
            continue
        r, i = _extract_int(line, 0)
        if r is None:
            continue
        c, i = _extract_int(line, i)
        if c is None:
            continue
        v, _ = _extract_float(line, i)
        if v is None:
            v = np.float32(1.0)
        if r < 1 or r > rows or c < 1 or c > cols:
            continue
        el.append((r - 1, c - 1, v))
    el.sort(key=lambda e: (e[0], e[1]))
    rp = np.zeros(max(rows, 0) + 1, np.int32)
    for e in el:
        rp[e[0] + 1] += 1
    rp = np.cumsum(rp).astype(np.int32)
    ci = np.array([e[1] for e in el], np.int32)
    vals = np.array([e[2] for e in el], np.float32)
    return rows, cols, rp, ci, vals


def ref_read_mtx(path):
    """The reference's own reader (oracle/_ref): (M, K, rp, ci, vals), or
    raises RuntimeError with its message."""
    R = ref()
    R.ref_read_mtx.restype = C.c_int64
    M, K = C.c_int32(), C.c_int32()
    err = C.create_string_buffer(256)
    p = os.fsencode(path)
    nnz = R.ref_read_mtx(p, C.byref(M), C.byref(K), None, None, None, C.c_int64(-1), err, 256)
    if nnz < 0:
        raise RuntimeError(err.value.decode())
    rp = np.zeros(max(M.value, 0) + 1, np.int32)
    ci = np.zeros(max(nnz, 1), np.int32)
    vals = np.zeros(max(nnz, 1), np.float32)
    R.ref_read_mtx(p, C.byref(M), C.byref(K), _ptr(rp), _ptr(ci), _ptr(vals), C.c_int64(nnz),
                   err, 256)
    return M.value, K.value, rp, ci[:nnz], vals[:nnz]

