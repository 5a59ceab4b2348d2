"""CPU: the MatrixMarket reader (xspmm_mtx_* / matrix_utils::io::read_mtx).

Pinned like the rest of the path:
  * golden vectors written by the reference's own reader
    (utils/matrix_io.hpp:27-98, compiled into oracle/_ref) from the fixture
    files under tests/golden/mtx/: comments, pattern/integer/complex/symmetric
    headers, CRLF, unreadable lines, out-of-range entries, overflowing and
    partial numbers, duplicates, files without entries or dimensions;
  * the oracle's restatement (oracle.read_mtx) against the same vectors;
  * the product against the oracle on seeded random files with mixed
    white space, line endings, number spellings and junk lines.
"""
from __future__ import annotations

import os
import subprocess

import numpy as np
import pytest

import oracle
import xspmm_amd as X
from tests.helpers import GOLDEN, golden_cases

MTX = golden_cases("mtx")
ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))


def same(a, b):
    M, K, rp, ci, vals = a
    M2, K2, rp2, ci2, vals2 = b
    assert (M, K) == (M2, K2)
    np.testing.assert_array_equal(np.asarray(rp, np.int64), np.asarray(rp2, np.int64))
    np.testing.assert_array_equal(np.asarray(ci, np.int64), np.asarray(ci2, np.int64))
    np.testing.assert_array_equal(np.asarray(vals, np.float32).view(np.uint32),
                                  np.asarray(vals2, np.float32).view(np.uint32))


@pytest.mark.parametrize("case", MTX, ids=[c["name"] for c in MTX])
def test_oracle_reader_matches_reference_golden(case):
    path = os.path.join(GOLDEN, str(case["source"]))
    if str(case["error"]):
        with pytest.raises(RuntimeError, match=str(case["error"])):
            oracle.read_mtx(path)
        return
    same(oracle.read_mtx(path), (int(case["M"]), int(case["K"]), case["rp"], case["ci"],
                                 case["vals"]))


@pytest.mark.parametrize("case", MTX, ids=[c["name"] for c in MTX])
def test_product_reader_matches_reference_golden(case):
    path = os.path.join(GOLDEN, str(case["source"]))
    if str(case["error"]):
        with pytest.raises(X.XspmmError) as e:
            X.read_mtx(path)
        assert e.value.code == X.ERR_IO and str(case["error"]) in str(e.value)
        return
    got = X.read_mtx(path)
    same(got, (int(case["M"]), int(case["K"]), case["rp"], case["ci"], case["vals"]))
    # other export types: int64 indices, fp16 values rounded to nearest even
    M, K, rp, ci, vals = X.read_mtx(path, np.int64, np.float16)
    assert rp.dtype == np.int64 and vals.dtype == np.float16
    np.testing.assert_array_equal(rp, case["rp"])
    with np.errstate(over="ignore"):  # 1e38 rounds to fp16 infinity on both sides
        np.testing.assert_array_equal(vals, case["vals"].astype(np.float16))


def test_missing_file_message():
    with pytest.raises(X.XspmmError) as e:
        X.read_mtx("/nonexistent/dir/m.mtx")
    assert e.value.code == X.ERR_IO
    assert "Could not open MTX file: /nonexistent/dir/m.mtx" in str(e.value)


def _random_mtx(rng, path):
    rows, cols = int(rng.integers(1, 60)), int(rng.integers(1, 60))
    eol = [b"\n", b"\r\n"][int(rng.integers(0, 2))]
    ws = [b" ", b"\t", b"  ", b" \t "]
    nums = ["{:d}", "{:.3f}", "{:.2e}", "{:+.1f}", "-{:.0f}.", "{:.1E}", "{:d}e", "{:d}x",
            ".{:d}", "{:d}e-50", "{:d}e50", "nan", "inf", "", "-", "+"]
    out = [b"%%MatrixMarket matrix coordinate real general", b"% c"]
    out.append(str(rows).encode() + ws[0] + str(cols).encode() + ws[0] + b"0")
    for _ in range(int(rng.integers(0, 120))):
        kind = int(rng.integers(0, 12))
        if kind == 0:
            out.append(b"")
        elif kind == 1:
            out.append(b"% " + bytes(rng.integers(97, 122, size=5).tolist()))
        elif kind == 2:
            out.append(b"junk " + str(int(rng.integers(0, 9))).encode())
        else:
            r = int(rng.integers(-1, rows + 3))
            c = int(rng.integers(-1, cols + 3))
            f = nums[int(rng.integers(0, len(nums)))]
            v = f.format(int(rng.integers(0, 100))) if "{" in f and "d" in f else (
                f.format(float(rng.uniform(-50, 50))) if "{" in f else f)
            w = ws[int(rng.integers(0, len(ws)))]
            line = w * int(rng.integers(0, 2)) + str(r).encode() + w + str(c).encode()
            if v:
                line += w + v.encode()
            out.append(line)
    data = eol.join(out) + (eol if rng.integers(0, 2) else b"")
    with open(path, "wb") as f:
        f.write(data)


@pytest.mark.parametrize("seed", range(40))
def test_product_reader_matches_oracle_on_random_files(seed, tmp_path):
    rng = np.random.default_rng(seed)
    path = tmp_path / f"r{seed}.mtx"
    _random_mtx(rng, path)
    same(X.read_mtx(path), oracle.read_mtx(str(path)))


def test_cpp_interface_reads_the_same_matrix():
    prog = os.path.join(ROOT, "xspmm_amd", "bin", "mtx_read")
    if not os.path.exists(prog):
        pytest.fail(f"{prog} is not built (make -C xspmm_amd/csrc examples)")
    for case in MTX:
        path = os.path.join(GOLDEN, str(case["source"]))
        out = subprocess.run([prog, path], capture_output=True, text=True, timeout=60)
        if str(case["error"]):
            assert out.returncode == 1 and str(case["error"]) in out.stdout
            continue
        assert out.returncode == 0, out.stdout + out.stderr
        M, K, nnz, rsum, csum, vsum = out.stdout.split()
        assert (int(M), int(K), int(nnz)) == (int(case["M"]), int(case["K"]), len(case["ci"]))
        assert int(rsum) == int(np.asarray(case["rp"], np.int64).sum())
        assert int(csum) == int(np.asarray(case["ci"], np.int64).sum())
        assert float(vsum) == pytest.approx(float(np.asarray(case["vals"], np.float64).sum()),
                                            rel=1e-12, abs=1e-12)
