"""Writes the golden vectors under tests/golden/ from the reference's own code.

Runs in the build container only (it needs /root/reference to have been
compiled into oracle/_ref/libxspmm_ref.so by `make -C oracle`).  The reference
functions called are its CPU implementations, exactly as shipped:
  csr_to_bcsr                    src/core/conversion.cpp:8-100
  compute_1d_jaccard_clustering  src/cpu/clustering_sylos_labini.cpp:51-120
  apply_permutation (CPU)        src/cpu/clustering_sylos_labini.cpp:125-178
The reference instantiates float values only; values are stored as float32.

Each case is saved as one .npz (inputs and outputs, no pickles).  Regenerate
with:  python tests/golden/make_golden.py
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.abspath(os.path.join(HERE, "..", "..")))

import oracle  # noqa: E402


def random_csr(rng, M, K, density, unsorted=False, dup=0.0, empty_rows=0.0, zeros=0.0):
    rows = []
    for _ in range(M):
        if rng.random() < empty_rows or K == 0:
            rows.append(np.zeros(0, np.int64))
            continue
        k = min(K, rng.binomial(K, density))
        r = rng.choice(K, size=k, replace=False) if k else np.zeros(0, np.int64)
        if dup > 0 and k:
            r = np.concatenate([r, rng.choice(r, size=max(1, int(dup * k)))])
        r = rng.permutation(r) if unsorted else np.sort(r)
        rows.append(r)
    lens = np.array([len(r) for r in rows], np.int64)
    rp = np.zeros(M + 1, np.int64)
    np.cumsum(lens, out=rp[1:])
    ci = np.concatenate(rows).astype(np.int64) if M else np.zeros(0, np.int64)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(np.float32)
    if zeros > 0 and len(vals):
        vals[rng.random(len(vals)) < zeros] = 0.0
    return rp, ci, vals


CONVERSION_CASES = [
    # name, M, K, density, rb, cb, flags
    ("conv_basic", 64, 64, 0.08, 16, 16, {}),
    ("conv_ragged", 77, 53, 0.10, 16, 16, {}),
    ("conv_unsorted_dups", 48, 70, 0.12, 16, 16, dict(unsorted=True, dup=0.3)),
    ("conv_empty_rows_zeros", 40, 40, 0.15, 16, 16, dict(empty_rows=0.4, zeros=0.3)),
    ("conv_block_4x4", 30, 37, 0.10, 4, 4, dict(unsorted=True, dup=0.2)),
    ("conv_block_3x5", 23, 29, 0.15, 3, 5, {}),
    ("conv_block_16x8", 50, 50, 0.05, 16, 8, dict(dup=0.1)),
    ("conv_wide", 33, 1500, 0.01, 16, 16, dict(unsorted=True)),
    ("conv_empty", 0, 10, 0.0, 16, 16, {}),
    ("conv_no_entries", 20, 20, 0.0, 16, 16, {}),
]

JACCARD_CASES = [
    # name, M, K, density, thresh, block_width, flags
    ("jac_basic", 200, 256, 0.02, 0.5, 16, {}),
    ("jac_ties", 300, 64, 0.03, 0.5, 16, dict(empty_rows=0.1)),
    ("jac_ties_bw4", 250, 32, 0.05, 0.5, 4, {}),
    ("jac_thresh_03", 220, 128, 0.04, 0.3, 16, {}),
    ("jac_thresh_0", 150, 64, 0.05, 0.0, 16, dict(empty_rows=0.2)),
    ("jac_thresh_1", 90, 96, 0.05, 1.0, 16, {}),
    ("jac_thresh_075", 200, 200, 0.03, 0.75, 8, dict(unsorted=True)),
    ("jac_thresh_neg", 60, 64, 0.05, -0.1, 16, {}),
    ("jac_bw1", 120, 40, 0.08, 0.5, 1, {}),
    ("jac_wide_words", 160, 4200, 0.003, 0.5, 16, {}),
    ("jac_dense", 64, 64, 0.6, 0.5, 16, {}),
]

PERM_CASES = [
    ("perm_basic", 100, 80, 0.05, {}),
    ("perm_empty_rows", 64, 64, 0.1, dict(empty_rows=0.5)),
    ("perm_single", 1, 10, 0.5, {}),
]


# MatrixMarket inputs (text, written under mtx/): the reader's edge cases.
def _mtx_cases(rng):
    big = ["%%MatrixMarket matrix coordinate real general", "% random, unsorted, no duplicates",
           "1000 800 5000"]
    cells = rng.choice(1000 * 800, size=5000, replace=False)
    for x in cells:
        big.append(f"{x // 800 + 1} {x % 800 + 1} {rng.uniform(-2, 2):.6g}")
    return {
        "basic": "%%MatrixMarket matrix coordinate real general\n% comment\n"
                 "4 5 6\n3 2 1.5\n1 1 -2\n4 5 7e-1\n1 5 3\n2 3 0.25\n3 1 8\n",
        "pattern": "%%MatrixMarket matrix coordinate pattern general\n3 3 4\n1 2\n3 3\n2 1\n1 1\n",
        "symmetric": "%%MatrixMarket matrix coordinate real symmetric\n4 4 5\n1 1 2\n2 1 -1\n"
                     "3 2 -1\n4 3 -1\n4 4 2\n",
        "integer_complex": "%%MatrixMarket matrix coordinate integer general\n3 4 4\n1 4 7\n"
                           "2 2 -3\n3 1 1 9\n3 3 2.5 -1.5\n",
        # CRLF, blank lines, indented comments, bad tokens, out-of-range
        # entries, awkward numbers (overflow -> the reader's 1.0 default,
        # underflow, partial exponents, signs, trailing text, inf/nan)
        "messy": "%%MatrixMarket matrix coordinate real general\r\n%c\r\n 6 7 99\r\n\r\n"
                 "1 1 1e50\r\n1 2 1e-50\r\n1 3 1e\r\n1 4 -.5\r\n1 5 +3\r\n1 6 .\r\n"
                 "1 7 -\r\n2 1 2.5x\r\n2 2 0x1p3\r\n2 3 inf\r\n2 4 nan\r\n2 5\t\t4.75\r\n"
                 "  % not a comment\r\nabc def\r\n1.5 2 3\r\n0 1 5\r\n7 1 5\r\n3 0 5\r\n"
                 "3 8 5\r\n-1 2 5\r\n99999999999 1 5\r\n3 3 1e38\r\n3 4 3.4028236e38\r\n"
                 "4 4 1.17549435e-38\r\n4 5 1e-45\r\n5 5 0.1\r\n5 6 1E+2\r\n6 7 1e+\r\n\r\n",
        # a CRLF blank line is "\r", not empty: read as the dimension line
        "crlf_blank_before_dims": "%%MatrixMarket matrix coordinate real general\r\n\r\n2 2 1\r\n1 1 1\r\n",
        "duplicates": "%%MatrixMarket matrix coordinate real general\n3 3 6\n2 2 1\n1 3 4\n"
                      "2 2 5\n1 3 6\n3 1 7\n2 2 9\n",
        "no_entries": "%%MatrixMarket matrix coordinate real general\n5 3 0\n",
        "only_comments": "%%MatrixMarket matrix coordinate real general\n% nothing else\n",
        "bad_dims": "%%MatrixMarket matrix coordinate real general\nrows cols nnz\n1 1 1\n",
        "no_final_newline": "%%MatrixMarket matrix coordinate real general\n2 2 2\n2 2 4\n1 1 3",
        "random_1000x800": "\n".join(big) + "\n",
    }


def write_mtx_cases(rng):
    d = os.path.join(HERE, "mtx")
    os.makedirs(d, exist_ok=True)
    n = 0
    for name, text in _mtx_cases(rng).items():
        path = os.path.join(d, name + ".mtx")
        with open(path, "wb") as f:
            f.write(text.encode())
        try:
            M, K, rp, ci, vals = oracle.ref_read_mtx(path)
            np.savez_compressed(os.path.join(HERE, f"mtx_{name}.npz"), kind="mtx",
                                source=f"mtx/{name}.mtx", M=M, K=K, rp=rp, ci=ci, vals=vals,
                                error="")
        except RuntimeError as e:
            np.savez_compressed(os.path.join(HERE, f"mtx_{name}.npz"), kind="mtx",
                                source=f"mtx/{name}.mtx", error=str(e))
        n += 1
    return n


def main():
    if "--only" in sys.argv and sys.argv[sys.argv.index("--only") + 1] == "mtx":
        if not oracle.ref_available():
            oracle.build()
        print(f"wrote {write_mtx_cases(np.random.default_rng(77))} MatrixMarket cases")
        return
    if not oracle.ref_available():
        oracle.build()
    if not oracle.ref_available():
        raise SystemExit("oracle/_ref/libxspmm_ref.so is missing (needs /root/reference)")
    rng = np.random.default_rng(20241201)
    n = 0
    for name, M, K, dens, rb, cb, flags in CONVERSION_CASES:
        rp, ci, vals = random_csr(rng, M, K, dens, **flags)
        for it in (np.int32, np.int64):
            brp, bci, bv = oracle.ref_csr_to_bcsr(M, K, rp, ci, vals, rb, cb, index_dtype=it)
            tag = "i32" if it == np.int32 else "i64"
            np.savez_compressed(os.path.join(HERE, f"{name}_{tag}.npz"), kind="conversion",
                                M=M, K=K, rb=rb, cb=cb, rp=rp.astype(it), ci=ci.astype(it),
                                vals=vals, brp=brp, bci=bci, bvals=bv)
            n += 1
    for name, M, K, dens, thr, bw, flags in JACCARD_CASES:
        rp, ci, _ = random_csr(rng, M, K, dens, **flags)
        for it in (np.int32, np.int64):
            perm = oracle.ref_jaccard(M, K, rp, ci, thr, bw, index_dtype=it)
            tag = "i32" if it == np.int32 else "i64"
            np.savez_compressed(os.path.join(HERE, f"{name}_{tag}.npz"), kind="jaccard",
                                M=M, K=K, thresh=np.float32(thr), bw=bw, rp=rp.astype(it),
                                ci=ci.astype(it), perm=perm)
            n += 1
    for name, M, K, dens, flags in PERM_CASES:
        rp, ci, vals = random_csr(rng, M, K, dens, **flags)
        perm = rng.permutation(M)
        for it in (np.int32, np.int64):
            nrp, nci, nv = oracle.ref_apply_perm(M, K, rp, ci, vals, perm, index_dtype=it)
            tag = "i32" if it == np.int32 else "i64"
            np.savez_compressed(os.path.join(HERE, f"{name}_{tag}.npz"), kind="permutation",
                                M=M, K=K, rp=rp.astype(it), ci=ci.astype(it), vals=vals,
                                perm=perm.astype(it), nrp=nrp, nci=nci, nvals=nv)
            n += 1
    n += write_mtx_cases(np.random.default_rng(77))
    print(f"wrote {n} golden cases to {HERE}")


if __name__ == "__main__":
    main()
