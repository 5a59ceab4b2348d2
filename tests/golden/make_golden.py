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


def main():
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
    print(f"wrote {n} golden cases to {HERE}")


if __name__ == "__main__":
    main()
