"""Shared test helpers: golden-case loading and small independent references."""
from __future__ import annotations

import glob
import os

import numpy as np

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden_cases(kind: str):
    out = []
    for path in sorted(glob.glob(os.path.join(GOLDEN, "*.npz"))):
        with np.load(path, allow_pickle=False) as z:
            if str(z["kind"]) != kind:
                continue
            d = {k: z[k] for k in z.files}
        d["name"] = os.path.basename(path)[:-4]
        out.append(d)
    return out


def dense_last_wins(M, K, rp, ci, vals, dtype=np.float64):
    """Dense matrix of a CSR; for duplicate (row, col) the later entry wins,
    the rule of the reference conversion (src/core/conversion.cpp:75-91)."""
    D = np.zeros((M, K), dtype)
    for r in range(M):
        for j in range(int(rp[r]), int(rp[r + 1])):
            D[r, int(ci[j])] = vals[j]
    return D


def dense_from_bcsr(M, K, rb, cb, brp, bci, bvals, dtype=np.float64):
    Mb = len(brp) - 1
    D = np.zeros((Mb * rb, max(1, (K + cb - 1) // cb) * cb), dtype)
    bv = np.asarray(bvals).reshape(-1, rb, cb) if len(bci) else np.zeros((0, rb, cb))
    for br in range(Mb):
        for b in range(int(brp[br]), int(brp[br + 1])):
            c = int(bci[b])
            D[br * rb:(br + 1) * rb, c * cb:(c + 1) * cb] = bv[b]
    return D[:M, :K]


def widen(a):
    return np.asarray(a).astype(np.int64)
