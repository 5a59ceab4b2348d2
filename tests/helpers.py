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


def nested_csr(rng, M, K, n_base=5, grow=0.1):
    """CSR rows that are random subsets of a few base patterns (a join leaves
    the clustering pattern as it is), a fraction `grow` of them with one or
    two columns of their own (a join grows it)."""
    base = [rng.choice(K, size=int(rng.integers(20, 60)), replace=False) for _ in range(n_base)]
    rows = []
    for _ in range(M):
        b = base[int(rng.integers(0, n_base))]
        r = b[rng.random(len(b)) < rng.uniform(0.6, 1.0)]
        if rng.random() < grow:
            r = np.concatenate([r, rng.integers(0, K, size=int(rng.integers(1, 3)))])
        rows.append(r)
    rp = np.zeros(M + 1, np.int64)
    rp[1:] = np.cumsum([len(x) for x in rows])
    return rp, np.concatenate(rows).astype(np.int64)
