"""Seeded synthetic inputs for the benchmark configurations and tests.

Every generator is deterministic for a given seed (numpy ``default_rng``,
PCG64) and returns a :class:`Problem`: a host CSR matrix (columns sorted
within each row, int32 indices), a dense row-major ``B`` and the SpMM
width ``N``.  The algorithms are written out in each docstring so the inputs
can be regenerated without this file.

Shapes follow the benchmark configurations:

* ``cpu_ref``     1024^2 fp32, 1 % uniform, N=64                (config 0)
* ``blocks``      8192^2 fp16, 5 % of 16x16 blocks dense, N=256 (config 1)
* ``templates``   16384^2 fp16, 0.5 %, 1024 x 82-col templates, N=128
                  (config 2, clustered; the headline workload)
* ``gnn``         131072^2 fp16 power-law adjacency, N=64        (config 3)
* ``pruned``      14336x4096 fp16, 90 % pruned, N=2048           (config 4)

plus the reference's ``checkers`` test shape (utils/matrix_gen.hpp:185-211),
the ``banded`` shape (utils/matrix_gen.hpp:69-90) and the ``triangular``
shape of the Tier-2 sweep (utils/matrix_gen.hpp:95-120).

Every generator takes ``dtype``: the same draws rounded to fp16 or fp32
(the default is the configuration's own type).
"""
from __future__ import annotations

from dataclasses import dataclass, field

import numpy as np


@dataclass
class Problem:
    name: str
    M: int
    K: int
    N: int
    rp: np.ndarray            # int32[M+1]
    ci: np.ndarray            # int32[nnz], sorted within each row
    vals: np.ndarray          # fp16 or fp32 [nnz]
    B: np.ndarray             # same dtype as vals, [K, N] row-major
    cluster: bool = False     # whether the config runs the clustering stage
    meta: dict = field(default_factory=dict)

    @property
    def nnz(self) -> int:
        return int(self.rp[-1])

    @property
    def dtype(self):
        return self.vals.dtype


def _csr_from_rows(M: int, rows: list[np.ndarray]):
    lens = np.fromiter((len(r) for r in rows), dtype=np.int64, count=M)
    rp = np.zeros(M + 1, np.int64)
    np.cumsum(lens, out=rp[1:])
    ci = np.concatenate(rows).astype(np.int32) if M else np.zeros(0, np.int32)
    return rp.astype(np.int32), ci


def _csr_from_coo(M: int, r: np.ndarray, c: np.ndarray):
    order = np.lexsort((c, r))
    r, c = r[order], c[order]
    counts = np.bincount(r, minlength=M)
    rp = np.zeros(M + 1, np.int64)
    np.cumsum(counts, out=rp[1:])
    return rp.astype(np.int32), c.astype(np.int32), order


def cpu_ref(seed: int = 0, N: int = 64, dtype=np.float32) -> Problem:
    """M=K=1024 fp32.  Each row draws 10 + Bernoulli(0.24) distinct columns
    uniformly without replacement (E[nnz/row] = 10.24, i.e. 1 %); columns
    sorted.  Values U(-1,1).  B is 1024x64 U(-1,1).  No clustering."""
    rng = np.random.default_rng(seed)
    M = K = 1024
    rows = []
    for _ in range(M):
        k = 10 + int(rng.random() < 0.24)
        rows.append(np.sort(rng.choice(K, size=k, replace=False)))
    rp, ci = _csr_from_rows(M, rows)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(dtype)
    B = rng.uniform(-1, 1, size=(K, N)).astype(dtype)
    return Problem("cpu_ref", M, K, N, rp, ci, vals, B, cluster=False)


def blocks(seed: int = 0, M: int = 8192, N: int = 256, frac: float = 0.05,
           dtype=np.float16) -> Problem:
    """M=K=8192 fp16.  round(frac * Mb * Kb) of the 16x16 blocks are chosen
    uniformly without replacement; each is fully dense with N(0,1) values.
    B is N(0,1).  No clustering (a Tier-1 workload)."""
    rng = np.random.default_rng(seed)
    K = M
    Mb, Kb = M // 16, K // 16
    nb = int(round(frac * Mb * Kb))
    sel = np.sort(rng.choice(Mb * Kb, size=nb, replace=False))
    bi, bj = sel // Kb, sel % Kb
    # expand each block into 256 entries
    ii = (bi[:, None] * 16 + np.repeat(np.arange(16), 16)[None, :]).ravel()
    jj = (bj[:, None] * 16 + np.tile(np.arange(16), 16)[None, :]).ravel()
    rp, ci, order = _csr_from_coo(M, ii, jj)
    vals = rng.standard_normal(len(ci)).astype(dtype)
    B = rng.standard_normal((K, N)).astype(dtype)
    return Problem("blocks", M, K, N, rp, ci, vals, B, cluster=False,
                   meta=dict(blocks=nb))


def templates(seed: int = 0, M: int = 16384, N: int = 128, n_templates: int = 1024,
              tcols: int = 82, keep: float = 0.7, dtype=np.float16) -> Problem:
    """M=K=16384 fp16, 0.5 % density.  1024 templates, each tcols=82 distinct
    uniform columns.  Row r uses template r mod 1024: it keeps a uniform
    subset of round(keep*82)=57 template columns and draws the other 25
    uniformly among columns not in the template (distinct).  Rows are then
    shuffled by a seeded permutation.  Values U(-1,1); B U(-1,1).  The config
    runs with clustering on (threshold 0.5, block width 16)."""
    rng = np.random.default_rng(seed)
    K = M
    tmpl = [rng.choice(K, size=tcols, replace=False) for _ in range(n_templates)]
    n_keep = int(round(keep * tcols))
    n_rand = tcols - n_keep
    rows = []
    for r in range(M):
        t = tmpl[r % n_templates]
        kept = rng.choice(t, size=n_keep, replace=False)
        while True:
            # distinct uniform draws, rejecting template columns
            cand = rng.choice(K, size=n_rand + 8, replace=False)
            cand = cand[~np.isin(cand, t)]
            if len(cand) >= n_rand:
                break
        rows.append(np.sort(np.concatenate([kept, cand[:n_rand]])))
    shuffle = rng.permutation(M)
    rows = [rows[i] for i in shuffle]
    rp, ci = _csr_from_rows(M, rows)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(dtype)
    B = rng.uniform(-1, 1, size=(K, N)).astype(dtype)
    return Problem("templates", M, K, N, rp, ci, vals, B, cluster=True,
                   meta=dict(n_templates=n_templates, tcols=tcols, keep=n_keep))


def _powerlaw_degrees(rng, M, alpha, dmax, mean):
    """Degrees floor(x) with x from a Pareto(alpha) truncated to
    [x_min, dmax+1); x_min is found by bisection so that E[d] = mean."""
    u = rng.random(M)

    def draw(xmin):
        a1 = 1.0 - alpha
        lo, hi = xmin ** a1, (dmax + 1.0) ** a1
        x = (lo + u * (hi - lo)) ** (1.0 / a1)
        return np.minimum(np.floor(x), dmax).astype(np.int64)

    lo, hi = 1.0, float(mean)
    for _ in range(60):
        mid = 0.5 * (lo + hi)
        if draw(mid).mean() < mean:
            lo = mid
        else:
            hi = mid
    return draw(hi)


def gnn(seed: int = 0, M: int = 131072, N: int = 64, alpha: float = 2.1,
        dmax: int = 4096, mean: float = 16.0, dtype=np.float16) -> Problem:
    """M=K=131072 adjacency.  Out-degrees d_i = floor(x_i), x_i from a
    Pareto(2.1) truncated to [x_min, 4097) with x_min bisected so the sample
    mean is 16; neighbours uniform without replacement; values 1/d_i (fp16).
    B is N(0,1) fp16.  Runs with clustering on."""
    rng = np.random.default_rng(seed)
    K = M
    deg = _powerlaw_degrees(rng, M, alpha, dmax, mean)
    rows = [np.sort(rng.choice(K, size=int(d), replace=False)) for d in deg]
    rp, ci = _csr_from_rows(M, rows)
    vals = np.repeat(1.0 / np.maximum(deg, 1), deg).astype(dtype)
    B = rng.standard_normal((K, N)).astype(dtype)
    return Problem("gnn", M, K, N, rp, ci, vals, B, cluster=True,
                   meta=dict(mean_degree=float(deg.mean()), max_degree=int(deg.max())))


def pruned(seed: int = 0, M: int = 14336, K: int = 4096, N: int = 2048,
           keep: float = 0.10, cluster: bool = False, dtype=np.float16) -> Problem:
    """A = 14336x4096 fp16 with exactly round(0.1*M*K) surviving positions,
    uniform without replacement (magnitude pruning of an N(0,0.02) weight);
    surviving values N(0,0.02).  B = 4096x2048 N(0,1) fp16."""
    rng = np.random.default_rng(seed)
    total = M * K
    nnz = int(round(keep * total))
    pos = np.sort(rng.choice(total, size=nnz, replace=False))
    r, c = pos // K, pos % K
    counts = np.bincount(r, minlength=M)
    rp = np.zeros(M + 1, np.int64)
    np.cumsum(counts, out=rp[1:])
    vals = (rng.standard_normal(nnz) * 0.02).astype(dtype)
    B = rng.standard_normal((K, N)).astype(dtype)
    return Problem("pruned", M, K, N, rp.astype(np.int32), c.astype(np.int32), vals, B,
                   cluster=cluster)


def checkers(M: int = 1024, K: int = 1024, N: int = 64, bs: int = 4, seed: int = 42,
             dtype=np.float32, shuffle: bool = True) -> Problem:
    """Entry (i, j) present iff (i//bs + j//bs) is odd (utils/matrix_gen.hpp:185-211),
    values U(0.1, 1), rows optionally shuffled; B = ones, so C[i, :] is the
    row sum of A (the closed form behind examples/01_uspmm_checkers.cpp)."""
    rng = np.random.default_rng(seed)
    rows = []
    for i in range(M):
        j = np.arange(K)
        rows.append(j[((i // bs + j // bs) % 2) == 1])
    if shuffle:
        order = rng.permutation(M)
        rows = [rows[i] for i in order]
    rp, ci = _csr_from_rows(M, rows)
    vals = rng.uniform(0.1, 1.0, size=len(ci)).astype(dtype)
    B = np.ones((K, N), dtype)
    return Problem("checkers", M, K, N, rp, ci, vals, B, cluster=True)


def banded(M: int = 1024, bandwidth: int = 8, N: int = 32, seed: int = 42,
           dtype=np.float32) -> Problem:
    """Band |i - j| <= bandwidth (utils/matrix_gen.hpp:69-90), values
    U(0.1, 1), B = ones (examples/05_core_spmm_benchmark.cpp:103-117)."""
    rng = np.random.default_rng(seed)
    rows = [np.arange(max(0, i - bandwidth), min(M - 1, i + bandwidth) + 1) for i in range(M)]
    rp, ci = _csr_from_rows(M, rows)
    vals = rng.uniform(0.1, 1.0, size=len(ci)).astype(dtype)
    B = np.ones((M, N), dtype)
    return Problem("banded", M, M, N, rp, ci, vals, B, cluster=False)


def triangular(size: int = 8192, density: float = 0.01, upper: bool = True, N: int | None = None,
               seed: int = 42, dtype=np.float32) -> Problem:
    """The triangular shape of the reference's Tier-2 sweep
    (examples/02_spmm_benchmark.cpp:60-61, :268-269; utils/matrix_gen.hpp:95-120):
    entry (i, j) of the upper (lower) triangle is present with probability
    `density`, the diagonal always, values U(0.1, 1); seeded here with numpy,
    not the reference's mt19937.  N defaults to `size` (examples/02 runs
    N = M = K); B is U(-1, 1) here (examples/02 uses ones, which would hide a
    column mix-up).  The sweep runs the Tier-2 pipeline with clustering on."""
    rng = np.random.default_rng(seed)
    N = size if N is None else N
    rows = []
    for i in range(size):
        lo, hi = (i, size) if upper else (0, i + 1)
        j = np.arange(lo, hi)
        keep = rng.random(hi - lo) < density
        keep[i - lo] = True
        rows.append(j[keep])
    rp, ci = _csr_from_rows(size, rows)
    vals = rng.uniform(0.1, 1.0, size=len(ci)).astype(dtype)
    B = rng.uniform(-1, 1, size=(size, N)).astype(dtype)
    return Problem("triangular", size, size, N, rp, ci, vals, B, cluster=True,
                   meta=dict(density=density, upper=upper))


# the density sweep of examples/05_core_spmm_benchmark.cpp:67-77
SWEEP_DENSITIES = {"90": 0.90, "50": 0.50, "5": 0.05, "0.5": 0.005, "0.1": 0.001}


def banded_sweep(density: float, M: int = 16384, N: int = 128, seed: int = 42,
                 dtype=np.float16) -> Problem:
    """The reference's Tier-1 density sweep (examples/05_core_spmm_benchmark.cpp:
    56-77, :103-117): A = M x M banded, bandwidth int(density * M / 2)
    (at least 1), every entry |i - j| <= bandwidth present with a value
    U(0.1, 1) (utils/matrix_gen.hpp:69-90; seeded here with numpy, not the
    reference's mt19937); B = ones, so C[i, :] is row i's sum; N = 128."""
    bw = max(1, int(density * M / 2.0))
    i = np.arange(M, dtype=np.int64)
    start = np.maximum(0, i - bw)
    end = np.minimum(M - 1, i + bw)
    lens = end - start + 1
    rp = np.zeros(M + 1, np.int64)
    np.cumsum(lens, out=rp[1:])
    nnz = int(rp[-1])
    # column of entry e in row r: start[r] + (e - rp[r])
    ci = (np.arange(nnz, dtype=np.int64) - np.repeat(rp[:-1] - start, lens)).astype(np.int32)
    rng = np.random.default_rng(seed)
    vals = rng.uniform(0.1, 1.0, size=nnz).astype(dtype)
    B = np.ones((M, N), dtype)
    return Problem(f"banded{density * 100:g}", M, M, N, rp.astype(np.int32), ci, vals, B,
                   cluster=False, meta=dict(bandwidth=bw, density=density))


def random_csr(M: int, K: int, N: int, density: float, seed: int = 0, dtype=np.float16,
               unsorted: bool = False, dup_frac: float = 0.0) -> Problem:
    """Uniform random CSR for parity tests: Binomial row lengths, optional
    unsorted columns and duplicated entries (same row, same column)."""
    rng = np.random.default_rng(seed)
    rows = []
    for _ in range(M):
        k = min(K, rng.binomial(K, density)) if K else 0
        r = rng.choice(K, size=k, replace=False) if k else np.zeros(0, np.int64)
        if dup_frac > 0 and k:
            nd = max(1, int(dup_frac * k))
            r = np.concatenate([r, rng.choice(r, size=nd)])
        r = rng.permutation(r) if unsorted else np.sort(r)
        rows.append(r)
    rp, ci = _csr_from_rows(M, rows)
    vals = rng.uniform(-1, 1, size=len(ci)).astype(dtype)
    B = rng.uniform(-1, 1, size=(K, N)).astype(dtype)
    return Problem("random", M, K, N, rp, ci, vals, B)


CONFIGS = {
    "cpu_ref": cpu_ref,
    "blocks": blocks,
    "templates": templates,
    "gnn": gnn,
    "pruned": pruned,
}
for _name, _d in SWEEP_DENSITIES.items():
    CONFIGS[f"banded{_name}"] = (lambda d: lambda **kw: banded_sweep(d, **kw))(_d)
    # the sweep in fp32, the type examples/05 runs it in (ValueType = float, :25)
    CONFIGS[f"banded{_name}_f32"] = (
        lambda d: lambda **kw: banded_sweep(d, **{"dtype": np.float32, **kw}))(_d)
