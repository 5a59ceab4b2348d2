"""GPU: the block analysis of MatrixMarket matrices (xspmm_amd.blocks_report),
the analysis of the reference's examples/04_real_matrices_benchmark.cpp:104-155.
Block counts before and after clustering must equal the oracle's (its
CSR->BCSR count on the read matrix and on the matrix permuted by its greedy).
"""
from __future__ import annotations

import json
import os

import numpy as np
import pytest

import oracle
import xspmm_amd as X
from tests.helpers import GOLDEN
from xspmm_amd import blocks_report

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def torch():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need an MI355X (torch.cuda.is_available() is False)")
    X.load()
    return torch


def write_mtx(path, M, K, rows, rng):
    lines = ["%%MatrixMarket matrix coordinate real general", f"{M} {K} {sum(map(len, rows))}"]
    ents = [(r, c) for r, cols in enumerate(rows) for c in cols]
    rng.shuffle(ents)
    for r, c in ents:
        lines.append(f"{r + 1} {c + 1} {rng.uniform(-1, 1):.5f}")
    with open(path, "w") as f:
        f.write("\n".join(lines) + "\n")


def oracle_blocks(path):
    M, K, rp, ci, vals = oracle.read_mtx(path)
    before = len(oracle.csr_to_bcsr(M, K, rp, ci, vals)[1])
    perm = oracle.jaccard(M, K, rp, ci)
    nrp, nci, nv = oracle.apply_perm(M, rp, ci, vals, perm)
    after = len(oracle.csr_to_bcsr(M, K, nrp, nci, nv)[1])
    return before, after


def clustered_rows(rng, M, K):
    base = [np.unique(rng.choice(K, size=int(rng.integers(8, 40)), replace=False)) for _ in range(25)]
    rows = []
    for r in rng.permutation(M):
        b = base[r % len(base)]
        rows.append(np.unique(np.concatenate([b[rng.random(len(b)) < 0.95],
                                              rng.integers(0, K, size=2)])))
    return rows


@pytest.mark.parametrize("gpu_cluster", [False, True])
def test_block_counts_match_oracle(torch, tmp_path, gpu_cluster):
    rng = np.random.default_rng(3)
    path = str(tmp_path / "clustered.mtx")
    write_mtx(path, 2000, 1500, clustered_rows(rng, 2000, 1500), rng)
    for p in (path, os.path.join(GOLDEN, "mtx", "random_1000x800.mtx")):
        rec = blocks_report.analyse(p, Ns=(64, 13), gpu_cluster=gpu_cluster, warmup=1, iters=2)
        before, after = oracle_blocks(p)
        print(blocks_report.report_text(rec), flush=True)
        assert (rec["blocks_before"], rec["blocks_after"]) == (before, after)
        assert len(rec["runs"]) == 2 and all(r["plan_execute_ms"] > 0 for r in rec["runs"])
    assert rec["blocks_before"] >= rec["blocks_after"]


def test_cli_text_and_json(torch, tmp_path, capsys):
    rng = np.random.default_rng(4)
    write_mtx(str(tmp_path / "a.mtx"), 300, 200, clustered_rows(rng, 300, 200), rng)
    write_mtx(str(tmp_path / "b.mtx"), 100, 90, clustered_rows(rng, 100, 90), rng)
    assert blocks_report.main([str(tmp_path), "--N", "16,24"]) == 0
    out = capsys.readouterr().out
    assert out.count(">>> Loaded:") == 2 and "Blocks Before" in out and "Reduction" in out
    assert blocks_report.main([str(tmp_path / "a.mtx"), "--json", "--fp16"]) == 0
    rec = json.loads(capsys.readouterr().out.strip())
    before, after = oracle_blocks(str(tmp_path / "a.mtx"))
    assert (rec["blocks_before"], rec["blocks_after"]) == (before, after)
