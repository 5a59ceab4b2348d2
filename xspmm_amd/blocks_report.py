"""Block analysis of MatrixMarket matrices on the GPU.

The analysis of the reference's examples/04_real_matrices_benchmark.cpp:104-155
for each matrix:
  * read the file (xspmm_mtx_*, the reference reader's result);
  * count the 16x16 blocks of A ("Blocks Before");
  * cluster the rows (Jaccard, threshold 0.5, width 16), permute, count again
    ("Blocks After"), and report the reduction;
then time, for each N, the Tier-2 pipeline on the original matrix with
B = ones (as the example does) and this library's prepared product.

    python -m xspmm_amd.blocks_report PATH [PATH ...] [--N 64,256] [--fp16]
                                      [--gpu-cluster] [--json]

PATH is a .mtx file or a directory searched for *.mtx.  Values are fp32 like
the example's; --fp16 reads them as fp16.  Clustering runs the host greedy,
as the reference does, unless --gpu-cluster.  With --json one JSON line per
matrix is printed instead of the text report.
"""
from __future__ import annotations

import argparse
import glob
import json
import os
import sys
import time

import numpy as np

import xspmm_amd as X


def mtx_files(paths):
    out = []
    for p in paths:
        if os.path.isdir(p):
            out += sorted(glob.glob(os.path.join(p, "*.mtx")))
        else:
            out.append(p)
    return out


def analyse(path, Ns=(64,), fp16=False, gpu_cluster=False, warmup=2, iters=10):
    import torch
    t0 = time.perf_counter()
    M, K, rp, ci, vals = X.read_mtx(path, np.int32, np.float16 if fp16 else np.float32)
    read_s = time.perf_counter() - t0
    nnz = len(ci)
    A = X.CSRMatrix.from_host(M, K, rp, ci, vals)
    blocks_before = X.csr_to_bcsr(A).num_blocks
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    if gpu_cluster:
        perm = X.jaccard_clustering(A, 0.5, 16)
    else:
        perm = torch.as_tensor(X.compute_1d_jaccard_clustering(M, K, rp, ci, 0.5, 16)).cuda()
    torch.cuda.synchronize()
    cluster_ms = (time.perf_counter() - t0) * 1e3
    Ap = X.apply_permutation(A, perm)
    blocks_after = X.csr_to_bcsr(Ap).num_blocks
    saved = blocks_before - blocks_after
    rec = {
        "file": os.path.basename(path), "M": M, "K": K, "nnz": nnz,
        "density_pct": 100.0 * nnz / (M * K) if M and K else 0.0,
        "blocks_before": blocks_before, "blocks_after": blocks_after,
        "blocks_saved": saved,
        "reduction_pct": 100.0 * saved / blocks_before if blocks_before else 0.0,
        "read_s": read_s, "clustering_ms": cluster_ms,
        "clustering": "gpu" if gpu_cluster else "host", "runs": [],
    }
    if gpu_cluster:
        os.environ["XSPMM_CLUSTER_DEVICE"] = "gpu"
    try:
        plan = X.SpMMPlan(A)
        for N in Ns:
            B = torch.ones((K, N), dtype=A.values.dtype, device=A.row_ptr.device)
            C = torch.empty((M, N), dtype=torch.float32, device=A.row_ptr.device)
            for _ in range(warmup):
                X.spmm_pipeline(A, B, C)
            torch.cuda.synchronize()
            _, st = X.spmm_pipeline(A, B, C)
            for _ in range(warmup):
                plan.execute(B, C)
            a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            a.record()
            for _ in range(iters):
                plan.execute(B, C)
            b.record()
            torch.cuda.synchronize()
            ex = a.elapsed_time(b) / iters
            rec["runs"].append({"N": N, "pipeline_ms": st, "plan_execute_ms": ex,
                                "plan_tflops": 2.0 * nnz * N / (ex * 1e-3) / 1e12 if ex > 0 else 0.0})
        plan.close()
    finally:
        if gpu_cluster:
            del os.environ["XSPMM_CLUSTER_DEVICE"]
    return rec


def report_text(rec):
    # the example's summary lines (examples/04:151-155), then the timings
    lines = [f">>> Loaded: {rec['file']} ({rec['M']}x{rec['K']})",
             f"    Blocks Before : {rec['blocks_before']}",
             f"    Blocks After  : {rec['blocks_after']}",
             f"    Reduction     : {rec['blocks_saved']} blocks ({rec['reduction_pct']:.2f}%)"]
    for r in rec["runs"]:
        st = r["pipeline_ms"]
        lines.append(f"    N={r['N']:<5d} pipeline total {st['total_pipeline_ms']:9.3f} ms "
                     f"(clustering {st['clustering_ms']:.3f}, spmm {st['spmm_ms']:.3f}) | "
                     f"prepared execute {r['plan_execute_ms']:.4f} ms = {r['plan_tflops']:.3f} TFLOPS")
    return "\n".join(lines)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("paths", nargs="+")
    ap.add_argument("--N", default="64", help="comma-separated N values")
    ap.add_argument("--fp16", action="store_true")
    ap.add_argument("--gpu-cluster", action="store_true")
    ap.add_argument("--json", action="store_true")
    args = ap.parse_args(argv)
    Ns = [int(x) for x in args.N.split(",") if x]
    files = mtx_files(args.paths)
    if not files:
        print("no .mtx files found", file=sys.stderr)
        return 1
    for f in files:
        rec = analyse(f, Ns, args.fp16, args.gpu_cluster)
        print(json.dumps(rec) if args.json else report_text(rec), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
