#!/usr/bin/env python3
"""Headline benchmark: BCSR SpMM on one MI355X.

Workload (default `templates`, BASELINE configs[2], the configuration the
north-star target is quoted on): A = 16384 x 16384 fp16, 0.5 % dense, rows
from 1024 column-pattern templates, shuffled; B = 16384 x 128 fp16; C fp32.
The Tier-2 preparation runs once, untimed by the step loop and reported
separately: Jaccard clustering (threshold 0.5, width 16; timed on the host
and on the GPU, which must give the same permutation) -> GPU row
permutation -> GPU CSR->BCSR.  A step is one Tier-1 SpMM call
C = A_bcsr * B on device-resident inputs (for fp16 one launch of the
column-batch MFMA kernel); the K steps are timed launched from Python and
replayed from one captured HIP graph, and the faster counts, so that host
launch overhead is not what a small product's line times.  `value` is the
effective throughput 2*nnz*N / t.

The JSON line also carries:
  roofline      algorithmic HBM bytes per call / measured call time vs 8 TB/s;
                `traffic` is the measured HBM bytes per call from rocprofv3
                FETCH_SIZE + WRITE_SIZE (profiles/spmm_traffic.json) when
                that profile exists, else null;
  cpu_baseline  the same BCSR SpMM on the host cores (C oracle, fp32
                accumulation), repeated over the full matrix for ~10 s.
Usage: python bench.py [--steps K] [--warmup W] [--config NAME]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

METRIC = "effective TFLOPS (2·nnz·N/t) + % HBM roofline, BCSR SpMM on 1 MI355X"
HBM_PEAK_GBS = 8000.0
FP16_PEAK_TFLOPS = 2500.0
FP32_MFMA_PEAK_TFLOPS = 157.3

WORKLOADS = {
    "templates": "configs[2]: 16384^2 fp16, 0.5%, 1024 templates x 82 cols, shuffled, "
                 "clustering on, N=128",
    "blocks": "configs[1]: 8192^2 fp16, 5% dense 16x16 blocks, N=256, Tier-1",
    "cpu_ref": "configs[0]: 1024^2 fp32, 1% uniform, N=64",
    "pruned": "configs[4]: 14336x4096 fp16, 90% pruned, N=2048, clustering off",
    "gnn": "configs[3]: 131072^2 power-law adjacency fp16, N=64, clustering on",
}
for _d in ("90", "50", "5", "0.5", "0.1"):
    WORKLOADS[f"banded{_d}"] = (f"examples/05 density sweep: banded 16384^2 at {_d}% "
                                "(bandwidth density*K/2), fp16, B = ones, N=128, Tier-1")
    WORKLOADS[f"banded{_d}_f32"] = (f"examples/05 density sweep as the reference runs it: banded "
                                    f"16384^2 at {_d}% (bandwidth density*K/2), fp32, B = ones, "
                                    "N=128, Tier-1")


def host_threads() -> int:
    n = len(os.sched_getaffinity(0))
    env = os.environ.get("OMP_NUM_THREADS")
    if env and env.isdigit():
        n = min(n, int(env))
    return max(1, n)


def cpu_baseline(p, N, nnz, seconds):
    """C oracle BCSR SpMM (fp32 accumulation) on all host threads, repeated
    over the whole matrix until `seconds` have elapsed; median per call."""
    import oracle

    t0 = time.perf_counter()
    brp, bci, bv = oracle.csr_to_bcsr(p.M, p.K, p.rp, p.ci, p.vals)
    conv_ms = (time.perf_counter() - t0) * 1e3
    threads = host_threads()

    def run(nthreads, budget, cap):
        times = []
        t_end = time.perf_counter() + budget
        while time.perf_counter() < t_end or not times:
            t0 = time.perf_counter()
            oracle.bcsr_spmm_f32(p.M, p.K, N, brp, bci, bv, p.B, nthreads=nthreads)
            times.append(time.perf_counter() - t0)
            if len(times) >= cap:
                break
        return statistics.median(times), len(times)

    t, n = run(threads, seconds, 200)
    # one thread, as the reference's CpuExecutor would run, when a call fits
    # the budget (estimated from the all-thread time)
    single = None
    if t * threads <= seconds:
        t1, n1 = run(1, seconds / 3, 20)
        single = {"value": 2.0 * nnz * N / t1 / 1e12, "ms_per_call": t1 * 1e3, "runs": n1}
    return {
        "value": 2.0 * nnz * N / t / 1e12,
        "unit": "TFLOPS",
        "cores": threads,
        "kind": "port",
        "sample": f"whole matrix ({len(bci)} blocks), {n} runs, median "
                  f"{t * 1e3:.1f} ms/call; BCSR tile product with fp32 accumulation "
                  f"(oracle/oracle.c xo_bcsr_spmm_f32)",
        "single_thread": single,
        "csr_to_bcsr_ms": conv_ms,
    }


def tier1_kernel(value_bytes, K, N, nnzb, Mb, band=False):
    """Name of the kernel one Tier-1 call launches (the launcher's own rule in
    xspmm_amd/csrc/spmm.hip: a grid csr_to_bcsr found to have contiguous,
    overlapping block-rows (`band`) takes the band kernel of its type where
    it covers the shape (fp16: N % 8 == 0; fp32: N % 4 == 0; B within 32-bit
    offsets); else fp16 takes the GEMM-tiled kernel when every block
    is present, else the column-batch kernel when N % 8 == 0 and B and the
    block grid fit its 32-bit offsets, unless XSPMM_SPMM_KERNEL selects
    another one; fp32 takes its column-batch kernel when N % 4 == 0 and B
    fits 32-bit offsets and the grid has at least 512 workgroups of 128
    columns, unless XSPMM_F32_KERNEL=tile or =batch forces one; otherwise
    the short-grid kernel where 64 * Kb * N <= 2^30, unless
    XSPMM_F32_SHORT=off)."""
    if value_bytes == 4:
        Kb = (K + 15) // 16
        if band and N % 4 == 0 and K * N * 4 <= 1 << 31 and N < 1 << 22 and Kb < 1 << 20:
            return "spmm_f32_band_kernel"
        choice = os.environ.get("XSPMM_F32_KERNEL", "")
        if (N % 4 == 0 and K * N * 4 <= 1 << 31 and Kb < 1 << 21 and choice != "tile"
                and (choice == "batch" or Mb * ((N + 127) // 128) >= 512)):
            return "spmm_f32_batch_kernel"
        if 64 * Kb * N <= 1 << 30 and os.environ.get("XSPMM_F32_SHORT", "") != "off":
            return "spmm_f32_short_kernel"
        return "spmm_f32_kernel"
    Kb = (K + 15) // 16
    fits = K * N * 2 <= 1 << 31 and N < 1 << 22 and Kb < 1 << 20
    if band and N % 8 == 0 and fits:
        return "spmm_f16_band_kernel"
    if (nnzb == Mb * Kb and N % 8 == 0 and Mb * Kb * 512 < 1 << 31 and K * N * 2 < 1 << 31
            and os.environ.get("XSPMM_SPMM_KERNEL", "") == ""):
        return "spmm_f16_dense_kernel"
    choice = os.environ.get("XSPMM_SPMM_KERNEL", "")
    if choice in ("", "batch") and N % 8 == 0 and fits:
        return "spmm_f16_batch_kernel"
    if choice == "gather" and N % 2 == 0 and fits:
        return "spmm_f16_gather_kernel"
    return "pack_b_panels + spmm_f16_kernel"


def _profile_json(name):
    try:
        with open(os.path.join(ROOT, "profiles", name)) as f:
            return json.load(f)
    except (OSError, ValueError):
        return {}


def load_traffic(config):
    """HBM bytes per SpMM launch from the committed rocprofv3 counter runs
    (profiles/spmm_traffic.json): FETCH_SIZE and WRITE_SIZE in KiB per
    dispatch, each scaled by what the same counter reads for a plain copy of
    known size (`bench.py --calibrate-copy`).  None when not profiled."""
    d = _profile_json("spmm_traffic.json")
    e = d.get("configs", {}).get(config)
    cal = d.get("calibration")
    if not e or not cal:
        return None
    return (e["fetch_kib"] * cal["fetch_scale"] + e["write_kib"] * cal["write_scale"]) * 1024.0


def load_mfma_busy(config):
    """Share of cycles the SpMM kernel's matrix cores were busy, from the
    committed rocprofv3 counter run (profiles/spmm_mfma_busy.json:
    SQ_VALU_MFMA_BUSY_CYCLES over the SIMD-cycles of the dispatch).  None when
    not profiled."""
    e = _profile_json("spmm_mfma_busy.json").get("configs", {}).get(config)
    return e.get("mfma_busy") if e else None


def calibrate_copy():
    """A plain device copy of known size, for scaling the rocprofv3 byte
    counters: 3 launches of dst.copy_(src) over 512 MiB (512 MiB read and
    512 MiB written per launch)."""
    import torch

    n = 512 << 20
    src = torch.ones(n // 2, dtype=torch.float16, device="cuda")
    dst = torch.empty_like(src)
    torch.cuda.synchronize()
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibration_copy_bytes_read": n, "calibration_copy_bytes_written": n,
                      "launches": 3}), flush=True)


def vendor_columns(Ap, Bm, B, C, ms, iters):
    """The same product by rocSPARSE (CSR, BSR) and rocBLAS (dense A, when it
    fits in 512 MB), each with its time and its relative Frobenius difference
    from this library's C (same inputs, fp32 accumulation)."""
    import torch
    from xspmm_amd import vendor as V

    def rel(Cv):
        return float(torch.linalg.norm(Cv - C) / max(float(torch.linalg.norm(C)), 1e-30))

    out = {"xspmm_ms": ms}
    iters = max(5, min(iters, 50))
    try:
        if Ap.row_ptr.dtype == torch.int32:
            Cv, t = V.csr_spmm(Ap, B, iters=iters)
            out.update(rocsparse_csr_ms=t, rocsparse_csr_rel_diff=rel(Cv), speedup_vs_csr=t / ms)
            Kp = Bm.num_block_cols * 16
            Bp = B if Kp == B.shape[0] else torch.cat(
                [B, torch.zeros((Kp - B.shape[0], B.shape[1]), dtype=B.dtype, device=B.device)])
            Cv, t = V.bsr_spmm(Bm, Bp, iters=iters)
            out.update(rocsparse_bsr_ms=t, rocsparse_bsr_rel_diff=rel(Cv), speedup_vs_bsr=t / ms)
            del Cv
        M, K = Ap.num_rows, Ap.num_cols
        if M * K * B.element_size() <= (512 << 20):
            D = torch.zeros((M, K), dtype=B.dtype, device=B.device)
            lens = Ap.row_ptr[1:] - Ap.row_ptr[:-1]
            rows = torch.repeat_interleave(torch.arange(M, device=B.device), lens.long())
            D[rows, Ap.col_ind.long()] = Ap.values
            Cv, t = V.dense_gemm(D, B, iters=iters)
            out.update(rocblas_dense_ms=t, rocblas_dense_rel_diff=rel(Cv), speedup_vs_dense=t / ms)
            del D, Cv
        torch.cuda.synchronize()
    except Exception as e:  # the comparison is context; report why it is missing
        out["error"] = str(e)
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--config", default="templates", choices=sorted(WORKLOADS))
    ap.add_argument("--n", type=int, default=None,
                    help="width N of B and C (default: the workload's own N)")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--cluster", choices=("config", "on", "off"), default="config",
                    help="override the workload's clustering setting")
    ap.add_argument("--dtype", choices=("config", "f16", "f32"), default="config",
                    help="value type of A and B (default: the workload's own; the same "
                         "draws rounded to the other type)")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-pipeline", action="store_true")
    ap.add_argument("--no-vendor", action="store_true",
                    help="skip the rocSPARSE / rocBLAS comparison columns")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only the known-size copy used to scale byte counters")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py measures one GPU only (this build has no multi-GPU path); "
              f"got --gpus {args.gpus}", file=sys.stderr)
        sys.exit(2)

    import numpy as np
    import torch

    import xspmm_amd as X
    from xspmm_amd import synth

    if not torch.cuda.is_available():
        print("bench.py needs an MI355X", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if args.calibrate_copy:
        calibrate_copy()
        return
    X.load()

    print(f"[bench] generating {args.config}", file=sys.stderr, flush=True)
    gen_kw = {"N": args.n} if args.n else {}
    if args.dtype != "config":
        gen_kw["dtype"] = np.float16 if args.dtype == "f16" else np.float32
    p = synth.CONFIGS[args.config](**gen_kw)
    if args.cluster != "config":
        p.cluster = args.cluster == "on"
    M, K, N, nnz = p.M, p.K, p.N, p.nnz
    A = X.CSRMatrix.from_host(M, K, p.rp, p.ci, p.vals)
    B = torch.as_tensor(p.B).cuda()

    # --- Tier-2 preparation (once) -----------------------------------------
    prep = {}
    if p.cluster:
        # the same permutation twice: host greedy (the reference's placement)
        # and the GPU engine; both wall-clock, the GPU one including its
        # preparation kernels and final synchronization
        t0 = time.perf_counter()
        perm = X.compute_1d_jaccard_clustering(M, K, p.rp, p.ci, 0.5, 16)
        prep["clustering_host_ms"] = (time.perf_counter() - t0) * 1e3
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        perm_d, engine = X.jaccard_clustering(A, 0.5, 16, return_engine=True)
        torch.cuda.synchronize()
        prep["clustering_gpu_ms"] = (time.perf_counter() - t0) * 1e3
        prep["clustering_gpu_engine"] = engine
        prep["clustering_gpu_equals_host"] = bool(np.array_equal(perm_d.cpu().numpy(), perm))
    else:
        perm = np.arange(M, dtype=p.rp.dtype)
        perm_d = torch.as_tensor(perm).cuda()
    torch.cuda.synchronize()
    e0, e1, e2 = (torch.cuda.Event(enable_timing=True) for _ in range(3))
    e0.record()
    Ap = X.apply_permutation(A, perm_d) if p.cluster else A
    e1.record()
    Bm = X.csr_to_bcsr(Ap)
    e2.record()
    torch.cuda.synchronize()
    prep["permutation_ms"] = e0.elapsed_time(e1)
    prep["conversion_ms"] = e1.elapsed_time(e2)
    nnzb, Mb = Bm.num_blocks, Bm.num_block_rows
    C = torch.empty((M, N), dtype=torch.float32, device="cuda")

    # --- timed Tier-1 steps ------------------------------------------------
    # The K steps are timed twice: launched from the Python loop, and replayed
    # from one captured HIP graph of the same K calls.  A step is one Tier-1
    # call (one kernel launch over the whole product) either way.  A
    # Python -> ctypes call costs about 10 us of host time, more than a small
    # product's kernel, so the eager loop times the host there; on large
    # products the eager launches queue back to back and run slightly ahead of
    # graph replay.  ms_per_step is the faster of the two (`timing` names it),
    # and the replay must leave C bit-identical to the eager calls.
    print(f"[bench] nnz={nnz} nnzb={nnzb}; warmup {args.warmup}", file=sys.stderr, flush=True)
    for _ in range(args.warmup):
        X.spmm(Bm, B, C, N)
    torch.cuda.synchronize()
    start, stop = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    wall0 = time.perf_counter()
    start.record()
    for _ in range(args.steps):
        X.spmm(Bm, B, C, N)
    stop.record()
    torch.cuda.synchronize()
    wall_eager = time.perf_counter() - wall0
    ms_eager = start.elapsed_time(stop) / args.steps
    C_eager = C.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        X.spmm(Bm, B, C, N)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(args.steps):
            X.spmm(Bm, B, C, N)
    torch.cuda.synchronize()
    graph.replay()  # untimed first replay
    torch.cuda.synchronize()
    C.fill_(float("nan"))
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    start.record()
    graph.replay()
    stop.record()
    torch.cuda.synchronize()
    wall_graph = time.perf_counter() - wall0
    ms_graph = start.elapsed_time(stop) / args.steps
    graph_equal = bool(torch.equal(C, C_eager))
    del graph, C_eager
    if not graph_equal:
        print("[bench] graph replay differs from the eager calls", file=sys.stderr, flush=True)
        sys.exit(1)
    if ms_graph < ms_eager:
        ms, wall, timing = ms_graph, wall_graph, "graph"
    else:
        ms, wall, timing = ms_eager, wall_eager, "eager"
    t = ms * 1e-3
    print(f"[bench] {args.steps} steps, {ms:.4f} ms/step ({timing}; eager {ms_eager:.4f}, "
          f"graph {ms_graph:.4f})", file=sys.stderr, flush=True)

    # spot check of C on sampled rows against an fp64 numpy product
    # (C is in the permuted row order: its row r is row perm[r] of A * B).
    # Elementwise sums, not a BLAS call: BLAS worker threads keep spinning
    # after a call and would slow the host clustering timed below.
    rows = np.random.default_rng(0).choice(M, size=min(256, M), replace=False)
    Ch = C.cpu().numpy()[rows].astype(np.float64)
    src = perm[rows]
    ref = np.stack([(p.vals[p.rp[r]:p.rp[r + 1]].astype(np.float64)[:, None]
                     * p.B[p.ci[p.rp[r]:p.rp[r + 1]]].astype(np.float64)).sum(axis=0) for r in src])
    spot = float(np.sqrt(np.sum((Ch - ref) ** 2)) / max(np.sqrt(np.sum(ref ** 2)), 1e-300))

    sT = p.vals.dtype.itemsize
    sI = p.rp.dtype.itemsize
    alg_bytes = nnzb * 256 * sT + nnzb * sI + (Mb + 1) * sI + K * N * sT + M * N * 4
    achieved = alg_bytes / t / 1e9
    eff = 2.0 * nnz * N / t / 1e12
    padded = 2.0 * nnzb * 256 * N / t / 1e12
    mfma_peak = FP16_PEAK_TFLOPS if sT == 2 else FP32_MFMA_PEAK_TFLOPS
    kernel = tier1_kernel(sT, K, N, nnzb, Mb, band=Bm.band_rows())
    # Matrix-core work the kernel executes: the column-batch kernels multiply
    # only the block columns that hold a non-zero entry (32 flops per such
    # column, row and output column: 16 rows x multiply-add), the other
    # kernels every block whole (the padded flops).  The bound is whichever of
    # HBM (algorithmic bytes) and the matrix cores (executed flops) the call
    # uses the larger share of.
    if "batch" in kernel:
        vals = Bm.values.view(-1, 16, 16)
        ncols = 0
        for i in range(0, vals.shape[0], 1 << 20):  # chunks bound the temporary
            ncols += int((vals[i:i + (1 << 20)] != 0).any(dim=1).sum())
        exec_flops = 32.0 * ncols * N
    else:
        ncols = None
        exec_flops = 2.0 * nnzb * 256 * N
    exec_tflops = exec_flops / t / 1e12
    hbm_frac = achieved / HBM_PEAK_GBS
    mfma_frac = exec_tflops / mfma_peak
    if mfma_frac > hbm_frac:
        roofline = {"bound": "mfma", "achieved": exec_tflops, "peak": mfma_peak, "unit": "TFLOP/s",
                    "frac": mfma_frac}
    else:
        roofline = {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                    "frac": hbm_frac}
    traffic_key = args.config + ("" if args.n is None else f"_n{args.n}")
    if args.dtype != "config" and not args.config.endswith("_" + args.dtype):
        traffic_key += "_" + args.dtype
    roofline.update({"traffic": load_traffic(traffic_key), "kernel": kernel,
                     "alg_bytes_per_call": alg_bytes,
                     "padded_flops_per_call": 2.0 * nnzb * 256 * N,
                     "executed_mfma_flops_per_call": exec_flops,
                     "nonzero_block_columns": ncols,
                     "hbm_frac": hbm_frac, "mfma_frac": mfma_frac})

    stages = stages_gpu = stages_bcsr = None
    pipe_form = None
    # Tier-2 stage times after untimed warm-up calls, as the reference's own
    # pipeline benchmark takes them (examples/02_spmm_benchmark.cpp:64, :122-124:
    # three warm-up calls, then one call with SpMMTimings)
    pipe_warmup = max(1, min(args.warmup, 3))
    if not args.no_pipeline:
        for _ in range(pipe_warmup):
            X.spmm_pipeline(A, B, optimize_pattern=p.cluster, timings=False)
        _, stages = X.spmm_pipeline(A, B, optimize_pattern=p.cluster)
        torch.cuda.synchronize()
        pipe_form = "packed column batches" if X.pipeline_last_packed() else "bcsr"
        if p.cluster:
            # the same pipeline with the clustering stage on the GPU engine
            os.environ["XSPMM_CLUSTER_DEVICE"] = "gpu"
        try:
            if p.cluster:
                for _ in range(pipe_warmup):
                    X.spmm_pipeline(A, B, optimize_pattern=True, timings=False)
                _, stages_gpu = X.spmm_pipeline(A, B, optimize_pattern=True)
                torch.cuda.synchronize()
            if pipe_form != "bcsr":
                # the BCSR form of the same pipeline (the reference's stage
                # sequence: padded blocks, Tier-1 SpMM, un-permutation)
                os.environ["XSPMM_PIPELINE_FORMAT"] = "bcsr"
                for _ in range(pipe_warmup):
                    X.spmm_pipeline(A, B, optimize_pattern=p.cluster, timings=False)
                _, stages_bcsr = X.spmm_pipeline(A, B, optimize_pattern=p.cluster)
                torch.cuda.synchronize()
        finally:
            os.environ.pop("XSPMM_CLUSTER_DEVICE", None)
            os.environ.pop("XSPMM_PIPELINE_FORMAT", None)

    # prepared product (plan): per-call time of execute(), which is the
    # Tier-1 SpMM with the un-permutation fused and the dispatch order
    # precomputed, against the pipeline's per-call SpMM + un-permutation
    plan_info = None
    if p.cluster and not args.no_pipeline:
        plan = X.SpMMPlan(A)
        Cp = torch.empty((M, N), dtype=torch.float32, device="cuda")
        for _ in range(args.warmup):
            plan.execute(B, Cp)
        torch.cuda.synchronize()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        a.record()
        for _ in range(args.steps):
            plan.execute(B, Cp)
        b.record()
        torch.cuda.synchronize()
        Cq, _ = X.spmm_pipeline(A, B, optimize_pattern=True)
        torch.cuda.synchronize()
        ex_ms = a.elapsed_time(b) / args.steps
        plan_info = {"execute_ms": ex_ms,
                     "prepare_ms": plan.timings["total_pipeline_ms"],
                     "equals_pipeline": bool(torch.equal(Cp, Cq)),
                     "packed_batches": plan.packed_batches,
                     "effective_tflops": 2.0 * nnz * N / (ex_ms * 1e-3) / 1e12}
        if plan.packed_batches > 0:
            # streamed per call: per batch the packed A' and B-row indices
            # (fp16: 1 KB + 128 B, offsets for 4 waves per block-row; fp32:
            # 256 B + 16 B, one offset per block-row), B once, C once, the
            # permutation once
            f16 = p.vals.dtype.itemsize == 2
            per_batch, per_row = (1152, 4) if f16 else (272, 1)
            pb = (plan.packed_batches * per_batch + (per_row * Mb + 1) * 8
                  + K * N * p.vals.dtype.itemsize + M * N * 4 + M * p.rp.dtype.itemsize)
            plan_info.update(bytes_per_call=pb, achieved_gbs=pb / (ex_ms * 1e-3) / 1e9,
                             hbm_frac=pb / (ex_ms * 1e-3) / 1e9 / HBM_PEAK_GBS)
            if not f16:
                # executed matrix-core work: per batch and 64 columns, four
                # v_mfma_f32_16x16x4f32 (16 x 16 x 4 multiply-adds each)
                fl = plan.packed_batches * ((N + 63) // 64) * 4 * 2 * 16 * 16 * 4
                plan_info.update(executed_mfma_tflops=fl / (ex_ms * 1e-3) / 1e12,
                                 mfma_frac=fl / (ex_ms * 1e-3) / 1e12 / FP32_MFMA_PEAK_TFLOPS)
        if stages:
            plan_info["pipeline_spmm_plus_unpermute_ms"] = stages["spmm_ms"] + stages["unpermutation_ms"]
        plan.close()

    vendor = None
    if not args.no_vendor:
        vendor = vendor_columns(Ap, Bm, B, C, ms, args.steps)
        if plan_info and "rocsparse_csr_ms" in vendor:
            plan_info["speedup_vs_rocsparse_csr"] = vendor["rocsparse_csr_ms"] / plan_info["execute_ms"]

    cpu = None
    if not args.no_cpu:
        print("[bench] cpu baseline", file=sys.stderr, flush=True)
        cpu = cpu_baseline(p, N, nnz, args.cpu_seconds)

    line = {
        "metric": METRIC,
        "value": eff,
        "unit": "TFLOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms,
        "ms_per_step_eager": ms_eager,
        "ms_per_step_graph": ms_graph,
        "timing": ("K steps launched from the Python loop" if timing == "eager" else
                   "K steps replayed from one captured HIP graph") +
                  " (HIP events on the launch stream; the faster of the two)",
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16" if sT == 2 else "f32",
        "data": "synthetic (seeded generator xspmm_amd/synth.py)",
        "config": {
            "workload": f"{args.config} ({WORKLOADS[args.config]})",
            "M": M, "K": K, "N": N, "nnz": nnz, "nnzb": nnzb,
            "index": "int32", "accumulate": "fp32",
            "clustering": bool(p.cluster),
        },
        "roofline": roofline,
        "hbm_gbs": achieved,
        "hbm_frac": achieved / HBM_PEAK_GBS,
        "padded_tflops": padded,
        # padded flops (every block x N) per second over the matrix-core peak;
        # the column-batch kernels never execute the padded flops, so this is
        # not a utilisation: mfma_busy is the counter-measured busy share
        "padded_mfma_frac": padded / mfma_peak,
        "mfma_busy": load_mfma_busy(traffic_key),
        "wall_s_timed_region": wall,
        "spot_check_rel_frob": spot,
        "prep": prep,
        "pipeline_stages_ms": stages,
        "pipeline_form": pipe_form,
        "pipeline_stages_ms_gpu_clustering": stages_gpu,
        # the same pipeline in the BCSR form (clustering on the GPU engine
        # when the workload clusters), when the default form is the packed one
        "pipeline_stages_ms_bcsr_form": stages_bcsr,
        "pipeline_warmup_calls": pipe_warmup if not args.no_pipeline else 0,
        "plan": plan_info,
        "vendor": vendor,
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
