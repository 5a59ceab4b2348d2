/*
 * oracle.h -- CPU restatement of the xSpMM SpMM hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  Only tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py may load this library, and only as the checker
 * (or as the timed CPU baseline).  The product library (libxspmm.so) never
 * links, loads or calls it.
 *
 * Every function restates one piece of the reference (IlyaNyrkov/xSpMM) and
 * cites the file:line it follows.  Index arrays are int64 throughout; callers
 * widen int32 data first.  Value arrays are moved as raw bytes of `vsz` bytes
 * (2 = fp16, 4 = fp32) wherever the reference only copies them.
 *
 * Pinning status (what checks each function; see tests/test_oracle.py):
 *   xo_bcsr_count / xo_bcsr_fill  -- golden vectors from the compiled
 *       reference (oracle/_ref), dense(BCSR) == dense(CSR) bit-exact,
 *       brute-force tiny cases, duplicate/ragged/unsorted fixtures.
 *   xo_jaccard                    -- golden vectors from the compiled
 *       reference (incl. exact-tie inputs), closed forms (no join ->
 *       reversed order, identical rows -> reversed order), brute force.
 *   xo_apply_perm / xo_unpermute  -- golden vectors from the compiled
 *       reference; bijection/round-trip invariants.
 *   xo_bcsr_spmm_*                -- closed forms (checkers x ones = row
 *       sums, identity blocks), fp64 dense GEMM on the densified matrix.
 */
#ifndef XSPMM_ORACLE_H
#define XSPMM_ORACLE_H
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* CSR -> BCSR structure.  src/core/conversion.cpp:29-68.
 * Writes bcsr_row_ptr[0..Mb] and returns nnzb (number of non-empty blocks).
 * Returns -1 if a column index is outside [0, K) (the reference has UB). */
int64_t xo_bcsr_count(int64_t M, int64_t K, int64_t rb, int64_t cb,
                      const int64_t* rp, const int64_t* ci,
                      int64_t* bcsr_row_ptr);

/* CSR -> BCSR col_ind + values.  src/core/conversion.cpp:36-93.
 * bcsr_row_ptr must come from xo_bcsr_count.  bcsr_vals must hold
 * nnzb*rb*cb elements of vsz bytes. */
void xo_bcsr_fill(int64_t M, int64_t K, int64_t rb, int64_t cb,
                  const int64_t* rp, const int64_t* ci,
                  const void* vals, int vsz,
                  const int64_t* bcsr_row_ptr,
                  int64_t* bcsr_col_ind, void* bcsr_vals);

/* 1-D Jaccard ("Sylos Labini") greedy row clustering.
 * src/cpu/clustering_sylos_labini.cpp:13-116.  perm[new] = old. */
void xo_jaccard(int64_t M, int64_t K, const int64_t* rp, const int64_t* ci,
                float dist_thresh, int64_t block_width, int64_t* perm);

/* Row gather: new row i = old row perm[i].
 * src/cpu/clustering_sylos_labini.cpp:125-178 (CPU twin of
 * src/hip/mtx_permutation.hip:12-67). */
void xo_apply_perm(int64_t M, const int64_t* rp, const int64_t* ci,
                   const void* vals, int vsz, const int64_t* perm,
                   int64_t* nrp, int64_t* nci, void* nvals);

/* Dense row scatter: out[perm[r], :] = in[r, :].
 * src/common/permutation.hpp:89-108. */
void xo_unpermute(int64_t M, int64_t N, const float* in, float* out,
                  const int64_t* perm);

/* BCSR SpMM truth in fp64: C = A_bcsr * B with the tile-kernel semantics of
 * src/common/spmm_math.hpp:38-145 (overwrite; empty block-rows give zeros;
 * columns >= N masked).  A values / B given as fp32 (fp16 inputs are widened
 * exactly by the caller).  Rows >= M and B rows >= K are treated as absent. */
void xo_bcsr_spmm_f64(int64_t M, int64_t K, int64_t N, int64_t Mb,
                      const int64_t* brp, const int64_t* bci,
                      const float* bvals, const float* B, double* C);

/* Same product accumulated in fp32, one output element at a time, blocks in
 * col_ind order (the reference's accumulation order per tile).  This is the
 * CPU baseline kernel.  Input values are fp16 bit patterns when vsz == 2,
 * fp32 when vsz == 4; C is fp32.  nthreads <= 1 runs single-threaded. */
void xo_bcsr_spmm_f32(int64_t M, int64_t K, int64_t N, int64_t Mb,
                      const int64_t* brp, const int64_t* bci,
                      const void* bvals, const void* B, int vsz, float* C,
                      int nthreads);

/* fp64 CSR SpMM truth C = A_csr * B (values and B as fp32). */
void xo_csr_spmm_f64(int64_t M, int64_t N, const int64_t* rp,
                     const int64_t* ci, const float* vals, const float* B,
                     double* C);

/* Relative Frobenius error ||C - C_ref||_F / ||C_ref||_F
 * (utils/matrix_compare.hpp:23-65); fills out[4] = {max_abs, max_rel,
 * frob, rel_frob} computed in fp64. */
void xo_errors(int64_t n, const float* actual, const double* expected,
               double* out);

/* Number of host threads the OpenMP runtime would use (for reporting). */
int xo_max_threads(void);

#ifdef __cplusplus
}
#endif
#endif
