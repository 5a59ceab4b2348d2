/*
 * xspmm_capi.h -- flat C ABI of libxspmm.so (MI355X / gfx950).
 *
 * The C++ template API under include/xspmm/ is the drop-in for C++ callers.
 * These entry points expose the same operations to FFI callers (ctypes, cgo,
 * JNI, ...): plain pointers, sizes and type codes, no C++ or torch types.
 * Each one cites the reference interface it replaces.
 *
 * Conventions
 *   - vtype: XSPMM_F32 or XSPMM_F16 (value type of A and B; C is always fp32).
 *   - itype: XSPMM_I32 or XSPMM_I64 (index type of every index array).
 *   - Unless stated otherwise pointers are device pointers on the current HIP
 *     device, and `stream` is a hipStream_t (NULL = the null stream).  Work is
 *     enqueued on `stream`; functions that must read a size back (the
 *     conversion count, the pipeline) synchronize that stream.
 *   - Return value: XSPMM_OK, or an error code with a message available from
 *     xspmm_last_error() (thread-local).  Nothing throws across this ABI.
 *   - Every function rejects negative sizes and unknown type codes with
 *     XSPMM_ERR_INVALID and leaves its outputs untouched.
 */
#ifndef XSPMM_CAPI_H
#define XSPMM_CAPI_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define XSPMM_F32 0
#define XSPMM_F16 1
#define XSPMM_I32 0
#define XSPMM_I64 1

#define XSPMM_OK 0
#define XSPMM_ERR_INVALID 1     /* bad argument (std::invalid_argument in C++) */
#define XSPMM_ERR_HIP 2         /* HIP runtime error (std::runtime_error "HIP Error: ...") */
#define XSPMM_ERR_UNSUPPORTED 3 /* valid request this build does not support */
#define XSPMM_ERR_IO 4          /* file cannot be opened or parsed (MatrixMarket reader) */

/* Message of the last failed call on this thread ("" if none). */
const char* xspmm_last_error(void);

/* ABI version (bumped on any signature change). */
int xspmm_abi_version(void);

/*
 * Tier-1 BCSR SpMM: C[M x N] = A_bcsr * B[K x N], row-major, ld = N.
 * A has 16x16 blocks: brp[Mb+1], bci[nnzb], bvals[nnzb*256] (row-major
 * blocks).  M <= 16*Mb and K <= 16*Kb are the element shape; rows of C
 * beyond M are not written and B rows beyond K are not read.  C is
 * overwritten.  bvals (and B when it is fp16) must start on a 16-byte
 * boundary: the kernels read them 16 bytes at a time, and a pointer off that
 * boundary fails with XSPMM_ERR_INVALID before anything is launched (the
 * same holds for the entry points below that take them).  Asynchronous on
 * `stream`.
 * Replaces xspmm::spmm(const BCSRMatrix<In, Idx>&, const In* B, Out* C, Idx N)
 * (reference include/xspmm/xspmm.hpp:14-18, src/hip/unstructured_mtx_mul.hip:108-146).
 */
int xspmm_bcsr_spmm(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb,
                    int64_t nnzb, const void* brp, const void* bci, const void* bvals,
                    const void* B, float* C, int64_t N, void* stream);

/*
 * Tier-1 BCSR SpMM that allocates nothing: the same arguments, kernels and
 * result (bit for bit) as xspmm_bcsr_spmm, but every temporary the launch
 * needs (the dispatch order of a long block-row grid, the repacked B panels
 * of the N % 8 != 0 path) comes from a fixed device array of
 * xspmm_noalloc_scratch_bytes() bytes (8 MiB) that each GPU holds for the
 * life of the process.  No hipMalloc, hipFree or allocating library call is
 * made (the array's device address is looked up once per device, on the
 * first call there).  A product that needs more scratch than the array holds
 * (e.g. more than 2^21 block-rows on a column-batch path) is rejected
 * with XSPMM_ERR_INVALID before anything is launched.  Every call on one GPU
 * shares that GPU's array: calls that overlap on one GPU (other streams,
 * other host threads) race and must be serialized by the caller.
 * Asynchronous on `stream`.
 * No counterpart in the reference: for callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).
 */
int xspmm_bcsr_spmm_noalloc(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb,
                            int64_t nnzb, const void* brp, const void* bci, const void* bvals,
                            const void* B, float* C, int64_t N, void* stream);

/* Size in bytes of the per-GPU scratch array of xspmm_bcsr_spmm_noalloc. */
int64_t xspmm_noalloc_scratch_bytes(void);

/*
 * Dispatch order of the Tier-1 column-batch kernels (fp16 and fp32) for a
 * block-row grid: when Tier-1 would order this grid's rows (at least 256
 * block-rows), writes the Mb block-row ids (int32) to `order` and sets
 * *written = 1; otherwise writes nothing and sets *written = 0.  Above 2048
 * block-rows the longest rows come first; up to 2048 each of the 8 XCDs
 * takes a contiguous range of block-rows (workgroup i runs block-row
 * start[i % 8] + i / 8), so neighbouring rows' shared B rows stay in one
 * XCD's L2.
 * Asynchronous on `stream`.
 * No counterpart in the reference: Tier-1 computes this order on every call
 * on long grids; a caller that multiplies one matrix many times computes it
 * once (as csr_to_bcsr does for a C++ BCSRMatrix) and passes it to
 * xspmm_bcsr_spmm_ordered.
 */
int xspmm_bcsr_dispatch_order(int itype, int64_t Mb, const void* brp, int32_t* order,
                              int* written, void* stream);

/*
 * The dispatch order that csr_to_bcsr keeps on a C++ BCSRMatrix, computed
 * once per matrix from its row_ptr and col_ind (bci), into `order` (Mb + 1
 * int32; the last entry is scratch).  Above 2048 block-rows: the longest rows
 * first (as xspmm_bcsr_dispatch_order), *written = 1, asynchronous on
 * `stream`.  From 256 to 2048 block-rows, when the block-rows hold at most 128
 * blocks on average and neighbouring block-rows are alike (the middle block
 * columns of at least half of 256 sampled neighbour pairs differ by at most
 * max(2, length / 8)): each of the 8 XCDs takes a contiguous range of
 * block-rows (workgroup i runs block-row start[i % 8] + i / 8), so the B rows
 * neighbours share stay in one XCD's L2, *written = 1; otherwise *written =
 * 0 (the identity: pass no order).  This range synchronizes `stream`.  Below
 * 256 block-rows nothing is written (*written = 0).  C is the same bit for
 * bit with any order.
 * No counterpart in the reference (whose kernel takes block-rows in grid
 * order, src/common/spmm_math.hpp:20-30).
 */
int xspmm_bcsr_dispatch_order_cols(int itype, int64_t Mb, const void* brp, const void* bci,
                                   int32_t* order, int* written, void* stream);

/*
 * xspmm_bcsr_spmm with a dispatch order from xspmm_bcsr_dispatch_order
 * (NULL: Tier-1 orders the rows itself, as xspmm_bcsr_spmm does).  C is the
 * same bit for bit: the order only decides which workgroup takes which
 * block-row.  `order` holds Mb int32 entries, a permutation of [0, Mb); an
 * id outside [0, Mb) is skipped, and a block-row that no entry names is not
 * written.  Asynchronous on `stream`.
 * No counterpart in the reference (see xspmm_bcsr_dispatch_order).
 */
int xspmm_bcsr_spmm_ordered(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb,
                            int64_t nnzb, const void* brp, const void* bci, const void* bvals,
                            const void* B, float* C, int64_t N, const int32_t* order,
                            void* stream);

/*
 * Whether a grid takes a band kernel (xspmm_bcsr_spmm_band): *band = 1 when
 * every block-row is one contiguous run of block columns, the grid is not
 * full, and the band kernel's B-row gathers (32 rows per aligned pair of block
 * columns in the span of each group of four block-rows) do not exceed the
 * column-batch kernel's (one row per non-zero column of each block, estimated
 * from nnz, the CSR entries behind the grid; 0 = not known, every column
 * counted); for fp32 (vtype XSPMM_F32) also when the block-rows hold at least
 * 16 blocks on average.  Fully populated grids (the GEMM-tiled kernel's) and
 * runs with the diagnostic switch XSPMM_SPMM_KERNEL (fp16) or
 * XSPMM_F32_KERNEL (fp32) set give 0.  Reads two
 * counters back (synchronizes `stream`).  csr_to_bcsr makes this check once
 * for a C++ BCSRMatrix (BCSRMatrix::get_band_rows).
 * No counterpart in the reference (whose Tier-1 has one kernel,
 * src/common/spmm_math.hpp:20-146).
 */
int xspmm_bcsr_band_rows(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnz,
                         int64_t nnzb, const void* brp, const void* bci, int* band, void* stream);

/*
 * xspmm_bcsr_spmm with the band kernel of vtype.  fp16: four neighbouring
 * block-rows share each 32-row B tile through LDS; fp32: four neighbouring
 * block-rows share each B load in registers (v_mfma_f32_16x16x4f32).  Only
 * correct when every block-row is one contiguous run of block columns
 * (xspmm_bcsr_band_rows checks; on other grids the kernels stay inside A, B
 * and C but C is wrong).  Shapes a band kernel does not cover (fp16: N % 8 !=
 * 0; fp32: N % 4 != 0 or B / C off a 16-byte boundary; K * N * value bytes >
 * 2^31) run the column-batch kernel instead.  fp32 grids of at most 4096
 * groups of four block-rows take a balanced launch where one group per
 * workgroup is predicted to leave CUs idle long enough to pay for its fixed
 * cost (about 25 us; wide bands, and grids of fewer workgroups than the CUs
 * hold): a plan kernel gives every workgroup an equal share of the groups'
 * blocks, and a group cut between shares is summed from its parts in a fixed
 * order (stream-ordered scratch, C the same on every call;
 * XSPMM_BAND_SPLIT=off keeps one group per workgroup, =force takes the
 * balanced launch wherever it can run).  Every block a
 * row holds multiplies all 16 of its columns, so an Inf/NaN in B gives NaN in
 * the rows the reference's does.  Asynchronous on `stream`.
 * Replaces, for banded grids, the same call as xspmm_bcsr_spmm
 * (reference src/hip/unstructured_mtx_mul.hip:108-146).
 */
int xspmm_bcsr_spmm_band(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb,
                         const void* brp, const void* bci, const void* bvals, const void* B, float* C,
                         int64_t N, void* stream);

/*
 * CSR -> BCSR, phase 1: writes bcsr_row_ptr[Mb+1] (device) for r x c blocks,
 * Mb = ceil(M/r), and stores nnzb in *nnzb_out (host).  Synchronizes `stream`.
 * Fails with XSPMM_ERR_INVALID if a column index lies outside [0, K).
 * Phase 2 fills bcsr_col_ind[nnzb] and bcsr_vals[nnzb*r*c] (device).
 * Replaces xspmm::csr_to_bcsr (reference include/xspmm/matrix/conversion.hpp:19-22,
 * src/core/conversion.cpp:8-100).
 */
int xspmm_csr_to_bcsr_count(int itype, int64_t M, int64_t K, int64_t nnz, const void* rp,
                            const void* ci, int64_t r_block, int64_t c_block,
                            void* bcsr_row_ptr, int64_t* nnzb_out, void* stream);
int xspmm_csr_to_bcsr_fill(int vtype, int itype, int64_t M, int64_t K, int64_t nnz,
                           const void* rp, const void* ci, const void* vals,
                           int64_t r_block, int64_t c_block, const void* bcsr_row_ptr,
                           void* bcsr_col_ind, void* bcsr_vals, void* stream);

/*
 * Row permutation of a CSR matrix: new row i = old row perm[i].
 * new_rp[M+1], new_ci[nnz], new_vals[nnz] are caller-allocated (device).
 * perm must be a permutation of [0, M).  Asynchronous on `stream`.
 * Replaces xspmm::apply_permutation (reference include/xspmm/clustering.hpp:34-38,
 * src/hip/mtx_permutation.hip:12-67).
 */
int xspmm_apply_permutation(int vtype, int itype, int64_t M, int64_t nnz, const void* rp,
                            const void* ci, const void* vals, const void* perm,
                            void* new_rp, void* new_ci, void* new_vals, void* stream);

/*
 * Dense row scatter out[perm[r], :] = in[r, :] of an M x N fp32 matrix.
 * Asynchronous on `stream`.
 * Replaces xspmm::unpermute_dense_matrix (reference include/xspmm/xspmm.hpp:35-40,
 * src/hip/mtx_permutation.hip:73-95).
 */
int xspmm_unpermute_dense(int itype, const float* in, float* out, const void* perm,
                          int64_t M, int64_t N, void* stream);

/*
 * Host Jaccard row clustering on HOST arrays rp[M+1], ci[nnz]; writes
 * perm_out[M] (host).  Identical result to the reference's
 * src/cpu/clustering_sylos_labini.cpp:51-120.  nthreads <= 0 picks the
 * number of online CPUs.
 * Replaces xspmm::compute_1d_jaccard_clustering (reference include/xspmm/clustering.hpp:19-25).
 */
int xspmm_jaccard_clustering_host(int itype, int64_t M, int64_t K, const void* rp,
                                  const void* ci, float dist_thresh, int64_t block_width,
                                  void* perm_out, int nthreads);

/*
 * GPU Jaccard row clustering on DEVICE arrays rp[M+1], ci[nnz]; writes the
 * device array perm_out[M].  The same permutation as
 * xspmm_jaccard_clustering_host (the reference's greedy,
 * src/cpu/clustering_sylos_labini.cpp:51-120), computed by one workgroup that
 * commits joins in the reference's visiting order.  engine_used (nullable,
 * host) receives 0 (closed form: dist_thresh outside [0, 1)), 1 (scan engine)
 * or 2 (row-list engine).  Synchronizes `stream`.  Limits: M < 2^30, at most
 * 524288 column blocks, M * ceil(blocks / 64) * 8 bytes of row bitmaps
 * within 16 GiB; beyond them it returns XSPMM_ERR_INVALID.
 * Replaces xspmm::compute_1d_jaccard_clustering for device matrices
 * (reference include/xspmm/clustering.hpp:19-25, src/xspmm.cpp:57-67).
 */
int xspmm_jaccard_clustering(int itype, int64_t M, int64_t K, int64_t nnz, const void* rp,
                             const void* ci, float dist_thresh, int64_t block_width,
                             void* perm_out, int* engine_used, void* stream);

/*
 * Tier-2 pipeline on device CSR arrays rp/ci/vals, device B and C.
 * hw_block_size must be 16.  With optimize_pattern != 0: cluster (host
 * greedy; the GPU engine when the environment sets XSPMM_CLUSTER_DEVICE=gpu) ->
 * permute -> convert -> SpMM -> unpermute; else convert -> SpMM.  timings
 * (nullable, host) receives the six SpMMTimings fields in declaration order:
 * clustering, permutation, conversion, spmm, unpermutation, total (ms);
 * fields of stages that do not run are left unchanged.  Returns after C is
 * complete.
 * Replaces xspmm::spmm(exec, const CSRMatrix&, B, C, N, hw_block_size,
 * optimize_pattern, SpMMTimings*) (reference include/xspmm/xspmm.hpp:24-32,
 * src/hip/unstructured_mtx_mul.hip:31-100).
 */
int xspmm_spmm_pipeline(int vtype, int itype, int64_t M, int64_t K, int64_t nnz,
                        const void* rp, const void* ci, const void* vals, const void* B,
                        float* C, int64_t N, int64_t hw_block_size, int optimize_pattern,
                        double* timings, void* stream);

/*
 * Device bytes of the temporaries that the last xspmm_spmm_pipeline call on
 * the calling thread held at once from the device's memory pool (0 before
 * any call): the permuted CSR, the permuted-order C and the BCSR arrays, or
 * for the packed form (xspmm_pipeline_last_form) the column batches.  The
 * BCSR arrays are sized from the bound min(nnz, Mb * Kb) on the block count
 * while that bound's block values fit 1 GiB, else exactly after the block
 * count is read; the batches from the bound min(2 nnz / 33 + min(4 Mb, nnz),
 * Mb * ceil(Kb / 2)) at 1152 bytes each, likewise.
 * No counterpart in the reference (whose pipeline makes a hipMalloc per
 * temporary, src/hip/unstructured_mtx_mul.hip:31-100); it lets a caller see
 * the pipeline's memory footprint.
 */
int xspmm_pipeline_temp_bytes(int64_t* bytes_out);

/*
 * Sets *packed_out to 1 when the last xspmm_spmm_pipeline call on the calling
 * thread converted A into packed column batches and multiplied those (fp16,
 * N % 8 == 0, K <= 167296, strictly increasing columns per row, finite
 * values, and batches that save at least a quarter of the block bytes), to 0
 * when it took the BCSR blocks.  C is the same bit for bit either way.
 * No counterpart in the reference, whose pipeline always converts to BCSR
 * (src/hip/unstructured_mtx_mul.hip:58-61, :86-89); it lets a caller see
 * which form ran.
 */
int xspmm_pipeline_last_form(int* packed_out);

/*
 * Prepared Tier-2 product ("plan"): the pipeline's clustering, permutation
 * and CSR->BCSR stages run once at creation, on device CSR arrays rp/ci/vals
 * (hw_block_size must be 16; clustering as in xspmm_spmm_pipeline); the plan
 * keeps the permutation, the BCSR matrix and the SpMM dispatch order on the
 * device and does not reference rp/ci/vals afterwards.  timings (nullable,
 * host) receives the clustering, permutation, conversion and total fields
 * of SpMMTimings (declaration order, six doubles); the spmm and
 * unpermutation fields are left unchanged.  Synchronizes `stream`.
 * No counterpart in the reference, whose pipeline repeats every stage per
 * call (src/hip/unstructured_mtx_mul.hip:31-100); for callers that multiply
 * the same matrix many times.
 */
typedef struct xspmm_plan_s* xspmm_plan_t;
int xspmm_plan_create(int vtype, int itype, int64_t M, int64_t K, int64_t nnz, const void* rp,
                      const void* ci, const void* vals, int64_t hw_block_size,
                      int optimize_pattern, double* timings, void* stream, xspmm_plan_t* plan_out);

/*
 * C[M x N] (fp32, device) = A * B[K x N] (device, the plan's value type) with
 * the plan's A, in the original row order: identical to xspmm_spmm_pipeline's
 * C.  Asynchronous on `stream`.  On the fp16 path with N % 8 == 0 it is one
 * kernel launch with the un-permutation fused into the store, which streams
 * the plan's packed column batches when it has them; otherwise it uses a
 * device workspace kept by the plan (grown, with a synchronization, when N
 * exceeds every earlier N).  Calls on one plan must not overlap.
 */
int xspmm_plan_execute(xspmm_plan_t plan, const void* B, float* C, int64_t N, void* stream);

/* Block count, block-row count, whether the rows were clustered and the
 * device permutation perm[new] = old (NULL when not clustered).  Any output
 * pointer may be NULL. */
int xspmm_plan_info(xspmm_plan_t plan, int64_t* num_blocks, int64_t* num_block_rows,
                    int* clustered, const void** perm);

/* Number of packed column batches the plan multiplies from (fp16 plans of
 * sparse blocks keep the SpMM kernel's batches -- A' operands and B-row
 * indices -- instead of streaming the BCSR blocks), or -1 when the plan
 * multiplies the BCSR matrix itself. */
int xspmm_plan_packed_batches(xspmm_plan_t plan, int64_t* batches);

/* Frees the plan's device memory (NULL is accepted). */
int xspmm_plan_destroy(xspmm_plan_t plan);

/*
 * MatrixMarket coordinate file -> host CSR, the same matrix as the
 * reference's reader (utils/matrix_io.hpp:27-98, matrix_utils::io::read_mtx):
 * comment/empty lines skipped, 1-based entries outside the matrix dropped,
 * missing or unreadable values read as 1.0, no symmetric expansion, entries
 * sorted by (row, column) with duplicates kept in file order.
 * xspmm_mtx_read parses the file once into a handle (XSPMM_ERR_IO with the
 * reference's message when it cannot be opened or has no readable dimension
 * line); xspmm_mtx_info gives rows, cols and the number of entries kept;
 * xspmm_mtx_export writes HOST arrays row_ptr[rows+1], col_ind[nnz] (index
 * type code) and values[nnz] (value type code; fp16 rounded to nearest even
 * from the float read); xspmm_mtx_free releases the handle (NULL accepted).
 */
typedef struct xspmm_mtx_s* xspmm_mtx_t;
int xspmm_mtx_read(const char* path, xspmm_mtx_t* out);
int xspmm_mtx_info(xspmm_mtx_t m, int64_t* rows, int64_t* cols, int64_t* nnz);
int xspmm_mtx_export(xspmm_mtx_t m, int itype, int vtype, void* row_ptr, void* col_ind,
                     void* values);
int xspmm_mtx_free(xspmm_mtx_t m);

#ifdef __cplusplus
}
#endif

#endif /* XSPMM_CAPI_H */
