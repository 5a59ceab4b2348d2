#pragma once
// Public SpMM API (reference: include/xspmm/xspmm.hpp:10-40).

#include <memory>

#include "xspmm/core/timings.hpp"
#include "xspmm/matrix/bcsr.hpp"
#include "xspmm/matrix/csr.hpp"

namespace xspmm {

// TIER 1: C = A * B for a 16x16 BCSR matrix A, row-major B (ld = N) and
// row-major C (ld = N).  C is overwritten; rows of block-rows with no blocks
// become zero.  Asynchronous on the executor's stream: call
// exec->synchronize() before reading C on the host.
// Instantiated for InputType in {float, __half}, OutputType float,
// IndexType in {int32_t, int64_t}.
template <typename InputType, typename OutputType, typename IndexType = int64_t>
void spmm(const BCSRMatrix<InputType, IndexType>& A,
          const InputType* B,
          OutputType* C,
          IndexType N);

// TIER 2: the automated pipeline.  With optimize_pattern: host Jaccard
// clustering (threshold 0.5, block width hw_block_size) -> GPU row
// permutation -> GPU CSR->BCSR -> Tier-1 SpMM -> GPU un-permutation of C.
// Without: GPU CSR->BCSR -> Tier-1 SpMM.  Returns after C is complete.
template <typename InputType, typename OutputType, typename IndexType = int64_t>
void spmm(std::shared_ptr<const Executor> exec,
          const CSRMatrix<InputType, IndexType>& A,
          const InputType* B,
          OutputType* C,
          IndexType N,
          IndexType hw_block_size = 16,
          bool optimize_pattern = true,
          SpMMTimings* timings = nullptr);

// out_matrix[perm[r], :] = in_matrix[r, :] for an M x N row-major matrix.
template <typename ValueType, typename IndexType>
void unpermute_dense_matrix(std::shared_ptr<const Executor> exec,
                            const ValueType* in_matrix,
                            ValueType* out_matrix,
                            const IndexType* perm,
                            IndexType M, IndexType N);

}  // namespace xspmm
