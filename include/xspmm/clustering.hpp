#pragma once
// Row reordering (reference: include/xspmm/clustering.hpp:19-38).

#include <memory>

#include "xspmm/core/executor.hpp"
#include "xspmm/matrix/csr.hpp"

namespace xspmm {

// 1-D Jaccard ("Sylos Labini") greedy row clustering on the host.  Rows are
// compared through bitmaps with one bit per block_width-wide column block;
// perm_out (A.get_num_rows() entries, resident on `exec`) receives
// perm[new_row] = old_row.  The result is identical to the reference's
// src/cpu/clustering_sylos_labini.cpp for every input.
template <typename ValueType, typename IndexType = int64_t>
void compute_1d_jaccard_clustering(std::shared_ptr<const Executor> exec,
                                   const CSRMatrix<ValueType, IndexType>& A,
                                   float dist_thresh,
                                   IndexType block_width,
                                   IndexType* perm_out);

// New CSR matrix on target_exec whose row i is row perm[i] of A.
template <typename ValueType, typename IndexType = int64_t>
CSRMatrix<ValueType, IndexType> apply_permutation(std::shared_ptr<const Executor> target_exec,
                                                  const CSRMatrix<ValueType, IndexType>& A,
                                                  const IndexType* perm);

}  // namespace xspmm
