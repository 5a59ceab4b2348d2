#pragma once
// CSR -> BCSR conversion (reference: include/xspmm/matrix/conversion.hpp:19-22).
//
// On a HipExecutor the conversion runs on the GPU (block detection, compaction
// and value scatter are HIP kernels); only the block count crosses to the host
// to size the result.  On a CpuExecutor it runs on the host.  The layout is the
// reference's bit for bit: block columns ascending per block-row, row-major
// r x c blocks, zero fill, and the last of duplicate entries wins.

#include <memory>

#include "xspmm/matrix/bcsr.hpp"
#include "xspmm/matrix/csr.hpp"

namespace xspmm {

template <typename ValueType, typename IndexType = int64_t>
BCSRMatrix<ValueType, IndexType> csr_to_bcsr(std::shared_ptr<const Executor> target_exec,
                                             const CSRMatrix<ValueType, IndexType>& csr,
                                             IndexType r_block, IndexType c_block);

}  // namespace xspmm
