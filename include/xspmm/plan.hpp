#pragma once

#include <cstdint>
#include <memory>

#include "xspmm/core/executor.hpp"
#include "xspmm/core/timings.hpp"
#include "xspmm/matrix/csr.hpp"

namespace xspmm {

namespace detail {
class PlanBase;
}

// Prepared Tier-2 product.  The constructor runs the pipeline's clustering,
// permutation and CSR->BCSR stages once (the same stages, threshold and
// placement as xspmm::spmm(exec, A, ...)) and keeps their results on the
// executor's device; A is not referenced afterwards.  execute() then
// multiplies by B with the Tier-1 SpMM alone -- on the fp16 path with
// N % 8 == 0 the un-permutation is fused into the kernel's store -- and gives
// the same C as xspmm::spmm(exec, A, B, C, N, hw_block_size, optimize_pattern).
// execute() is asynchronous on the device's null stream, like the Tier-1
// entry point; calls on one plan must not overlap.
// No counterpart in the reference (its pipeline repeats every stage per call,
// src/hip/unstructured_mtx_mul.hip:31-100).  HipExecutor only.
template <typename ValueType, typename IndexType = int64_t>
class SpMMPlan {
public:
    SpMMPlan(std::shared_ptr<const Executor> exec, const CSRMatrix<ValueType, IndexType>& A,
             IndexType hw_block_size = 16, bool optimize_pattern = true,
             SpMMTimings* timings = nullptr);
    ~SpMMPlan();
    SpMMPlan(SpMMPlan&& other) noexcept;
    SpMMPlan& operator=(SpMMPlan&& other) noexcept;
    SpMMPlan(const SpMMPlan&) = delete;
    SpMMPlan& operator=(const SpMMPlan&) = delete;

    // C[M x N] = A * B[K x N]; B and C are device pointers (row-major, ld = N).
    void execute(const ValueType* B, float* C, IndexType N) const;

    IndexType get_num_blocks() const;
    bool is_clustered() const;
    // Device permutation perm[new] = old, or nullptr when not clustered.
    const IndexType* get_permutation() const;

private:
    std::shared_ptr<const Executor> exec_;
    detail::PlanBase* impl_ = nullptr;
};

}  // namespace xspmm
