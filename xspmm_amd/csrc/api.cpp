// api.cpp -- the public C++ API (include/xspmm/*.hpp): executor dispatch and
// explicit instantiations (reference src/xspmm.cpp, src/core/conversion.cpp).
//
// Dispatch follows the reference: the executor's dynamic type picks the
// backend.  HipExecutor runs the HIP kernels of this library on the null
// stream of its device.  CpuExecutor keeps the reference's CPU coverage:
// conversion, clustering and permutation run on the host, while SpMM, the
// pipeline and un-permutation throw the reference's messages
// (src/xspmm.cpp:51, :133, :161).
//
// Instantiated for ValueType/InputType in {float, __half} and IndexType in
// {int32_t, int64_t}; OutputType is float.
#include <hip/hip_fp16.h>

#include <algorithm>
#include <type_traits>
#include <vector>

#include "internal.hpp"
#include "xspmm/clustering.hpp"
#include "xspmm/matrix/conversion.hpp"
#include "xspmm/plan.hpp"
#include "xspmm/xspmm.hpp"

namespace xspmm {

namespace {

template <typename T>
struct DevType { using type = T; };
template <>
struct DevType<__half> { using type = uint16_t; };
template <typename T>
using dev_t = typename DevType<T>::type;

template <typename T>
const dev_t<T>* dev(const T* p) { return reinterpret_cast<const dev_t<T>*>(p); }
template <typename T>
dev_t<T>* dev(T* p) { return reinterpret_cast<dev_t<T>*>(p); }

const HipExecutor* as_hip(const std::shared_ptr<const Executor>& e)
{
    return dynamic_cast<const HipExecutor*>(e.get());
}
const CpuExecutor* as_cpu(const std::shared_ptr<const Executor>& e)
{
    return dynamic_cast<const CpuExecutor*>(e.get());
}

// Makes the executor's device current for the calling thread.
void use_device(const HipExecutor* h) { XSPMM_HIP_CHECK(hipSetDevice(h->get_device_id())); }

constexpr hipStream_t kStream = nullptr;  // the null stream, as in the reference

// Device copies of a CSR matrix that lives on a CPU executor.
template <typename T, typename I>
struct DeviceCsr {
    detail::Scratch rp, ci, vals;
    const I* d_rp = nullptr;
    const I* d_ci = nullptr;
    const T* d_vals = nullptr;
};

template <typename T, typename I>
void device_view(const CSRMatrix<T, I>& A, DeviceCsr<T, I>& v)
{
    const int64_t M = A.get_num_rows(), nnz = A.get_nnz();
    if (as_hip(A.get_executor())) {
        v.d_rp = A.get_row_ptr();
        v.d_ci = A.get_col_ind();
        v.d_vals = A.get_values();
        return;
    }
    std::vector<I> rp((size_t)M + 1), ci((size_t)nnz);
    std::vector<T> vals((size_t)nnz);
    A.get_executor()->copy_to_host(rp.data(), A.get_row_ptr(), sizeof(I) * (size_t)(M + 1));
    if (nnz > 0) {
        A.get_executor()->copy_to_host(ci.data(), A.get_col_ind(), sizeof(I) * (size_t)nnz);
        A.get_executor()->copy_to_host(vals.data(), A.get_values(), sizeof(T) * (size_t)nnz);
    }
    v.rp = detail::Scratch(sizeof(I) * (size_t)(M + 1), kStream);
    v.ci = detail::Scratch(sizeof(I) * (size_t)(nnz > 0 ? nnz : 1), kStream);
    v.vals = detail::Scratch(sizeof(T) * (size_t)(nnz > 0 ? nnz : 1), kStream);
    XSPMM_HIP_CHECK(hipMemcpy(v.rp.get(), rp.data(), sizeof(I) * (size_t)(M + 1), hipMemcpyHostToDevice));
    if (nnz > 0) {
        XSPMM_HIP_CHECK(hipMemcpy(v.ci.get(), ci.data(), sizeof(I) * (size_t)nnz, hipMemcpyHostToDevice));
        XSPMM_HIP_CHECK(hipMemcpy(v.vals.get(), vals.data(), sizeof(T) * (size_t)nnz, hipMemcpyHostToDevice));
    }
    v.d_rp = v.rp.template as<I>();
    v.d_ci = v.ci.template as<I>();
    v.d_vals = v.vals.template as<T>();
}

// Host CSR arrays of a matrix on any executor.
template <typename T, typename I>
void host_csr(const CSRMatrix<T, I>& A, std::vector<I>& rp, std::vector<I>& ci, std::vector<T>* vals)
{
    const int64_t M = A.get_num_rows(), nnz = A.get_nnz();
    rp.resize((size_t)M + 1);
    ci.resize((size_t)nnz);
    A.get_executor()->copy_to_host(rp.data(), A.get_row_ptr(), sizeof(I) * (size_t)(M + 1));
    if (nnz > 0) A.get_executor()->copy_to_host(ci.data(), A.get_col_ind(), sizeof(I) * (size_t)nnz);
    if (vals) {
        vals->resize((size_t)nnz);
        if (nnz > 0)
            A.get_executor()->copy_to_host(vals->data(), A.get_values(), sizeof(T) * (size_t)nnz);
    }
}

// Host CSR -> BCSR for CpuExecutor targets (the algorithm of the reference's
// src/core/conversion.cpp:8-100).
template <typename T, typename I>
BCSRMatrix<T, I> host_csr_to_bcsr(std::shared_ptr<const Executor> target, const CSRMatrix<T, I>& csr,
                                  I rb, I cb)
{
    if (rb <= 0 || cb <= 0) throw std::invalid_argument("csr_to_bcsr: block sizes must be positive.");
    const int64_t M = csr.get_num_rows(), K = csr.get_num_cols();
    std::vector<I> rp, ci;
    std::vector<T> vals;
    host_csr(csr, rp, ci, &vals);
    const int64_t Mb = (M + rb - 1) / rb, Kb = (K + cb - 1) / cb, bsz = (int64_t)rb * cb;
    std::vector<I> brp(1, 0), bci;
    std::vector<T> bv;
    std::vector<int64_t> last((size_t)Kb, -1), rank((size_t)Kb, 0);
    for (int64_t br = 0; br < Mb; ++br) {
        const int64_t r0 = br * rb, r1 = std::min<int64_t>(M, r0 + rb);
        const size_t first = bci.size();
        for (int64_t r = r0; r < r1; ++r)
            for (int64_t k = rp[(size_t)r]; k < (int64_t)rp[(size_t)r + 1]; ++k) {
                const int64_t c = ci[(size_t)k];
                if (c < 0 || c >= K) throw std::invalid_argument("csr_to_bcsr: column index out of range.");
                if (last[(size_t)(c / cb)] != br) {
                    last[(size_t)(c / cb)] = br;
                    bci.push_back((I)(c / cb));
                }
            }
        std::sort(bci.begin() + (std::ptrdiff_t)first, bci.end());
        for (size_t j = first; j < bci.size(); ++j) rank[(size_t)bci[j]] = (int64_t)(j - first);
        brp.push_back((I)bci.size());
        const size_t vbase = first * (size_t)bsz;
        bv.resize(bci.size() * (size_t)bsz, T(0.0f));
        for (int64_t r = r0; r < r1; ++r)
            for (int64_t k = rp[(size_t)r]; k < (int64_t)rp[(size_t)r + 1]; ++k) {
                const int64_t c = ci[(size_t)k];
                bv[vbase + (size_t)(rank[(size_t)(c / cb)] * bsz + (r % rb) * cb + c % cb)] = vals[(size_t)k];
            }
    }
    BCSRMatrix<T, I> out(target, (I)Mb, (I)Kb, (I)bci.size(), rb, cb);
    out.copy_from_host(brp.data(), bci.data(), bv.data());
    out.set_shape((I)M, (I)K);
    return out;
}

}  // namespace

// ---------------------------------------------------------------------------
// Tier 1
// ---------------------------------------------------------------------------
template <typename InputType, typename OutputType, typename IndexType>
void spmm(const BCSRMatrix<InputType, IndexType>& A, const InputType* B, OutputType* C, IndexType N)
{
    static_assert(std::is_same<OutputType, float>::value, "xSpMM: OutputType must be float.");
    auto exec = A.get_executor();
    if (const HipExecutor* h = as_hip(exec)) {
        if (A.get_r_block() != 16 || A.get_c_block() != 16)
            throw std::invalid_argument("xSpMM: the MFMA tile kernel requires 16x16 blocks.");
        use_device(h);
        if (A.get_band_rows()) {
            detail::bcsr_spmm_band<dev_t<InputType>, IndexType>(
                A.get_num_rows(), A.get_num_cols(), A.get_num_block_rows(), A.get_num_block_cols(),
                A.get_num_blocks(), A.get_bcsr_row_ptr(), A.get_bcsr_col_ind(), dev(A.get_bcsr_values()),
                dev(B), C, N, kStream);
            return;
        }
        (void)detail::bcsr_spmm_ex<dev_t<InputType>, IndexType>(
            A.get_num_rows(), A.get_num_cols(), A.get_num_block_rows(), A.get_num_block_cols(),
            A.get_num_blocks(), A.get_bcsr_row_ptr(), A.get_bcsr_col_ind(), dev(A.get_bcsr_values()),
            dev(B), C, N, A.get_dispatch_order(), nullptr, kStream);
        return;
    }
    throw std::runtime_error("xSpMM: CPU SpMM fallback is not yet implemented. Please use a GPU Executor.");
}

// ---------------------------------------------------------------------------
// Clustering: the host greedy for every executor, as in the reference; a
// HipExecutor can run the GPU engine instead (XSPMM_CLUSTER_DEVICE=gpu)
// ---------------------------------------------------------------------------
template <typename ValueType, typename IndexType>
void compute_1d_jaccard_clustering(std::shared_ptr<const Executor> exec,
                                   const CSRMatrix<ValueType, IndexType>& A, float dist_thresh,
                                   IndexType block_width, IndexType* perm_out)
{
    const int64_t M = A.get_num_rows();
    if (M == 0) return;
    if (const HipExecutor* h = as_hip(exec)) {
        // perm_out lives on the executor's device: host greedy on copies,
        // or the GPU engine with XSPMM_CLUSTER_DEVICE=gpu (same permutation)
        use_device(h);
        DeviceCsr<ValueType, IndexType> v;
        device_view(A, v);
        detail::jaccard_clustering_dispatch<IndexType>(M, A.get_num_cols(), A.get_nnz(), v.d_rp, v.d_ci,
                                                       dist_thresh, block_width, perm_out, kStream);
        return;
    }
    std::vector<IndexType> rp, ci, perm((size_t)M);
    host_csr<ValueType, IndexType>(A, rp, ci, nullptr);
    detail::jaccard_clustering_host<IndexType>(M, A.get_num_cols(), rp.data(), ci.data(), dist_thresh,
                                               block_width, perm.data(), 0);
    exec->copy_from_host(perm_out, perm.data(), sizeof(IndexType) * (size_t)M);
}

// ---------------------------------------------------------------------------
// Permutation
// ---------------------------------------------------------------------------
template <typename ValueType, typename IndexType>
CSRMatrix<ValueType, IndexType> apply_permutation(std::shared_ptr<const Executor> target_exec,
                                                  const CSRMatrix<ValueType, IndexType>& A,
                                                  const IndexType* perm)
{
    const IndexType M = A.get_num_rows(), K = A.get_num_cols(), nnz = A.get_nnz();
    if (const HipExecutor* h = as_hip(target_exec)) {
        use_device(h);
        if (M == 0) return CSRMatrix<ValueType, IndexType>(target_exec, 0, 0, 0);  // mtx_permutation.hip:22
        DeviceCsr<ValueType, IndexType> src;
        device_view(A, src);
        CSRMatrix<ValueType, IndexType> out(target_exec, M, K, nnz);
        detail::apply_permutation<dev_t<ValueType>, IndexType>(
            M, nnz, src.d_rp, src.d_ci, dev(src.d_vals), perm, out.get_row_ptr(), out.get_col_ind(),
            dev(out.get_values()), kStream);
        return out;
    }
    if (as_cpu(target_exec)) {
        // clustering_sylos_labini.cpp:125-178
        std::vector<IndexType> rp, ci, hperm((size_t)M);
        std::vector<ValueType> vals;
        host_csr(A, rp, ci, &vals);
        if (M > 0) target_exec->copy_to_host(hperm.data(), perm, sizeof(IndexType) * (size_t)M);
        std::vector<IndexType> nrp(1, 0), nci;
        std::vector<ValueType> nv;
        nci.reserve((size_t)nnz);
        nv.reserve((size_t)nnz);
        for (IndexType i = 0; i < M; ++i) {
            const IndexType o = hperm[(size_t)i];
            if (o < 0 || o >= M) throw std::invalid_argument("apply_permutation: perm entry out of range.");
            for (IndexType j = rp[(size_t)o]; j < rp[(size_t)o + 1]; ++j) {
                nci.push_back(ci[(size_t)j]);
                nv.push_back(vals[(size_t)j]);
            }
            nrp.push_back((IndexType)nci.size());
        }
        if ((IndexType)nci.size() != nnz)
            throw std::invalid_argument("apply_permutation: perm is not a permutation.");
        CSRMatrix<ValueType, IndexType> out(target_exec, M, K, nnz);
        out.copy_from_host(nrp.data(), nci.data(), nv.data());
        return out;
    }
    throw std::runtime_error("xSpMM: Unsupported Executor type in apply_permutation.");
}

// ---------------------------------------------------------------------------
// Conversion
// ---------------------------------------------------------------------------
template <typename ValueType, typename IndexType>
BCSRMatrix<ValueType, IndexType> csr_to_bcsr(std::shared_ptr<const Executor> target_exec,
                                             const CSRMatrix<ValueType, IndexType>& csr,
                                             IndexType r_block, IndexType c_block)
{
    const HipExecutor* th = as_hip(target_exec);
    const HipExecutor* sh = as_hip(csr.get_executor());
    if (!th && !sh) return host_csr_to_bcsr(target_exec, csr, r_block, c_block);
    use_device(th ? th : sh);

    const int64_t M = csr.get_num_rows(), K = csr.get_num_cols(), nnz = csr.get_nnz();
    if (r_block <= 0 || c_block <= 0)
        throw std::invalid_argument("csr_to_bcsr: block sizes must be positive.");
    const int64_t Mb = (M + r_block - 1) / r_block, Kb = (K + c_block - 1) / c_block;
    DeviceCsr<ValueType, IndexType> src;
    device_view(csr, src);
    detail::Scratch brp((size_t)(Mb + 1) * sizeof(IndexType), kStream);
    const int64_t nnzb = detail::csr_to_bcsr_count<IndexType>(M, K, nnz, src.d_rp, src.d_ci, r_block,
                                                             c_block, brp.as<IndexType>(), kStream);
    const size_t nvals = (size_t)nnzb * (size_t)r_block * (size_t)c_block;
    BCSRMatrix<ValueType, IndexType> out(target_exec, (IndexType)Mb, (IndexType)Kb, (IndexType)nnzb,
                                         r_block, c_block);
    out.set_shape((IndexType)M, (IndexType)K);
    if (th) {
        XSPMM_HIP_CHECK(hipMemcpyAsync(out.get_bcsr_row_ptr(), brp.get(), sizeof(IndexType) * (size_t)(Mb + 1),
                                       hipMemcpyDeviceToDevice, kStream));
        detail::csr_to_bcsr_fill<dev_t<ValueType>, IndexType>(
            M, K, nnz, src.d_rp, src.d_ci, dev(src.d_vals), r_block, c_block, brp.as<IndexType>(),
            out.get_bcsr_col_ind(), dev(out.get_bcsr_values()), kStream);
        // the column-batch kernels' dispatch order, once (see BCSRMatrix);
        // owned by `out` from the allocation on, so a failed launch frees it
        if (r_block == 16 && c_block == 16 && detail::spmm_order_cols_wanted(Mb)) {
            int32_t* order = nullptr;
            target_exec->allocate(reinterpret_cast<void**>(&order), (size_t)(Mb + 1) * sizeof(int32_t));
            out.set_dispatch_order(order);
            if (!detail::spmm_dispatch_order_cols<IndexType>(out.get_bcsr_row_ptr(), out.get_bcsr_col_ind(),
                                                             Mb, order, kStream))
                out.set_dispatch_order(nullptr);  // the identity: not worth a load per workgroup
        }
        // grids of contiguous, overlapping block-rows: the band kernels
        if (r_block == 16 && c_block == 16)
            out.set_band_rows(detail::spmm_band_wanted<IndexType>(out.get_bcsr_row_ptr(), out.get_bcsr_col_ind(),
                                                                  M, K, Mb, Kb, nnz, nnzb, 0,
                                                                  (int)sizeof(ValueType), kStream));
    } else {
        // GPU-resident input, host target: convert on the GPU, then copy down.
        detail::Scratch bci((size_t)(nnzb > 0 ? nnzb : 1) * sizeof(IndexType), kStream);
        detail::Scratch bv((nvals > 0 ? nvals : 1) * sizeof(ValueType), kStream);
        detail::csr_to_bcsr_fill<dev_t<ValueType>, IndexType>(
            M, K, nnz, src.d_rp, src.d_ci, dev(src.d_vals), r_block, c_block, brp.as<IndexType>(),
            bci.as<IndexType>(), bv.as<dev_t<ValueType>>(), kStream);
        XSPMM_HIP_CHECK(hipStreamSynchronize(kStream));
        XSPMM_HIP_CHECK(hipMemcpy(out.get_bcsr_row_ptr(), brp.get(), sizeof(IndexType) * (size_t)(Mb + 1),
                                  hipMemcpyDeviceToHost));
        if (nnzb > 0) {
            XSPMM_HIP_CHECK(hipMemcpy(out.get_bcsr_col_ind(), bci.get(), sizeof(IndexType) * (size_t)nnzb,
                                      hipMemcpyDeviceToHost));
            XSPMM_HIP_CHECK(hipMemcpy(out.get_bcsr_values(), bv.get(), sizeof(ValueType) * nvals,
                                      hipMemcpyDeviceToHost));
        }
    }
    return out;
}

// ---------------------------------------------------------------------------
// Un-permutation
// ---------------------------------------------------------------------------
template <typename ValueType, typename IndexType>
void unpermute_dense_matrix(std::shared_ptr<const Executor> exec, const ValueType* in_matrix,
                            ValueType* out_matrix, const IndexType* perm, IndexType M, IndexType N)
{
    static_assert(std::is_same<ValueType, float>::value, "xSpMM: unpermute is instantiated for float.");
    if (const HipExecutor* h = as_hip(exec)) {
        use_device(h);
        detail::unpermute_dense<IndexType>(in_matrix, out_matrix, perm, M, N, kStream);
        return;
    }
    throw std::runtime_error("CPU unpermute not yet implemented in pipeline.");
}

// ---------------------------------------------------------------------------
// Tier 2
// ---------------------------------------------------------------------------
template <typename InputType, typename OutputType, typename IndexType>
void spmm(std::shared_ptr<const Executor> exec, const CSRMatrix<InputType, IndexType>& A,
          const InputType* B, OutputType* C, IndexType N, IndexType hw_block_size,
          bool optimize_pattern, SpMMTimings* timings)
{
    static_assert(std::is_same<OutputType, float>::value, "xSpMM: OutputType must be float.");
    static_assert(sizeof(SpMMTimings) == 6 * sizeof(double), "SpMMTimings layout");
    if (const HipExecutor* h = as_hip(exec)) {
        use_device(h);
        DeviceCsr<InputType, IndexType> src;
        device_view(A, src);
        detail::spmm_pipeline<dev_t<InputType>, IndexType>(
            A.get_num_rows(), A.get_num_cols(), A.get_nnz(), src.d_rp, src.d_ci, dev(src.d_vals),
            dev(B), C, N, hw_block_size, optimize_pattern,
            timings ? reinterpret_cast<double*>(timings) : nullptr, kStream);
        return;
    }
    throw std::runtime_error("xSpMM: CPU pipeline fallback is not yet implemented.");
}

// ---------------------------------------------------------------------------
// Prepared Tier-2 product
// ---------------------------------------------------------------------------
template <typename ValueType, typename IndexType>
SpMMPlan<ValueType, IndexType>::SpMMPlan(std::shared_ptr<const Executor> exec,
                                         const CSRMatrix<ValueType, IndexType>& A,
                                         IndexType hw_block_size, bool optimize_pattern,
                                         SpMMTimings* timings)
    : exec_(std::move(exec))
{
    const HipExecutor* h = as_hip(exec_);
    if (!h) throw std::runtime_error("xSpMM: CPU pipeline fallback is not yet implemented.");
    use_device(h);
    DeviceCsr<ValueType, IndexType> src;
    device_view(A, src);
    impl_ = detail::make_plan<dev_t<ValueType>, IndexType>(
        A.get_num_rows(), A.get_num_cols(), A.get_nnz(), src.d_rp, src.d_ci, dev(src.d_vals),
        hw_block_size, optimize_pattern, timings ? reinterpret_cast<double*>(timings) : nullptr,
        kStream);
}

template <typename ValueType, typename IndexType>
SpMMPlan<ValueType, IndexType>::~SpMMPlan()
{
    if (impl_) {
        if (const HipExecutor* h = as_hip(exec_)) (void)hipSetDevice(h->get_device_id());
        delete impl_;
    }
}

template <typename ValueType, typename IndexType>
SpMMPlan<ValueType, IndexType>::SpMMPlan(SpMMPlan&& o) noexcept : exec_(std::move(o.exec_)), impl_(o.impl_)
{
    o.impl_ = nullptr;
}

template <typename ValueType, typename IndexType>
SpMMPlan<ValueType, IndexType>& SpMMPlan<ValueType, IndexType>::operator=(SpMMPlan&& o) noexcept
{
    if (this != &o) {
        delete impl_;
        exec_ = std::move(o.exec_);
        impl_ = o.impl_;
        o.impl_ = nullptr;
    }
    return *this;
}

template <typename ValueType, typename IndexType>
void SpMMPlan<ValueType, IndexType>::execute(const ValueType* B, float* C, IndexType N) const
{
    if (!impl_) throw std::runtime_error("xSpMM: empty (moved-from) plan.");
    use_device(as_hip(exec_));
    impl_->execute(dev(B), C, (int64_t)N, kStream);
}

template <typename ValueType, typename IndexType>
IndexType SpMMPlan<ValueType, IndexType>::get_num_blocks() const
{
    return impl_ ? (IndexType)impl_->num_blocks() : 0;
}

template <typename ValueType, typename IndexType>
bool SpMMPlan<ValueType, IndexType>::is_clustered() const
{
    return impl_ && impl_->clustered();
}

template <typename ValueType, typename IndexType>
const IndexType* SpMMPlan<ValueType, IndexType>::get_permutation() const
{
    return impl_ ? static_cast<const IndexType*>(impl_->permutation()) : nullptr;
}

// ---------------------------------------------------------------------------
// Explicit instantiations
// ---------------------------------------------------------------------------
#define XSPMM_INSTANTIATE(T, I)                                                                       \
    template void spmm<T, float, I>(const BCSRMatrix<T, I>&, const T*, float*, I);                   \
    template void spmm<T, float, I>(std::shared_ptr<const Executor>, const CSRMatrix<T, I>&,         \
                                    const T*, float*, I, I, bool, SpMMTimings*);                     \
    template void compute_1d_jaccard_clustering<T, I>(std::shared_ptr<const Executor>,              \
                                                      const CSRMatrix<T, I>&, float, I, I*);         \
    template CSRMatrix<T, I> apply_permutation<T, I>(std::shared_ptr<const Executor>,               \
                                                     const CSRMatrix<T, I>&, const I*);              \
    template BCSRMatrix<T, I> csr_to_bcsr<T, I>(std::shared_ptr<const Executor>,                    \
                                                const CSRMatrix<T, I>&, I, I);                       \
    template class SpMMPlan<T, I>;
XSPMM_INSTANTIATE(float, int32_t)
XSPMM_INSTANTIATE(float, int64_t)
XSPMM_INSTANTIATE(__half, int32_t)
XSPMM_INSTANTIATE(__half, int64_t)
#undef XSPMM_INSTANTIATE

template void unpermute_dense_matrix<float, int32_t>(std::shared_ptr<const Executor>, const float*,
                                                     float*, const int32_t*, int32_t, int32_t);
template void unpermute_dense_matrix<float, int64_t>(std::shared_ptr<const Executor>, const float*,
                                                     float*, const int64_t*, int64_t, int64_t);

}  // namespace xspmm
