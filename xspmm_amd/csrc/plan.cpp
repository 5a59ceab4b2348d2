// plan.cpp -- prepared Tier-2 products (plan and workspace reuse).
//
// The Tier-2 pipeline (reference src/hip/unstructured_mtx_mul.hip:31-100,
// here spmm_pipeline) clusters, permutes and converts A on every call.  A
// plan runs those stages once, with the pipeline's stage order, threshold
// (0.5) and clustering placement, and keeps their results on the device:
// the permutation, the BCSR matrix of the permuted rows and the batch
// kernel's dispatch order.  execute() is then the Tier-1 SpMM alone.
//   * fp16, N % 8 == 0, on the batch kernel: its store writes product row r
//     straight into C row perm[r] -- the un-permutation of the pipeline fused
//     into the SpMM, one launch, no temporary;
//   * packed column batches, when they take at most 3/4 of the BCSR values'
//     bytes: fp16, the batch kernel's batches (spmm_f16_packed); fp32, the
//     pipeline's packed fp32 batches formed from the permuted CSR
//     (csr_pack_analyse / csr_pack_emit, spmm_f32_packed); both with the
//     fused store;
//   * a fully populated block grid takes the GEMM-tiled kernel, as in the
//     pipeline, with the same fused store;
//   * otherwise (fp32, other N) the product goes to a workspace kept by the
//     plan (it only grows) and is un-permuted into C.
// C equals the pipeline's C bit for bit: the same kernels accumulate in the
// same order, only the row a result is stored to differs.  execute() does not
// allocate once the workspace is large enough (never, on the fused path).
// Calls on one plan must not overlap (they share the workspace).
#include <cstdlib>
#include <cstring>
#include <limits>
#include <vector>

#include "internal.hpp"

namespace xspmm {
namespace detail {

namespace {

// Device memory owned for the plan's lifetime (not stream-ordered: a plan
// outlives the streams it is used on).
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) { reset(bytes); }
    ~DeviceBuffer() {
        if (p_) (void)hipFree(p_);
    }
    DeviceBuffer(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(const DeviceBuffer&) = delete;
    DeviceBuffer& operator=(DeviceBuffer&& o) noexcept {
        if (this != &o) {
            if (p_) (void)hipFree(p_);
            p_ = o.p_;
            n_ = o.n_;
            o.p_ = nullptr;
            o.n_ = 0;
        }
        return *this;
    }
    void reset(size_t bytes) {
        if (p_) XSPMM_HIP_CHECK(hipFree(p_));
        p_ = nullptr;
        n_ = 0;
        if (bytes) XSPMM_HIP_CHECK(hipMalloc(&p_, bytes));
        n_ = bytes;
    }
    size_t size() const { return n_; }
    template <typename T>
    T* as() const { return static_cast<T*>(p_); }

private:
    void* p_ = nullptr;
    size_t n_ = 0;
};

template <typename T, typename I>
class Plan final : public PlanBase {
public:
    Plan(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const T* vals, int64_t hw,
         bool optimize_pattern, double* tm, hipStream_t s)
    {
        if (M < 0 || K < 0 || nnz < 0) throw std::invalid_argument("CSR dimensions must be non-negative.");
        if (hw != 16)
            throw std::invalid_argument("xSpMM: the MFMA tile kernel requires hw_block_size == 16.");
        M_ = M;
        K_ = K;
        Mb_ = (M + 15) / 16;
        Kb_ = (K + 15) / 16;
        clustered_ = optimize_pattern;
        StageTimer total(tm != nullptr, s), step(tm != nullptr, s);
        total.start();

        const I* crp = rp;
        const I* cci = ci;
        const T* cvals = vals;
        Scratch nrp, nci, nvals;
        if (optimize_pattern) {
            step.start();
            perm_.reset((size_t)(M > 0 ? M : 1) * sizeof(I));
            jaccard_clustering_dispatch<I>(M, K, nnz, rp, ci, 0.5f, hw, perm_.as<I>(), s);
            if (tm) step.stop(&tm[0]);

            step.start();
            nrp = Scratch((size_t)(M + 1) * sizeof(I), s);
            nci = Scratch((size_t)(nnz > 0 ? nnz : 1) * sizeof(I), s);
            nvals = Scratch((size_t)(nnz > 0 ? nnz : 1) * sizeof(T), s);
            apply_permutation<T, I>(M, nnz, rp, ci, vals, perm_.as<I>(), nrp.as<I>(), nci.as<I>(),
                                    nvals.as<T>(), s);
            crp = nrp.as<I>();
            cci = nci.as<I>();
            cvals = nvals.as<T>();
            if (tm) step.stop(&tm[1]);
        }

        step.start();
        brp_.reset((size_t)(Mb_ + 1) * sizeof(I));
        nnzb_ = csr_to_bcsr_count<I>(M, K, nnz, crp, cci, 16, 16, brp_.as<I>(), s);
        bci_.reset((size_t)(nnzb_ > 0 ? nnzb_ : 1) * sizeof(I));
        bvals_.reset((size_t)(nnzb_ > 0 ? nnzb_ : 1) * 256 * sizeof(T));
        csr_to_bcsr_fill<T, I>(M, K, nnz, crp, cci, cvals, 16, 16, brp_.as<I>(), bci_.as<I>(),
                               bvals_.as<T>(), s);
        if (spmm_order_cols_wanted(Mb_)) {
            order_.reset((size_t)(Mb_ + 1) * sizeof(int32_t));
            if (!spmm_dispatch_order_cols<I>(brp_.as<I>(), bci_.as<I>(), Mb_, order_.as<int32_t>(), s))
                order_.reset(0);  // the identity: not worth a load per workgroup
        }
        if constexpr (sizeof(T) == 2)
            pack(s);
        else
            pack32(M, K, nnz, crp, cci, reinterpret_cast<const uint32_t*>(cvals), s);
        if (tm) step.stop(&tm[2]);
        if (tm) total.stop(&tm[5]);
        XSPMM_HIP_CHECK(hipStreamSynchronize(s));
        step.finish();
        total.finish();
    }

    // Packed column batches: the batch kernel's batches, formed once.  Kept
    // when they take at most 3/4 of the BCSR values' bytes (sparse blocks);
    // a fully populated grid keeps the GEMM-tiled kernel instead.
    void pack(hipStream_t s)
    {
        if (nnzb_ == 0 || nnzb_ == Mb_ * Kb_ || !spmm_f16_pack_supported(K_, Mb_, Kb_)) return;
        if (const char* e = std::getenv("XSPMM_PLAN_PACK"))
            if (std::strcmp(e, "off") == 0) return;
        const uint16_t* v = reinterpret_cast<const uint16_t*>(bvals_.as<T>());
        Scratch counts((size_t)Mb_ * spmm_batch_waves() * sizeof(int32_t), s);
        spmm_f16_pack_count<I>(M_, K_, Mb_, Kb_, brp_.as<I>(), bci_.as<I>(), v,
                               counts.as<int32_t>(), s);
        DeviceBuffer offsets((size_t)(Mb_ * spmm_batch_waves() + 1) * sizeof(int64_t));
        const int64_t nb = spmm_f16_pack_offsets(counts.as<int32_t>(), Mb_ * spmm_batch_waves(),
                                                 offsets.as<int64_t>(), s);
        if ((double)nb * (1024.0 + 128.0) > 0.75 * (double)nnzb_ * 512.0) return;
        pa_.reset((size_t)(nb > 0 ? nb : 1) * 1024);
        prow_.reset((size_t)(nb > 0 ? nb : 1) * 128);
        spmm_f16_pack_fill<I>(M_, K_, Mb_, Kb_, brp_.as<I>(), bci_.as<I>(), v,
                              offsets.as<int64_t>(), pa_.as<void>(), prow_.as<uint32_t>(), s);
        poff_ = std::move(offsets);
        nbatches_ = nb;
        packed_ = true;
    }

    // Packed fp32 column batches from the (permuted) CSR, as the pipeline
    // forms them; kept when the device's decision takes them (sorted input,
    // batches at most 3/4 of the BCSR values' bytes).
    void pack32(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const uint32_t* v,
                hipStream_t s)
    {
        if (M == 0 || nnz == 0 || !csr_pack_covers(K)) return;
        if (const char* e = std::getenv("XSPMM_PLAN_PACK"))
            if (std::strcmp(e, "off") == 0) return;
        Carve cv;
        const size_t o_bc = cv.take((size_t)Mb_ * sizeof(I));
        const size_t o_brp = cv.take((size_t)(Mb_ + 1) * sizeof(I));
        const size_t o_cnt = cv.take((size_t)Mb_ * sizeof(int32_t));
        const size_t o_err = cv.take(sizeof(int));
        const size_t o_flags = cv.take(sizeof(unsigned int));
        const size_t o_st = cv.take(5 * sizeof(int64_t));
        Scratch tmp(cv.end, s);
        char* b = tmp.as<char>();
        DeviceBuffer offsets((size_t)(Mb_ + 1) * sizeof(int64_t));
        csr_pack_analyse<I, uint32_t>(M, K, nnz, rp, ci, v, reinterpret_cast<I*>(b + o_bc),
                                      reinterpret_cast<I*>(b + o_brp), reinterpret_cast<int32_t*>(b + o_cnt),
                                      offsets.as<int64_t>(), reinterpret_cast<int*>(b + o_err),
                                      reinterpret_cast<unsigned int*>(b + o_flags),
                                      std::numeric_limits<int64_t>::max() / 2048,
                                      reinterpret_cast<int64_t*>(b + o_st), s);
        const PackStatus st = csr_pack_status(reinterpret_cast<const int64_t*>(b + o_st), s);
        if (!st.go) return;
        pa_.reset((size_t)st.nbatches * 256);
        prow_.reset((size_t)st.nbatches * 16);
        csr_pack_emit<I, uint32_t>(M, K, nnz, rp, ci, v, offsets.as<int64_t>(),
                                   reinterpret_cast<const int64_t*>(b + o_st), st.nbatches, pa_.as<void>(),
                                   prow_.as<uint32_t>(), s);
        poff_ = std::move(offsets);
        nbatches_ = st.nbatches;
        packed_ = true;
    }

    void execute(const void* Bv, float* C, int64_t N, hipStream_t s) override
    {
        if (N < 0) throw std::invalid_argument("xSpMM: negative N.");
        if (M_ == 0 || N == 0) return;
        const T* B = static_cast<const T*>(Bv);
        const int32_t* order = order_.size() ? order_.as<int32_t>() : nullptr;
        if constexpr (sizeof(T) == 2) {
            if (packed_ && spmm_f16_packed<I>(M_, K_, Mb_, poff_.as<int64_t>(), pa_.as<void>(),
                                              prow_.as<uint32_t>(),
                                              reinterpret_cast<const uint16_t*>(B), C, N, order,
                                              clustered_ ? perm_.as<I>() : nullptr, s))
                return;
        } else {
            if (packed_ && spmm_f32_packed<I>(M_, K_, Mb_, poff_.as<int64_t>(), pa_.as<void>(),
                                              prow_.as<uint32_t>(), reinterpret_cast<const float*>(B), C,
                                              N, order, clustered_ ? perm_.as<I>() : nullptr, s))
                return;
        }
        if (!clustered_) {
            bcsr_spmm_ex<T, I>(M_, K_, Mb_, Kb_, nnzb_, brp_.as<I>(), bci_.as<I>(), bvals_.as<T>(),
                               B, C, N, order, nullptr, s);
            return;
        }
        if (bcsr_spmm_ex<T, I>(M_, K_, Mb_, Kb_, nnzb_, brp_.as<I>(), bci_.as<I>(),
                               bvals_.as<T>(), B, C, N, order, perm_.as<I>(), s))
            return;
        const size_t need = (size_t)M_ * (size_t)N * sizeof(float);
        if (ws_.size() < need) {
            XSPMM_HIP_CHECK(hipStreamSynchronize(s));  // the old workspace may be in use
            ws_.reset(need);
        }
        bcsr_spmm_ex<T, I>(M_, K_, Mb_, Kb_, nnzb_, brp_.as<I>(), bci_.as<I>(), bvals_.as<T>(), B,
                           ws_.as<float>(), N, order, nullptr, s);
        unpermute_dense<I>(ws_.as<float>(), C, perm_.as<I>(), M_, N, s);
    }

    int64_t num_blocks() const override { return nnzb_; }
    int64_t num_packed_batches() const override { return packed_ ? nbatches_ : -1; }
    int64_t num_block_rows() const override { return Mb_; }
    bool clustered() const override { return clustered_; }
    const void* permutation() const override { return clustered_ ? perm_.as<void>() : nullptr; }

private:
    int64_t M_ = 0, K_ = 0, Mb_ = 0, Kb_ = 0, nnzb_ = 0, nbatches_ = 0;
    bool clustered_ = false, packed_ = false;
    DeviceBuffer perm_, brp_, bci_, bvals_, order_, ws_;
    DeviceBuffer poff_, pa_, prow_;  // packed column batches
};

}  // namespace

template <typename T, typename I>
PlanBase* make_plan(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const T* vals,
                    int64_t hw, bool optimize_pattern, double* tm, hipStream_t s)
{
    return new Plan<T, I>(M, K, nnz, rp, ci, vals, hw, optimize_pattern, tm, s);
}

#define XSPMM_MAKE_PLAN(T, I)                                                                  \
    template PlanBase* make_plan<T, I>(int64_t, int64_t, int64_t, const I*, const I*, const T*, \
                                       int64_t, bool, double*, hipStream_t);
XSPMM_MAKE_PLAN(uint16_t, int32_t)
XSPMM_MAKE_PLAN(uint16_t, int64_t)
XSPMM_MAKE_PLAN(float, int32_t)
XSPMM_MAKE_PLAN(float, int64_t)
#undef XSPMM_MAKE_PLAN

}  // namespace detail
}  // namespace xspmm
