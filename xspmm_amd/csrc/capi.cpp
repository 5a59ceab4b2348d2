// capi.cpp -- extern "C" entry points declared in include/xspmm_capi.h.
// Each maps type codes onto the internal launchers and turns exceptions into
// error codes (std::invalid_argument -> XSPMM_ERR_INVALID, "HIP Error" ->
// XSPMM_ERR_HIP, any other failure -> XSPMM_ERR_UNSUPPORTED).
#include <hip/hip_fp16.h>

#include <cstring>
#include <string>
#include <utility>

#include "internal.hpp"
#include "xspmm_capi.h"

using namespace xspmm::detail;

// The opaque handles of the C ABI.
struct xspmm_plan_s {
    PlanBase* impl;
};
struct xspmm_mtx_s {
    MtxData data;
};

namespace {

thread_local std::string g_last_error;

template <typename F>
int guarded(F&& f)
{
    try {
        f();
        g_last_error.clear();
        return XSPMM_OK;
    } catch (const std::invalid_argument& e) {
        g_last_error = e.what();
        return XSPMM_ERR_INVALID;
    } catch (const MtxError& e) {
        g_last_error = e.what();
        return XSPMM_ERR_IO;
    } catch (const std::exception& e) {
        g_last_error = e.what();
        return std::strncmp(e.what(), "HIP Error", 9) == 0 ? XSPMM_ERR_HIP : XSPMM_ERR_UNSUPPORTED;
    } catch (...) {
        g_last_error = "unknown error";
        return XSPMM_ERR_UNSUPPORTED;
    }
}

template <typename T>
struct Tag { using type = T; };

// Calls f(Tag<value>, Tag<index>) for the requested type codes.
template <typename F>
void with_types(int vtype, int itype, F&& f)
{
    if (itype != XSPMM_I32 && itype != XSPMM_I64) throw std::invalid_argument("unknown index type code");
    if (vtype != XSPMM_F32 && vtype != XSPMM_F16) throw std::invalid_argument("unknown value type code");
    if (vtype == XSPMM_F16) {
        if (itype == XSPMM_I32) f(Tag<uint16_t>{}, Tag<int32_t>{});
        else f(Tag<uint16_t>{}, Tag<int64_t>{});
    } else {
        if (itype == XSPMM_I32) f(Tag<float>{}, Tag<int32_t>{});
        else f(Tag<float>{}, Tag<int64_t>{});
    }
}

template <typename F>
void with_index(int itype, F&& f)
{
    if (itype == XSPMM_I32) f(Tag<int32_t>{});
    else if (itype == XSPMM_I64) f(Tag<int64_t>{});
    else throw std::invalid_argument("unknown index type code");
}

hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

void require(bool ok, const char* what)
{
    if (!ok) throw std::invalid_argument(what);
}

}  // namespace

extern "C" {

const char* xspmm_last_error(void) { return g_last_error.c_str(); }

int xspmm_abi_version(void) { return 4; }

int xspmm_bcsr_spmm(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb,
                    int64_t nnzb, const void* brp, const void* bci, const void* bvals,
                    const void* B, float* C, int64_t N, void* stream)
{
    return guarded([&] {
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            bcsr_spmm<T, I>(M, K, Mb, Kb, nnzb, static_cast<const I*>(brp), static_cast<const I*>(bci),
                            static_cast<const T*>(bvals), static_cast<const T*>(B), C, N,
                            as_stream(stream));
        });
    });
}

int xspmm_bcsr_spmm_noalloc(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb,
                            int64_t nnzb, const void* brp, const void* bci, const void* bvals,
                            const void* B, float* C, int64_t N, void* stream)
{
    return guarded([&] {
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            bcsr_spmm_noalloc<T, I>(M, K, Mb, Kb, nnzb, static_cast<const I*>(brp),
                                    static_cast<const I*>(bci), static_cast<const T*>(bvals),
                                    static_cast<const T*>(B), C, N, as_stream(stream));
        });
    });
}

int64_t xspmm_noalloc_scratch_bytes(void) { return (int64_t)kNoAllocScratchBytes; }

int xspmm_bcsr_dispatch_order(int itype, int64_t Mb, const void* brp, int32_t* order,
                              int* written, void* stream)
{
    return guarded([&] {
        if (Mb < 0) throw std::invalid_argument("xSpMM: negative number of block-rows.");
        if (!written) throw std::invalid_argument("xSpMM: written must not be NULL.");
        *written = 0;
        if (!spmm_order_wanted(Mb)) return;
        if (!brp || !order) throw std::invalid_argument("xSpMM: brp and order must not be NULL.");
        with_index(itype, [&](auto ti) {
            using I = typename decltype(ti)::type;
            spmm_dispatch_order<I>(static_cast<const I*>(brp), Mb, order, as_stream(stream));
        });
        *written = 1;
    });
}

int xspmm_bcsr_dispatch_order_cols(int itype, int64_t Mb, const void* brp, const void* bci,
                                   int32_t* order, int* written, void* stream)
{
    return guarded([&] {
        if (Mb < 0) throw std::invalid_argument("xSpMM: negative number of block-rows.");
        if (!written) throw std::invalid_argument("xSpMM: written must not be NULL.");
        *written = 0;
        if (!spmm_order_cols_wanted(Mb)) return;
        if (!brp || !bci || !order)
            throw std::invalid_argument("xSpMM: brp, bci and order must not be NULL.");
        bool used = false;
        with_index(itype, [&](auto ti) {
            using I = typename decltype(ti)::type;
            used = spmm_dispatch_order_cols<I>(static_cast<const I*>(brp), static_cast<const I*>(bci), Mb,
                                               order, as_stream(stream));
        });
        *written = used ? 1 : 0;
    });
}

int xspmm_bcsr_spmm_ordered(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb,
                            int64_t nnzb, const void* brp, const void* bci, const void* bvals,
                            const void* B, float* C, int64_t N, const int32_t* order, void* stream)
{
    return guarded([&] {
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            (void)bcsr_spmm_ex<T, I>(M, K, Mb, Kb, nnzb, static_cast<const I*>(brp),
                                     static_cast<const I*>(bci), static_cast<const T*>(bvals),
                                     static_cast<const T*>(B), C, N, order, nullptr,
                                     as_stream(stream));
        });
    });
}

int xspmm_bcsr_band_rows(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnz,
                         int64_t nnzb, const void* brp, const void* bci, int* band, void* stream)
{
    return guarded([&] {
        if (!band) throw std::invalid_argument("xSpMM: band must not be NULL.");
        *band = 0;
        if (vtype != XSPMM_F16 && vtype != XSPMM_F32) throw std::invalid_argument("xSpMM: unknown value type.");
        if (M < 0 || K < 0 || Mb < 0 || Kb < 0 || nnzb < 0)
            throw std::invalid_argument("xSpMM: negative size passed to BCSR SpMM.");
        if (Mb == 0 || nnzb == 0) return;
        if (!brp || !bci) throw std::invalid_argument("xSpMM: brp and bci must not be NULL.");
        with_index(itype, [&](auto ti) {
            using I = typename decltype(ti)::type;
            *band = spmm_band_wanted<I>(static_cast<const I*>(brp), static_cast<const I*>(bci), M, K, Mb, Kb,
                                        nnz, nnzb, 0, vtype == XSPMM_F16 ? 2 : 4, as_stream(stream))
                        ? 1
                        : 0;
        });
    });
}

int xspmm_bcsr_spmm_band(int vtype, int itype, int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb,
                         const void* brp, const void* bci, const void* bvals, const void* B, float* C,
                         int64_t N, void* stream)
{
    return guarded([&] {
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            bcsr_spmm_band<T, I>(M, K, Mb, Kb, nnzb, static_cast<const I*>(brp), static_cast<const I*>(bci),
                                 static_cast<const T*>(bvals), static_cast<const T*>(B), C, N, as_stream(stream));
        });
    });
}

int xspmm_csr_to_bcsr_count(int itype, int64_t M, int64_t K, int64_t nnz, const void* rp,
                            const void* ci, int64_t r_block, int64_t c_block,
                            void* bcsr_row_ptr, int64_t* nnzb_out, void* stream)
{
    return guarded([&] {
        require(nnzb_out != nullptr, "nnzb_out is null");
        with_index(itype, [&](auto ti) {
            using I = typename decltype(ti)::type;
            *nnzb_out = csr_to_bcsr_count<I>(M, K, nnz, static_cast<const I*>(rp),
                                             static_cast<const I*>(ci), r_block, c_block,
                                             static_cast<I*>(bcsr_row_ptr), as_stream(stream));
        });
    });
}

int xspmm_csr_to_bcsr_fill(int vtype, int itype, int64_t M, int64_t K, int64_t nnz,
                           const void* rp, const void* ci, const void* vals,
                           int64_t r_block, int64_t c_block, const void* bcsr_row_ptr,
                           void* bcsr_col_ind, void* bcsr_vals, void* stream)
{
    return guarded([&] {
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            csr_to_bcsr_fill<T, I>(M, K, nnz, static_cast<const I*>(rp), static_cast<const I*>(ci),
                                   static_cast<const T*>(vals), r_block, c_block,
                                   static_cast<const I*>(bcsr_row_ptr), static_cast<I*>(bcsr_col_ind),
                                   static_cast<T*>(bcsr_vals), as_stream(stream));
        });
    });
}

int xspmm_apply_permutation(int vtype, int itype, int64_t M, int64_t nnz, const void* rp,
                            const void* ci, const void* vals, const void* perm,
                            void* new_rp, void* new_ci, void* new_vals, void* stream)
{
    return guarded([&] {
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            apply_permutation<T, I>(M, nnz, static_cast<const I*>(rp), static_cast<const I*>(ci),
                                    static_cast<const T*>(vals), static_cast<const I*>(perm),
                                    static_cast<I*>(new_rp), static_cast<I*>(new_ci),
                                    static_cast<T*>(new_vals), as_stream(stream));
        });
    });
}

int xspmm_unpermute_dense(int itype, const float* in, float* out, const void* perm, int64_t M,
                          int64_t N, void* stream)
{
    return guarded([&] {
        with_index(itype, [&](auto ti) {
            using I = typename decltype(ti)::type;
            unpermute_dense<I>(in, out, static_cast<const I*>(perm), M, N, as_stream(stream));
        });
    });
}

int xspmm_jaccard_clustering_host(int itype, int64_t M, int64_t K, const void* rp,
                                  const void* ci, float dist_thresh, int64_t block_width,
                                  void* perm_out, int nthreads)
{
    return guarded([&] {
        with_index(itype, [&](auto ti) {
            using I = typename decltype(ti)::type;
            jaccard_clustering_host<I>(M, K, static_cast<const I*>(rp), static_cast<const I*>(ci),
                                       dist_thresh, block_width, static_cast<I*>(perm_out), nthreads);
        });
    });
}

int xspmm_jaccard_clustering(int itype, int64_t M, int64_t K, int64_t nnz, const void* rp,
                             const void* ci, float dist_thresh, int64_t block_width,
                             void* perm_out, int* engine_used, void* stream)
{
    return guarded([&] {
        with_index(itype, [&](auto ti) {
            using I = typename decltype(ti)::type;
            jaccard_clustering_device<I>(M, K, nnz, static_cast<const I*>(rp),
                                         static_cast<const I*>(ci), dist_thresh, block_width,
                                         static_cast<I*>(perm_out), as_stream(stream), engine_used);
        });
    });
}

int xspmm_spmm_pipeline(int vtype, int itype, int64_t M, int64_t K, int64_t nnz,
                        const void* rp, const void* ci, const void* vals, const void* B,
                        float* C, int64_t N, int64_t hw_block_size, int optimize_pattern,
                        double* timings, void* stream)
{
    return guarded([&] {
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            require(M >= 0 && K >= 0 && nnz >= 0 && N >= 0, "CSR dimensions must be non-negative.");
            require(hw_block_size == 16,
                    "xSpMM: the MFMA tile kernel requires hw_block_size == 16.");
            spmm_pipeline<T, I>(M, K, nnz, static_cast<const I*>(rp), static_cast<const I*>(ci),
                                static_cast<const T*>(vals), static_cast<const T*>(B), C, N,
                                hw_block_size, optimize_pattern != 0, timings, as_stream(stream));
        });
    });
}

int xspmm_pipeline_temp_bytes(int64_t* bytes_out)
{
    return guarded([&] {
        require(bytes_out != nullptr, "xspmm_pipeline_temp_bytes: bytes_out is null.");
        *bytes_out = (int64_t)last_pipeline_temp_bytes();
    });
}

int xspmm_pipeline_last_form(int* packed_out)
{
    return guarded([&] {
        require(packed_out != nullptr, "xspmm_pipeline_last_form: packed_out is null.");
        *packed_out = last_pipeline_packed() ? 1 : 0;
    });
}

int xspmm_plan_create(int vtype, int itype, int64_t M, int64_t K, int64_t nnz, const void* rp,
                      const void* ci, const void* vals, int64_t hw_block_size,
                      int optimize_pattern, double* timings, void* stream, xspmm_plan_t* plan_out)
{
    return guarded([&] {
        require(plan_out != nullptr, "xspmm_plan_create: plan_out is null.");
        *plan_out = nullptr;
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            require(M >= 0 && K >= 0 && nnz >= 0, "CSR dimensions must be non-negative.");
            require(hw_block_size == 16,
                    "xSpMM: the MFMA tile kernel requires hw_block_size == 16.");
            PlanBase* impl = make_plan<T, I>(M, K, nnz, static_cast<const I*>(rp),
                                             static_cast<const I*>(ci), static_cast<const T*>(vals),
                                             hw_block_size, optimize_pattern != 0, timings,
                                             as_stream(stream));
            *plan_out = new xspmm_plan_s{impl};
        });
    });
}

int xspmm_plan_execute(xspmm_plan_t plan, const void* B, float* C, int64_t N, void* stream)
{
    return guarded([&] {
        require(plan != nullptr, "xspmm_plan_execute: null plan.");
        require(N >= 0, "xSpMM: negative N.");
        plan->impl->execute(B, C, N, as_stream(stream));
    });
}

int xspmm_plan_info(xspmm_plan_t plan, int64_t* num_blocks, int64_t* num_block_rows,
                    int* clustered, const void** perm)
{
    return guarded([&] {
        require(plan != nullptr, "xspmm_plan_info: null plan.");
        if (num_blocks) *num_blocks = plan->impl->num_blocks();
        if (num_block_rows) *num_block_rows = plan->impl->num_block_rows();
        if (clustered) *clustered = plan->impl->clustered() ? 1 : 0;
        if (perm) *perm = plan->impl->permutation();
    });
}

int xspmm_plan_packed_batches(xspmm_plan_t plan, int64_t* batches)
{
    return guarded([&] {
        require(plan != nullptr && batches != nullptr, "xspmm_plan_packed_batches: null argument.");
        *batches = plan->impl->num_packed_batches();
    });
}

int xspmm_plan_destroy(xspmm_plan_t plan)
{
    return guarded([&] {
        if (!plan) return;
        delete plan->impl;
        delete plan;
    });
}

int xspmm_mtx_read(const char* path, xspmm_mtx_t* out)
{
    return guarded([&] {
        require(out != nullptr && path != nullptr, "xspmm_mtx_read: null argument.");
        *out = nullptr;
        auto* m = new xspmm_mtx_s{read_matrix_market(path)};
        *out = m;
    });
}

int xspmm_mtx_info(xspmm_mtx_t m, int64_t* rows, int64_t* cols, int64_t* nnz)
{
    return guarded([&] {
        require(m != nullptr, "xspmm_mtx_info: null handle.");
        if (rows) *rows = m->data.rows;
        if (cols) *cols = m->data.cols;
        if (nnz) *nnz = (int64_t)m->data.values.size();
    });
}

int xspmm_mtx_export(xspmm_mtx_t m, int itype, int vtype, void* row_ptr, void* col_ind,
                     void* values)
{
    return guarded([&] {
        require(m != nullptr, "xspmm_mtx_export: null handle.");
        const MtxData& d = m->data;
        const size_t nnz = d.values.size();
        require(row_ptr != nullptr && (nnz == 0 || (col_ind != nullptr && values != nullptr)),
                "xspmm_mtx_export: null output array.");
        with_types(vtype, itype, [&](auto tv, auto ti) {
            using T = typename decltype(tv)::type;
            using I = typename decltype(ti)::type;
            I* rp = static_cast<I*>(row_ptr);
            I* ci = static_cast<I*>(col_ind);
            for (size_t i = 0; i < d.row_ptr.size(); ++i) rp[i] = (I)d.row_ptr[i];
            for (size_t k = 0; k < nnz; ++k) ci[k] = (I)d.col_ind[k];
            T* v = static_cast<T*>(values);
            for (size_t k = 0; k < nnz; ++k) {
                if constexpr (sizeof(T) == 2) {
                    const __half h = __float2half(d.values[k]);  // round to nearest even
                    std::memcpy(&v[k], &h, 2);
                } else {
                    v[k] = d.values[k];
                }
            }
        });
    });
}

int xspmm_mtx_free(xspmm_mtx_t m)
{
    return guarded([&] { delete m; });
}

}  // extern "C"
