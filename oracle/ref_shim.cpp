// ref_shim.cpp -- flat C entry points over the reference's own CPU code.
//
// TEST INFRASTRUCTURE ONLY.  Built by oracle/Makefile together with the
// reference sources compiled where they lie under /root/reference
// (src/core/conversion.cpp, src/core/executor.cpp,
// src/cpu/clustering_sylos_labini.cpp, src/xspmm.cpp), into
// oracle/_ref/libxspmm_ref.so.  tests/golden/make_golden.py calls it through
// ctypes to write golden vectors that pin the C restatement in oracle.c.
//
// The MatrixMarket reader is the reference's header utils/matrix_io.hpp
// (matrix_utils::io::read_mtx<float>, :27-98), included where it lies.
//
// Everything runs on the reference's CpuExecutor (src/core/executor.cpp:44-72),
// so "device" pointers are host memory.  The reference instantiates float
// values only (src/core/conversion.cpp:106-108, src/xspmm.cpp:110-114), so
// values are passed as float here; the structure is type-agnostic.
#include <cstdint>
#include <cstring>
#include <memory>

#include "xspmm/clustering.hpp"
#include "xspmm/core/executor.hpp"
#include "xspmm/matrix/conversion.hpp"
#include "matrix_io.hpp"

namespace {

template <typename I>
xspmm::CSRMatrix<float, I> make_csr(const std::shared_ptr<const xspmm::Executor>& ex,
                                    I M, I K, I nnz, const I* rp, const I* ci,
                                    const float* vals)
{
    xspmm::CSRMatrix<float, I> A(ex, M, K, nnz);
    A.copy_from_host(rp, ci, vals);
    return A;
}

template <typename I>
int64_t csr_to_bcsr(I M, I K, I nnz, const I* rp, const I* ci, const float* vals,
                    I rb, I cb, I* out_rp, I* out_ci, float* out_vals,
                    int64_t cap_blocks)
{
    auto ex = std::make_shared<const xspmm::CpuExecutor>();
    auto A = make_csr<I>(ex, M, K, nnz, rp, ci, vals);
    auto Bm = xspmm::csr_to_bcsr<float, I>(ex, A, rb, cb);
    int64_t nnzb = Bm.get_num_blocks();
    if (nnzb <= cap_blocks) {
        std::memcpy(out_rp, Bm.get_bcsr_row_ptr(), sizeof(I) * (size_t)(Bm.get_num_block_rows() + 1));
        if (nnzb > 0) {
            std::memcpy(out_ci, Bm.get_bcsr_col_ind(), sizeof(I) * (size_t)nnzb);
            std::memcpy(out_vals, Bm.get_bcsr_values(), sizeof(float) * (size_t)(nnzb * rb * cb));
        }
    }
    return nnzb;
}

template <typename I>
void jaccard(I M, I K, I nnz, const I* rp, const I* ci, float thresh, I bw, I* perm)
{
    auto ex = std::make_shared<const xspmm::CpuExecutor>();
    std::unique_ptr<float[]> vals(new float[nnz > 0 ? nnz : 1]());
    auto A = make_csr<I>(ex, M, K, nnz, rp, ci, vals.get());
    xspmm::compute_1d_jaccard_clustering<float, I>(ex, A, thresh, bw, perm);
}

template <typename I>
void apply_perm(I M, I K, I nnz, const I* rp, const I* ci, const float* vals,
                const I* perm, I* nrp, I* nci, float* nvals)
{
    auto ex = std::make_shared<const xspmm::CpuExecutor>();
    auto A = make_csr<I>(ex, M, K, nnz, rp, ci, vals);
    auto P = xspmm::apply_permutation<float, I>(ex, A, perm);
    std::memcpy(nrp, P.get_row_ptr(), sizeof(I) * (size_t)(M + 1));
    if (nnz > 0) {
        std::memcpy(nci, P.get_col_ind(), sizeof(I) * (size_t)nnz);
        std::memcpy(nvals, P.get_values(), sizeof(float) * (size_t)nnz);
    }
}

}  // namespace

extern "C" {

int64_t ref_csr_to_bcsr_i32(int32_t M, int32_t K, int32_t nnz, const int32_t* rp,
                            const int32_t* ci, const float* vals, int32_t rb, int32_t cb,
                            int32_t* out_rp, int32_t* out_ci, float* out_vals,
                            int64_t cap_blocks)
{
    return csr_to_bcsr<int32_t>(M, K, nnz, rp, ci, vals, rb, cb, out_rp, out_ci, out_vals, cap_blocks);
}

int64_t ref_csr_to_bcsr_i64(int64_t M, int64_t K, int64_t nnz, const int64_t* rp,
                            const int64_t* ci, const float* vals, int64_t rb, int64_t cb,
                            int64_t* out_rp, int64_t* out_ci, float* out_vals,
                            int64_t cap_blocks)
{
    return csr_to_bcsr<int64_t>(M, K, nnz, rp, ci, vals, rb, cb, out_rp, out_ci, out_vals, cap_blocks);
}

void ref_jaccard_i32(int32_t M, int32_t K, int32_t nnz, const int32_t* rp, const int32_t* ci,
                     float thresh, int32_t bw, int32_t* perm)
{
    jaccard<int32_t>(M, K, nnz, rp, ci, thresh, bw, perm);
}

void ref_jaccard_i64(int64_t M, int64_t K, int64_t nnz, const int64_t* rp, const int64_t* ci,
                     float thresh, int64_t bw, int64_t* perm)
{
    jaccard<int64_t>(M, K, nnz, rp, ci, thresh, bw, perm);
}

void ref_apply_perm_i32(int32_t M, int32_t K, int32_t nnz, const int32_t* rp, const int32_t* ci,
                        const float* vals, const int32_t* perm, int32_t* nrp, int32_t* nci,
                        float* nvals)
{
    apply_perm<int32_t>(M, K, nnz, rp, ci, vals, perm, nrp, nci, nvals);
}

void ref_apply_perm_i64(int64_t M, int64_t K, int64_t nnz, const int64_t* rp, const int64_t* ci,
                        const float* vals, const int64_t* perm, int64_t* nrp, int64_t* nci,
                        float* nvals)
{
    apply_perm<int64_t>(M, K, nnz, rp, ci, vals, perm, nrp, nci, nvals);
}

// Reads `path` with the reference's reader.  Returns nnz (the number of
// entries kept) and fills the outputs when nnz <= cap, or -1 with the
// exception message in err.
int64_t ref_read_mtx(const char* path, int32_t* M, int32_t* K, int32_t* rp, int32_t* ci,
                     float* vals, int64_t cap, char* err, int32_t errlen)
{
    try {
        auto h = matrix_utils::io::read_mtx<float>(path);
        *M = h.num_rows;
        *K = h.num_cols;
        const int64_t nnz = (int64_t)h.values.size();
        if (nnz <= cap) {
            std::memcpy(rp, h.row_ptr.data(), sizeof(int32_t) * h.row_ptr.size());
            if (nnz > 0) {
                std::memcpy(ci, h.col_ind.data(), sizeof(int32_t) * (size_t)nnz);
                std::memcpy(vals, h.values.data(), sizeof(float) * (size_t)nnz);
            }
        }
        return nnz;
    } catch (const std::exception& e) {
        std::strncpy(err, e.what(), (size_t)errlen - 1);
        err[errlen - 1] = '\0';
        return -1;
    }
}

}  // extern "C"
