// pipeline.cpp -- Tier-2 automated pipeline on raw device pointers.
//
// Stage order, thresholds and timing fields follow the reference
// (src/hip/unstructured_mtx_mul.hip:31-100):
//   clustering on : cluster (threshold 0.5, width hw_block_size) ->
//                   permute rows -> CSR->BCSR -> SpMM into C_temp ->
//                   un-permute C_temp into C;
//   clustering off: CSR->BCSR -> SpMM into C.
// Every stage except clustering runs on the GPU.  Clustering runs the host
// greedy on copies of row_ptr/col_ind, as the reference does; with
// XSPMM_CLUSTER_DEVICE=gpu it runs the GPU engine instead (the same
// permutation), within that engine's shape limits.  Each timed stage is
// bracketed by HIP events on the pipeline stream, so host work inside a
// bracket counts too (the reference's HipTimer does the same); the events
// are read once the pipeline has drained instead of after each stage.
// Differences from the reference, with identical results: C / C_temp are not
// memset first (the SpMM overwrites every element), temporaries come from one
// stream-ordered allocation instead of hipMalloc/hipFree pairs, taken before
// the first stage, and permuted row_ptr[M] is the sum of the gathered lengths
// (equal to nnz for a permutation).  The BCSR arrays are part of that
// allocation, sized from the bound min(nnz, Mb * Kb) on the block count, when
// the bound's block values take at most kFusedConversionBytes: the
// conversion's count and fill then run back to back with no host round trip.
// Above that the bound can exceed the exact size many times over (256x when
// every block is full), so the conversion reads the count first and takes the
// arrays at their exact size, as the reference does
// (src/core/conversion.cpp:66-73).
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "internal.hpp"

namespace xspmm {
namespace detail {

namespace {

// Largest bound-sized BCSR value array the fused conversion takes (above it,
// exact sizing after one host round trip).
constexpr size_t kFusedConversionBytes = size_t(1) << 30;

// Device bytes of the last pipeline call's temporaries on this thread.
thread_local size_t g_last_temp_bytes = 0;

}  // namespace

size_t last_pipeline_temp_bytes() { return g_last_temp_bytes; }


template <typename I>
void jaccard_clustering_dispatch(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                                 float dist_thresh, int64_t block_width, I* d_perm, hipStream_t s)
{
    if (M < 0 || K < 0 || nnz < 0) throw std::invalid_argument("CSR dimensions must be non-negative.");
    if (M == 0) return;
    if (block_width <= 0) throw std::invalid_argument("clustering: block_width must be positive.");
    const char* where = std::getenv("XSPMM_CLUSTER_DEVICE");
    const bool gpu = where && std::strcmp(where, "gpu") == 0;
    if (gpu && clustering_device_supported(M, K, block_width)) {
        jaccard_clustering_device<I>(M, K, nnz, rp, ci, dist_thresh, block_width, d_perm, s, nullptr);
        return;
    }
    std::vector<I> h_rp((size_t)M + 1), h_ci((size_t)(nnz > 0 ? nnz : 1)), h_perm((size_t)M);
    XSPMM_HIP_CHECK(hipMemcpyAsync(h_rp.data(), rp, sizeof(I) * (size_t)(M + 1),
                                   hipMemcpyDeviceToHost, s));
    if (nnz > 0)
        XSPMM_HIP_CHECK(hipMemcpyAsync(h_ci.data(), ci, sizeof(I) * (size_t)nnz,
                                       hipMemcpyDeviceToHost, s));
    XSPMM_HIP_CHECK(hipStreamSynchronize(s));
    jaccard_clustering_host<I>(M, K, h_rp.data(), h_ci.data(), dist_thresh, block_width,
                               h_perm.data(), 0);
    XSPMM_HIP_CHECK(hipMemcpyAsync(d_perm, h_perm.data(), sizeof(I) * (size_t)M,
                                   hipMemcpyHostToDevice, s));
    XSPMM_HIP_CHECK(hipStreamSynchronize(s));
}

template void jaccard_clustering_dispatch<int32_t>(int64_t, int64_t, int64_t, const int32_t*,
                                                   const int32_t*, float, int64_t, int32_t*,
                                                   hipStream_t);
template void jaccard_clustering_dispatch<int64_t>(int64_t, int64_t, int64_t, const int64_t*,
                                                   const int64_t*, float, int64_t, int64_t*,
                                                   hipStream_t);

template <typename T, typename I>
void spmm_pipeline(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const T* vals,
                   const T* B, float* C, int64_t N, int64_t hw, bool optimize_pattern,
                   double* tm, hipStream_t s)
{
    if (M < 0 || K < 0 || nnz < 0 || N < 0)
        throw std::invalid_argument("CSR dimensions must be non-negative.");
    if (hw != 16)
        throw std::invalid_argument("xSpMM: the MFMA tile kernel requires hw_block_size == 16.");
    const bool timed = tm != nullptr;
    StageTimer total(timed, s), step(timed, s);
    total.start();
    const int64_t Mb = (M + 15) / 16, Kb = (K + 15) / 16;

    // Every temporary is taken before the first stage, so the stage times
    // hold the stages' own work, except exactly sized BCSR arrays, which the
    // conversion stage takes once it has read the block count.  The bound
    // min(nnz, Mb * Kb) on the block count holds since each block holds an
    // entry.
    const int64_t cap = std::max<int64_t>(1, std::min<int64_t>(nnz, Mb * Kb));
    const bool fused = (size_t)cap * 256 * sizeof(T) <= kFusedConversionBytes;
    // all in one allocation
    Carve cv;
    size_t o_perm = 0, o_nrp = 0, o_nci = 0, o_nvals = 0, o_ctmp = 0;
    if (optimize_pattern) {
        o_perm = cv.take((size_t)(M > 0 ? M : 1) * sizeof(I));
        o_nrp = cv.take((size_t)(M + 1) * sizeof(I));
        o_nci = cv.take((size_t)(nnz > 0 ? nnz : 1) * sizeof(I));
        o_nvals = cv.take((size_t)(nnz > 0 ? nnz : 1) * sizeof(T));
        o_ctmp = cv.take((size_t)(M > 0 ? M : 1) * (size_t)(N > 0 ? N : 1) * sizeof(float));
    }
    const size_t o_brp = cv.take((size_t)(Mb + 1) * sizeof(I));
    const size_t o_err = cv.take(sizeof(int));
    const size_t o_bci = fused ? cv.take((size_t)cap * sizeof(I)) : 0;
    const size_t o_bvals = fused ? cv.take((size_t)cap * 256 * sizeof(T)) : 0;
    Scratch tmp(cv.end, s);
    g_last_temp_bytes = cv.end;
    char* const base = tmp.as<char>();
    const Piece d_perm{base + o_perm}, nrp{base + o_nrp}, nci{base + o_nci}, nvals{base + o_nvals},
        c_tmp{base + o_ctmp}, brp{base + o_brp}, err{base + o_err};
    Piece bci{base + o_bci}, bvals{base + o_bvals};
    Scratch blocks;  // exactly sized BCSR arrays (when not fused)

    // the stage's CSR: the caller's, or the permuted copy
    const I* crp = rp;
    const I* cci = ci;
    const T* cvals = vals;
    if (optimize_pattern) {
        // 1. Clustering.
        step.start();
        jaccard_clustering_dispatch<I>(M, K, nnz, rp, ci, 0.5f, hw, d_perm.as<I>(), s);
        if (timed) step.stop(&tm[0]);

        // 2. Permutation.
        step.start();
        apply_permutation<T, I>(M, nnz, rp, ci, vals, d_perm.as<I>(), nrp.as<I>(), nci.as<I>(),
                                nvals.as<T>(), s);
        if (timed) step.stop(&tm[1]);
        crp = nrp.as<I>();
        cci = nci.as<I>();
        cvals = nvals.as<T>();
    }

    // 3. Conversion (the fill writes nothing if the count finds invalid input).
    step.start();
    csr_to_bcsr_count_async<I>(M, K, nnz, crp, cci, 16, 16, brp.as<I>(), err.as<int>(), s);
    int64_t nnzb = 0;
    if (!fused) {
        nnzb = csr_to_bcsr_result<I>(brp.as<I>(), Mb, err.as<int>(), s);
        Carve bc;
        const size_t o_ci = bc.take((size_t)(nnzb > 0 ? nnzb : 1) * sizeof(I));
        const size_t o_v = bc.take((size_t)(nnzb > 0 ? nnzb : 1) * 256 * sizeof(T));
        blocks = Scratch(bc.end, s);
        g_last_temp_bytes += bc.end;
        bci = Piece{blocks.as<char>() + o_ci};
        bvals = Piece{blocks.as<char>() + o_v};
    }
    csr_to_bcsr_fill<T, I>(M, K, nnz, crp, cci, cvals, 16, 16, brp.as<I>(), bci.as<I>(),
                           bvals.as<T>(), s, err.as<int>());
    if (timed) step.stop(&tm[2]);
    if (fused) nnzb = csr_to_bcsr_result<I>(brp.as<I>(), Mb, err.as<int>(), s);

    if (optimize_pattern) {
        // 4. SpMM into the permuted-order temporary.
        step.start();
        bcsr_spmm<T, I>(M, K, Mb, Kb, nnzb, brp.as<I>(), bci.as<I>(), bvals.as<T>(), B,
                        c_tmp.as<float>(), N, s);
        if (timed) step.stop(&tm[3]);

        // 5. Un-permutation.
        step.start();
        unpermute_dense<I>(c_tmp.as<float>(), C, d_perm.as<I>(), M, N, s);
        if (timed) step.stop(&tm[4]);
    } else {
        step.start();
        bcsr_spmm<T, I>(M, K, Mb, Kb, nnzb, brp.as<I>(), bci.as<I>(), bvals.as<T>(), B, C, N, s);
        if (timed) step.stop(&tm[3]);
    }
    if (timed) total.stop(&tm[5]);
    XSPMM_HIP_CHECK(hipStreamSynchronize(s));
    step.finish();
    total.finish();
}

#define XSPMM_INST_PIPE(T, I)                                                                 \
    template void spmm_pipeline<T, I>(int64_t, int64_t, int64_t, const I*, const I*, const T*, \
                                      const T*, float*, int64_t, int64_t, bool, double*,       \
                                      hipStream_t);
XSPMM_INST_PIPE(uint16_t, int32_t)
XSPMM_INST_PIPE(uint16_t, int64_t)
XSPMM_INST_PIPE(float, int32_t)
XSPMM_INST_PIPE(float, int64_t)
#undef XSPMM_INST_PIPE

}  // namespace detail
}  // namespace xspmm
