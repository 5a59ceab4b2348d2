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
//
// Products that the packed kernels cover take a third form: the conversion
// writes column batches (csr_pack_analyse / csr_pack_emit in convert.hip)
// instead of padded blocks, and a packed product multiplies them, its store
// writing product row r to C row perm[r] (un-permutation fused; no C_temp).
// fp16: the batches the BCSR column-batch kernel would form, multiplied by
// spmm_f16_packed, so C is the BCSR form's bit for bit.  fp32: a strip's
// non-zero columns four at a time, multiplied by spmm_f32_packed (the same
// products summed in another order).  The batch arrays are sized from a
// bound (csr_pack_batch_bound) so the conversion is queued without a host
// round trip; the device decides whether the form is taken (sorted input,
// for fp16 finite, whose batches save a quarter of the block bytes), and when
// it is not, the host converts to BCSR at the exact size (the count is then
// known), inside the unused batch arrays when they hold it, else in a new
// allocation after releasing them.  Bound-sized batch arrays above 256 MiB
// are not taken: the host reads the status first and sizes the batches (or
// the BCSR arrays) exactly.  XSPMM_PIPELINE_FORMAT=bcsr keeps the BCSR form.
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <limits>
#include <type_traits>
#include <vector>

#include "internal.hpp"

namespace xspmm {
namespace detail {

namespace {

// Largest bound-sized BCSR value array the fused conversion takes (above it,
// exact sizing after one host round trip).
constexpr size_t kFusedConversionBytes = size_t(1) << 30;

// Largest bound-sized batch arrays the packed conversion takes (above it,
// exact sizing after one host round trip): the bound can exceed the exact
// size many times over for dense blocks (17x for fp32 full blocks), and
// what the pipeline holds stays reserved in the device pool.  gnn's bound
// (184 MB fp16, 151 MB fp32) stays under it: its exact path costs about
// 100 us more (the host read and a new pool allocation).
constexpr size_t kPackedFusedBytes = size_t(256) << 20;

// Bytes of one packed column batch: fp16, its A' operand (1 KB) and 32 B-row
// indices; fp32, its A' operand (16 rows x 4 slots) and 4 B-row indices.
constexpr size_t kPackedBatchBytes = 1024 + 128;
constexpr size_t kPacked32BatchBytes = 256 + 16;

// Device bytes of the last pipeline call's temporaries on this thread, and
// whether it multiplied packed column batches.
thread_local size_t g_last_temp_bytes = 0;
thread_local bool g_last_packed = false;

}  // namespace

size_t last_pipeline_temp_bytes() { return g_last_temp_bytes; }
bool last_pipeline_packed() { return g_last_packed; }


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

// The pipeline converts into packed column batches when the packed kernel
// covers the product (the same rules as spmm_f16_packed's and
// spmm_f32_packed's), the strip kernels' LDS holds the column blocks, and
// XSPMM_PIPELINE_FORMAT is not "bcsr".
template <typename T>
bool packed_pipeline_covers(int64_t K, int64_t Mb, int64_t Kb, int64_t N, const void* B, const void* C)
{
    if (const char* e = std::getenv("XSPMM_PIPELINE_FORMAT"))
        if (std::strcmp(e, "bcsr") == 0) return false;
    if (N <= 0 || (N + 127) / 128 > 65535 || !csr_pack_covers(K)) return false;
    if constexpr (sizeof(T) == 2)
        return N % 8 == 0 && K * N * 2 <= (int64_t(1) << 31) && N < (int64_t(1) << 22) &&
               spmm_f16_pack_supported(K, Mb, Kb);
    else
        return N % 4 == 0 && K * N * 4 <= (int64_t(1) << 31) && Mb <= 0x7fffffffLL &&
               (reinterpret_cast<uintptr_t>(B) & 15) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0;
}

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
    const int nw = spmm_batch_waves();

    // Products the packed kernels cover convert straight into packed column
    // batches (csr_pack_analyse / csr_pack_emit): no padded blocks are written
    // or read.  Strips with unsorted or duplicate columns, fp16 non-finite
    // values, fully populated grids and products whose batches would not save
    // a quarter of the block bytes take the BCSR path; the device decides,
    // and the host learns the outcome after the conversion's kernels are
    // queued.
    using V = std::conditional_t<sizeof(T) == 2, uint16_t, uint32_t>;  // value bits
    constexpr size_t kBatchBytes = sizeof(T) == 2 ? kPackedBatchBytes : kPacked32BatchBytes;
    constexpr size_t kBatchABytes = sizeof(T) == 2 ? 1024 : 256;  // A' operand of a batch
    const int pnw = sizeof(T) == 2 ? nw : 1;                         // batch counts per strip
    const bool try_packed = M > 0 && nnz > 0 && packed_pipeline_covers<T>(K, Mb, Kb, N, B, C);
    // The batch arrays are sized from csr_pack_batch_bound while that takes
    // at most kPackedFusedBytes (then the whole conversion is queued with no
    // host round trip), else exactly, after reading the count.
    const int64_t pbound =
        try_packed ? std::max<int64_t>(1, csr_pack_batch_bound(M, K, nnz, (int)sizeof(T))) : 0;
    const bool pfused = try_packed && (size_t)pbound * kBatchBytes <= kPackedFusedBytes;
    // Every temporary is taken before the first stage, so the stage times
    // hold the stages' own work, except arrays sized from a count the
    // conversion stage reads first (exactly sized BCSR arrays or batches).
    // The bound min(nnz, Mb * Kb) on the block count holds since each block
    // holds an entry.
    const int64_t cap = std::max<int64_t>(1, std::min<int64_t>(nnz, Mb * Kb));
    const bool fused = !try_packed && (size_t)cap * 256 * sizeof(T) <= kFusedConversionBytes;
    // all in one allocation
    Carve cv;
    size_t o_perm = 0, o_nrp = 0, o_nci = 0, o_nvals = 0, o_ctmp = 0;
    if (optimize_pattern) {
        o_perm = cv.take((size_t)(M > 0 ? M : 1) * sizeof(I));
        o_nrp = cv.take((size_t)(M + 1) * sizeof(I));
        o_nci = cv.take((size_t)(nnz > 0 ? nnz : 1) * sizeof(I));
        o_nvals = cv.take((size_t)(nnz > 0 ? nnz : 1) * sizeof(T));
        if (!try_packed)
            o_ctmp = cv.take((size_t)(M > 0 ? M : 1) * (size_t)(N > 0 ? N : 1) * sizeof(float));
    }
    const size_t o_brp = cv.take((size_t)(Mb + 1) * sizeof(I));
    const size_t o_err = cv.take(sizeof(int));
    const size_t o_bci = fused ? cv.take((size_t)cap * sizeof(I)) : 0;
    const size_t o_bvals = fused ? cv.take((size_t)cap * 256 * sizeof(T)) : 0;
    size_t o_bcounts = 0, o_counts = 0, o_offsets = 0, o_flags = 0, o_status = 0, o_order = 0;
    if (try_packed) {
        o_bcounts = cv.take((size_t)Mb * sizeof(I));
        o_counts = cv.take((size_t)Mb * pnw * sizeof(int32_t));
        o_offsets = cv.take((size_t)(Mb * pnw + 1) * sizeof(int64_t));
        o_flags = cv.take(sizeof(unsigned int));
        o_status = cv.take(5 * sizeof(int64_t));
        o_order = cv.take((size_t)Mb * sizeof(int32_t));
    }
    // Temporaries reported: the most held at once (the bound-sized batches
    // are released before a BCSR fallback takes its arrays).
    size_t live = 0;
    g_last_temp_bytes = 0;
    g_last_packed = false;
    auto took = [&](size_t bytes) {
        live += bytes;
        g_last_temp_bytes = std::max(g_last_temp_bytes, live);
    };
    Scratch tmp(cv.end, s);
    took(cv.end);
    // bound-sized batches: A' operands, then B-row indices
    Scratch pbatch(pfused ? (size_t)pbound * kBatchBytes : 0, s);
    took(pfused ? (size_t)pbound * kBatchBytes : 0);
    char* const base = tmp.as<char>();
    const Piece d_perm{base + o_perm}, nrp{base + o_nrp}, nci{base + o_nci}, nvals{base + o_nvals},
        brp{base + o_brp}, err{base + o_err};
    Piece c_tmp{base + o_ctmp}, bci{base + o_bci}, bvals{base + o_bvals};
    const Piece bcounts{base + o_bcounts}, counts{base + o_counts}, offsets{base + o_offsets},
        flags{base + o_flags}, status{base + o_status}, order{base + o_order};
    void* pa = pbatch.get();
    uint32_t* prows =
        pfused ? reinterpret_cast<uint32_t*>(pbatch.as<char>() + (size_t)pbound * kBatchABytes) : nullptr;
    Scratch blocks;  // exactly sized BCSR arrays or batches
    Scratch ctmp_late;

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
    int64_t nnzb = 0;
    bool packed = false;
    step.start();
    if (try_packed) {
        const V* vb = reinterpret_cast<const V*>(cvals);
        csr_pack_analyse<I, V>(M, K, nnz, crp, cci, vb, bcounts.as<I>(), brp.as<I>(), counts.as<int32_t>(),
                            offsets.as<int64_t>(), err.as<int>(), flags.as<unsigned int>(),
                            pfused ? pbound : std::numeric_limits<int64_t>::max() / 2048,
                            status.as<int64_t>(), s);
        if (pfused)
            csr_pack_emit<I, V>(M, K, nnz, crp, cci, vb, offsets.as<int64_t>(), status.as<int64_t>(),
                                pbound, pa, prows, s);
        if (spmm_order_wanted(Mb)) spmm_dispatch_order<I>(brp.as<I>(), Mb, order.as<int32_t>(), s);
        if (timed) step.stop(&tm[2]);
        const PackStatus st = csr_pack_status(status.as<int64_t>(), s);
        if (st.err)
            throw std::invalid_argument(
                "csr_to_bcsr: invalid CSR (column index outside [0, K) or bad row_ptr).");
        nnzb = st.nnzb;
        packed = st.go;
        if (packed && !pfused) {
            // exactly sized batches (the bracket adds to the conversion time)
            step.start();
            blocks = Scratch((size_t)st.nbatches * kBatchBytes, s);
            took((size_t)st.nbatches * kBatchBytes);
            pa = blocks.get();
            prows = reinterpret_cast<uint32_t*>(blocks.as<char>() + (size_t)st.nbatches * kBatchABytes);
            csr_pack_emit<I, V>(M, K, nnz, crp, cci, vb, offsets.as<int64_t>(), status.as<int64_t>(),
                                st.nbatches, pa, prows, s);
            if (timed) step.stop(&tm[2]);
        }
        if (!packed) {
            // the BCSR form, exactly sized from the count (the bracket adds
            // to the conversion time)
            step.start();
            Carve bc;
            const size_t o_ci = bc.take((size_t)(nnzb > 0 ? nnzb : 1) * sizeof(I));
            const size_t o_v = bc.take((size_t)(nnzb > 0 ? nnzb : 1) * 256 * sizeof(T));
            char* bb = nullptr;
            if (pfused && bc.end <= (size_t)pbound * kBatchBytes) {
                bb = pbatch.as<char>();  // the unused batch arrays hold them
            } else {
                if (pfused) {
                    pbatch = Scratch();
                    live -= (size_t)pbound * kBatchBytes;
                }
                blocks = Scratch(bc.end, s);
                took(bc.end);
                bb = blocks.as<char>();
            }
            bci = Piece{bb + o_ci};
            bvals = Piece{bb + o_v};
            csr_to_bcsr_fill<T, I>(M, K, nnz, crp, cci, cvals, 16, 16, brp.as<I>(), bci.as<I>(),
                                   bvals.as<T>(), s, err.as<int>());
            if (timed) step.stop(&tm[2]);
        }
    } else {
        csr_to_bcsr_count_async<I>(M, K, nnz, crp, cci, 16, 16, brp.as<I>(), err.as<int>(), s);
        if (!fused) {
            nnzb = csr_to_bcsr_result<I>(brp.as<I>(), Mb, err.as<int>(), s);
            Carve bc;
            const size_t o_ci = bc.take((size_t)(nnzb > 0 ? nnzb : 1) * sizeof(I));
            const size_t o_v = bc.take((size_t)(nnzb > 0 ? nnzb : 1) * 256 * sizeof(T));
            blocks = Scratch(bc.end, s);
            took(bc.end);
            bci = Piece{blocks.as<char>() + o_ci};
            bvals = Piece{blocks.as<char>() + o_v};
        }
        csr_to_bcsr_fill<T, I>(M, K, nnz, crp, cci, cvals, 16, 16, brp.as<I>(), bci.as<I>(),
                               bvals.as<T>(), s, err.as<int>());
        if (timed) step.stop(&tm[2]);
        if (fused) nnzb = csr_to_bcsr_result<I>(brp.as<I>(), Mb, err.as<int>(), s);
    }

    g_last_packed = packed;
    if (packed) {
        // 4 + 5. The packed product; with clustering its store writes product
        // row r to C row perm[r] (the un-permutation, fused: that stage's
        // time is not set).
        step.start();
        const int32_t* ord = spmm_order_wanted(Mb) ? order.as<int32_t>() : nullptr;
        const I* rmap = optimize_pattern ? d_perm.as<I>() : nullptr;
        bool ok;
        if constexpr (sizeof(T) == 2)
            ok = spmm_f16_packed<I>(M, K, Mb, offsets.as<int64_t>(), pa, prows,
                                    reinterpret_cast<const uint16_t*>(B), C, N, ord, rmap, s);
        else
            ok = spmm_f32_packed<I>(M, K, Mb, offsets.as<int64_t>(), pa, prows,
                                    reinterpret_cast<const float*>(B), C, N, ord, rmap, s);
        if (!ok) throw std::runtime_error("xSpMM: the packed product does not cover this shape.");
        if (timed) step.stop(&tm[3]);
    } else if (optimize_pattern) {
        if (try_packed) {
            ctmp_late = Scratch((size_t)M * (size_t)(N > 0 ? N : 1) * sizeof(float), s);
            took((size_t)M * (size_t)(N > 0 ? N : 1) * sizeof(float));
            c_tmp = Piece{ctmp_late.as<char>()};
        }
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
