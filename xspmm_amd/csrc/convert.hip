// convert.hip -- CSR -> BCSR on the GPU, bit-exact with the reference's host
// conversion (src/core/conversion.cpp:8-100).
//
// Layout produced (identical to the reference):
//   Mb = ceil(M/r), Kb = ceil(K/c); bcsr_row_ptr = running block counts;
//   per block-row the distinct column blocks col/c in ascending order;
//   each block r x c row-major, zero-filled, entry (row, col) at
//   (block * r + row % r) * c + col % c; for duplicate (row, col) entries the
//   last one in CSR order wins.
//
// One 256-thread workgroup per block-row ("strip") of r CSR rows:
//   count: mark the strip's column blocks in an LDS bitmap (atomicOr), popcount
//          -> blocks per strip; a device scan turns counts into bcsr_row_ptr.
//   fill:  rebuild the bitmap, exclusive popcount prefix per 32-bit word gives
//          each column block its rank in the strip (= position among the sorted
//          block columns); emit col_ind from the set bits, zero the strip's
//          value blocks, then scatter every entry to its slot.  A strip whose
//          rows are all strictly increasing in column cannot hold duplicates and
//          is scattered with all threads; otherwise one thread walks each row in
//          order so the last duplicate wins.
#include "internal.hpp"
#include "scan.hpp"

namespace xspmm {
namespace detail {

namespace {

constexpr int kThreads = 256;
constexpr int64_t kMaxStripRows = 1024;
constexpr size_t kMaxLds = 64 * 1024;

struct StripView {
    int64_t* bounds;  // [nr+1] row starts of the strip (clamped to [0, nnz])
    int64_t nr;
};

// Does a new row start at entry q (q in (bounds[0], bounds[nr]])?
__device__ __forceinline__ bool row_starts_at(const StripView& sv, int64_t q)
{
    int64_t lo = 0, hi = sv.nr;  // lower_bound over bounds[0..nr]
    while (lo < hi) {
        const int64_t mid = (lo + hi) >> 1;
        if (sv.bounds[mid] < q) lo = mid + 1; else hi = mid;
    }
    return lo <= sv.nr && sv.bounds[lo] == q;
}

// Row (0..nr-1) within the strip that holds entry q.
__device__ __forceinline__ int64_t row_of(const StripView& sv, int64_t q)
{
    int64_t lo = 0, hi = sv.nr;  // last j with bounds[j] <= q
    while (lo < hi) {
        const int64_t mid = (lo + hi + 1) >> 1;
        if (sv.bounds[mid] <= q) lo = mid; else hi = mid - 1;
    }
    return lo;
}

// Loads the strip's row bounds, clears the bitmap, then marks column blocks.
// Returns via shared flags whether the strip is strictly sorted and valid.
template <typename I>
__device__ void build_strip_bitmap(int64_t M, int64_t K, int64_t nnz, const I* __restrict__ rp,
                                   const I* __restrict__ ci, int64_t rb, int64_t cb,
                                   int64_t nwords, StripView& sv, uint32_t* bitmap,
                                   int* s_unsorted, int* s_bad)
{
    const int64_t br = blockIdx.x;
    const int64_t r0 = br * rb;
    const int64_t r1 = (r0 + rb < M) ? r0 + rb : M;
    sv.nr = r1 - r0;
    if (threadIdx.x == 0) {
        *s_unsorted = 0;
        *s_bad = 0;
    }
    for (int64_t i = threadIdx.x; i <= sv.nr; i += kThreads) {
        int64_t v = (int64_t)rp[r0 + i];
        if (v < 0 || v > nnz) {
            *s_bad = 1;
            v = v < 0 ? 0 : nnz;
        }
        sv.bounds[i] = v;
    }
    for (int64_t w = threadIdx.x; w < nwords; w += kThreads) bitmap[w] = 0u;
    __syncthreads();
    for (int64_t i = threadIdx.x; i < sv.nr; i += kThreads)
        if (sv.bounds[i + 1] < sv.bounds[i]) *s_bad = 1;
    __syncthreads();
    if (*s_bad) return;  // uniform: every thread sees the same flag

    const int64_t e0 = sv.bounds[0];
    const int64_t e1 = sv.bounds[sv.nr];
    for (int64_t idx = e0 + threadIdx.x; idx < e1; idx += kThreads) {
        const int64_t c = (int64_t)ci[idx];
        if (c < 0 || c >= K) {
            *s_bad = 1;
            continue;
        }
        const int64_t bc = c / cb;
        atomicOr(&bitmap[bc >> 5], 1u << (bc & 31));
        if (idx + 1 < e1 && !row_starts_at(sv, idx + 1)) {
            if ((int64_t)ci[idx + 1] <= c) *s_unsorted = 1;
        }
    }
    __syncthreads();
}

template <typename I>
__global__ __launch_bounds__(kThreads) void conv_count_kernel(int64_t M, int64_t K, int64_t nnz,
                                                              const I* __restrict__ rp,
                                                              const I* __restrict__ ci,
                                                              int64_t rb, int64_t cb,
                                                              int64_t nwords, I* __restrict__ counts,
                                                              int* __restrict__ err)
{
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int s_unsorted, s_bad;
    __shared__ int64_t red[kThreads / 64];
    StripView sv;
    sv.bounds = reinterpret_cast<int64_t*>(smem);
    uint32_t* bitmap = reinterpret_cast<uint32_t*>(sv.bounds + rb + 1);
    build_strip_bitmap(M, K, nnz, rp, ci, rb, cb, nwords, sv, bitmap, &s_unsorted, &s_bad);
    int64_t cnt = 0;
    for (int64_t w = threadIdx.x; w < nwords; w += kThreads) cnt += __popc(bitmap[w]);
    const int64_t total = block_sum(cnt, red);
    if (threadIdx.x == 0) {
        counts[blockIdx.x] = (I)total;
        if (s_bad) atomicOr(err, 1);
    }
}

// err (nullable): the count pass's flag; when it is set (a strip held an
// invalid row_ptr or column) no strip writes anything, so a BCSR buffer sized
// from the bound min(nnz, Mb * Kb) is never overrun by offsets that a
// malformed row_ptr can produce.
template <typename T, typename I>
__global__ __launch_bounds__(kThreads) void conv_fill_kernel(
    int64_t M, int64_t K, int64_t nnz, const I* __restrict__ rp, const I* __restrict__ ci,
    const T* __restrict__ vals, int64_t rb, int64_t cb, int64_t nwords,
    const I* __restrict__ brp, I* __restrict__ bci, T* __restrict__ bvals,
    const int* __restrict__ err)
{
    if (err && *err) return;  // uniform: before any barrier
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int s_unsorted, s_bad;
    __shared__ int64_t red[kThreads / 64];
    StripView sv;
    sv.bounds = reinterpret_cast<int64_t*>(smem);
    uint32_t* bitmap = reinterpret_cast<uint32_t*>(sv.bounds + rb + 1);
    uint32_t* prefix = bitmap + nwords;
    build_strip_bitmap(M, K, nnz, rp, ci, rb, cb, nwords, sv, bitmap, &s_unsorted, &s_bad);
    if (s_bad) return;

    // Exclusive popcount prefix over words; each thread owns a contiguous run.
    const int64_t per = (nwords + kThreads - 1) / kThreads;
    const int64_t w0 = (int64_t)threadIdx.x * per;
    const int64_t w1 = (w0 + per < nwords) ? w0 + per : nwords;
    int64_t mine = 0;
    for (int64_t w = w0; w < w1; ++w) mine += __popc(bitmap[w]);
    int64_t total;
    int64_t run = block_exclusive_scan(mine, &total, red);
    for (int64_t w = w0; w < w1; ++w) {
        prefix[w] = (uint32_t)run;
        run += __popc(bitmap[w]);
    }

    const int64_t br = blockIdx.x;
    const int64_t base = (int64_t)brp[br];
    const int64_t nb = (int64_t)brp[br + 1] - base;
    if (nb != total) return;  // row_ptr does not describe this matrix: write nothing

    // col_ind: set bits in ascending order.
    for (int64_t w = w0; w < w1; ++w) {
        uint32_t bits = bitmap[w];
        int64_t o = base + prefix[w];
        while (bits) {
            const int b = __ffs(bits) - 1;
            bci[o++] = (I)(w * 32 + b);
            bits &= bits - 1;
        }
    }

    // Zero the strip's blocks.
    const int64_t bsz = rb * cb;
    T* out = bvals + base * bsz;
    const int64_t nel = nb * bsz;
    const size_t bytes = (size_t)nel * sizeof(T);
    if ((reinterpret_cast<uintptr_t>(out) & 15) == 0 && (bytes & 15) == 0) {
        uint4* o4 = reinterpret_cast<uint4*>(out);
        const int64_t n4 = (int64_t)(bytes >> 4);
        for (int64_t i = threadIdx.x; i < n4; i += kThreads) o4[i] = make_uint4(0, 0, 0, 0);
    } else {
        for (int64_t i = threadIdx.x; i < nel; i += kThreads) out[i] = T(0);
    }
    __syncthreads();  // zero stores complete before any scatter store below

    auto place = [&](int64_t idx, int64_t r_in) {
        const int64_t c = (int64_t)ci[idx];
        const int64_t bc = c / cb;
        const int64_t w = bc >> 5;
        const uint32_t below = bitmap[w] & ((1u << (bc & 31)) - 1u);
        const int64_t rank = (int64_t)prefix[w] + __popc(below);
        out[rank * bsz + r_in * cb + (c - bc * cb)] = vals[idx];
    };
    const int64_t e0 = sv.bounds[0];
    const int64_t e1 = sv.bounds[sv.nr];
    if (!s_unsorted) {
        for (int64_t idx = e0 + threadIdx.x; idx < e1; idx += kThreads) place(idx, row_of(sv, idx));
    } else {
        for (int64_t r = threadIdx.x; r < sv.nr; r += kThreads)
            for (int64_t idx = sv.bounds[r]; idx < sv.bounds[r + 1]; ++idx) place(idx, r);
    }
}

struct ConvGeometry {
    int64_t Mb, Kb, nwords;
    size_t count_lds, fill_lds;
};

ConvGeometry conv_geometry(int64_t M, int64_t K, int64_t nnz, int64_t rb, int64_t cb)
{
    if (M < 0 || K < 0 || nnz < 0)
        throw std::invalid_argument("CSR dimensions must be non-negative.");
    if (rb <= 0 || cb <= 0) throw std::invalid_argument("csr_to_bcsr: block sizes must be positive.");
    if (rb > kMaxStripRows)
        throw std::invalid_argument("csr_to_bcsr: r_block above 1024 is not supported on the GPU.");
    ConvGeometry g;
    g.Mb = (M + rb - 1) / rb;
    g.Kb = (K + cb - 1) / cb;
    g.nwords = (g.Kb + 31) / 32;
    if (g.nwords == 0) g.nwords = 1;
    const size_t bounds = (size_t)(rb + 1) * sizeof(int64_t);
    g.count_lds = bounds + (size_t)g.nwords * 4;
    g.fill_lds = bounds + (size_t)g.nwords * 8;
    if (g.fill_lds > kMaxLds)
        throw std::invalid_argument("csr_to_bcsr: too many column blocks for the GPU conversion "
                                    "(needs ceil(K/c) <= 261600 for r = 16).");
    if (g.Mb > 0x7fffffffLL) throw std::invalid_argument("csr_to_bcsr: too many block-rows.");
    return g;
}

}  // namespace

template <typename I>
int64_t csr_to_bcsr_count(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                          int64_t rb, int64_t cb, I* brp, hipStream_t s)
{
    const ConvGeometry g = conv_geometry(M, K, nnz, rb, cb);  // argument checks first
    Scratch err(sizeof(int), s);
    csr_to_bcsr_count_async<I>(M, K, nnz, rp, ci, rb, cb, brp, err.as<int>(), s);
    return csr_to_bcsr_result<I>(brp, g.Mb, err.as<int>(), s);
}

template <typename I>
void csr_to_bcsr_count_async(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                             int64_t rb, int64_t cb, I* brp, int* err, hipStream_t s)
{
    const ConvGeometry g = conv_geometry(M, K, nnz, rb, cb);
    Scratch counts((size_t)(g.Mb > 0 ? g.Mb : 1) * sizeof(I), s);
    hipLaunchKernelGGL(set_value_kernel<int>, dim3(1), dim3(64), 0, s, err, 0);
    XSPMM_LAUNCH_CHECK();
    if (g.Mb > 0) {
        hipLaunchKernelGGL(conv_count_kernel<I>, dim3((unsigned)g.Mb), dim3(kThreads), g.count_lds,
                           s, M, K, nnz, rp, ci, rb, cb, g.nwords, counts.as<I>(), err);
        XSPMM_LAUNCH_CHECK();
    }
    device_exclusive_scan(ArrayValue<I>{counts.as<I>()}, g.Mb, brp, s);
}

template <typename I>
int64_t csr_to_bcsr_result(const I* brp, int64_t Mb, const int* err, hipStream_t s)
{
    I nnzb = 0;
    int bad = 0;
    XSPMM_HIP_CHECK(hipMemcpyAsync(&nnzb, brp + Mb, sizeof(I), hipMemcpyDeviceToHost, s));
    XSPMM_HIP_CHECK(hipMemcpyAsync(&bad, err, sizeof(int), hipMemcpyDeviceToHost, s));
    XSPMM_HIP_CHECK(hipStreamSynchronize(s));
    if (bad)
        throw std::invalid_argument(
            "csr_to_bcsr: invalid CSR (column index outside [0, K) or bad row_ptr).");
    return (int64_t)nnzb;
}

template <typename T, typename I>
void csr_to_bcsr_fill(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                      const T* vals, int64_t rb, int64_t cb, const I* brp, I* bci, T* bvals,
                      hipStream_t s, const int* err)
{
    const ConvGeometry g = conv_geometry(M, K, nnz, rb, cb);
    if (g.Mb == 0) return;
    hipLaunchKernelGGL((conv_fill_kernel<T, I>), dim3((unsigned)g.Mb), dim3(kThreads), g.fill_lds,
                       s, M, K, nnz, rp, ci, vals, rb, cb, g.nwords, brp, bci, bvals, err);
    XSPMM_LAUNCH_CHECK();
}

#define XSPMM_INST_COUNT(I)                                                                      \
    template int64_t csr_to_bcsr_count<I>(int64_t, int64_t, int64_t, const I*, const I*, int64_t, \
                                          int64_t, I*, hipStream_t);                             \
    template void csr_to_bcsr_count_async<I>(int64_t, int64_t, int64_t, const I*, const I*,      \
                                             int64_t, int64_t, I*, int*, hipStream_t);           \
    template int64_t csr_to_bcsr_result<I>(const I*, int64_t, const int*, hipStream_t);
XSPMM_INST_COUNT(int32_t)
XSPMM_INST_COUNT(int64_t)
#undef XSPMM_INST_COUNT
#define XSPMM_INST_FILL(T, I)                                                                    \
    template void csr_to_bcsr_fill<T, I>(int64_t, int64_t, int64_t, const I*, const I*,         \
                                         const T*, int64_t, int64_t, const I*, I*, T*,          \
                                         hipStream_t, const int*);
XSPMM_INST_FILL(uint16_t, int32_t)
XSPMM_INST_FILL(uint16_t, int64_t)
XSPMM_INST_FILL(float, int32_t)
XSPMM_INST_FILL(float, int64_t)
#undef XSPMM_INST_FILL

}  // namespace detail
}  // namespace xspmm
