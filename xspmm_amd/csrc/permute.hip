// permute.hip -- CSR row permutation and dense un-permutation (HBM-bound copies).
//
// apply_permutation (reference src/hip/mtx_permutation.hip:12-67 with kernels
// src/common/permutation.hpp:15-66): new row i = old row perm[i], entries of a
// row keep their order.  Here the new row_ptr is a device scan of the gathered
// row lengths (no separate lengths array, no host round trip), and the gather
// is flattened: each workgroup owns 32 consecutive new rows, i.e. one
// contiguous output range, and every thread copies output entries, locating
// its row by binary search over the workgroup's row starts held in LDS.
// Writes are fully coalesced; reads are contiguous within each source row.
//
// unpermute_dense (reference src/common/permutation.hpp:89-108):
// out[perm[r], :] = in[r, :], moved as 16-byte vectors when N and both
// pointers allow it.
#include "internal.hpp"
#include "scan.hpp"

namespace xspmm {
namespace detail {

namespace {

constexpr int kThreads = 256;
constexpr int kRowsPerGroup = 32;

template <typename I>
struct PermutedRowLength {
    const I* rp;
    const I* perm;
    int64_t M;
    int64_t nnz;
    __device__ int64_t operator()(int64_t i) const
    {
        const int64_t o = (int64_t)perm[i];
        if (o < 0 || o >= M) return 0;
        int64_t a = (int64_t)rp[o], b = (int64_t)rp[o + 1];
        a = a < 0 ? 0 : (a > nnz ? nnz : a);
        b = b < a ? a : (b > nnz ? nnz : b);
        return b - a;
    }
};

template <typename T, typename I>
__global__ __launch_bounds__(kThreads) void gather_rows_kernel(
    int64_t M, int64_t nnz, const I* __restrict__ rp, const I* __restrict__ ci,
    const T* __restrict__ vals, const I* __restrict__ perm, const I* __restrict__ nrp,
    I* __restrict__ nci, T* __restrict__ nvals)
{
    __shared__ int64_t s_start[kRowsPerGroup + 1];
    __shared__ int64_t s_src[kRowsPerGroup];
    const int64_t r0 = (int64_t)blockIdx.x * kRowsPerGroup;
    const int64_t nr = (M - r0 < kRowsPerGroup) ? M - r0 : kRowsPerGroup;
    for (int64_t t = threadIdx.x; t <= nr; t += kThreads) s_start[t] = (int64_t)nrp[r0 + t];
    for (int64_t t = threadIdx.x; t < nr; t += kThreads) {
        const int64_t o = (int64_t)perm[r0 + t];
        s_src[t] = (o >= 0 && o < M) ? (int64_t)rp[o] : 0;
    }
    __syncthreads();
    const int64_t q0 = s_start[0];
    const int64_t q1 = s_start[nr] < nnz ? s_start[nr] : nnz;
    for (int64_t q = q0 + threadIdx.x; q < q1; q += kThreads) {
        int64_t lo = 0, hi = nr - 1;  // last row with start <= q
        while (lo < hi) {
            const int64_t mid = (lo + hi + 1) >> 1;
            if (s_start[mid] <= q) lo = mid; else hi = mid - 1;
        }
        const int64_t src = s_src[lo] + (q - s_start[lo]);
        if (src >= 0 && src < nnz) {
            nci[q] = ci[src];
            nvals[q] = vals[src];
        }
    }
}

// Rows narrower than the workgroup are packed: a workgroup moves
// rows_per_group = floor(256 / w) whole rows of w = N/4 (or N) elements;
// wider rows use ceil(w / 256) workgroups per row.
template <typename V, typename I>
__global__ __launch_bounds__(kThreads) void unpermute_kernel(int64_t M, int64_t w,
                                                             int64_t rows_per_group,
                                                             int64_t groups_per_row,
                                                             const I* __restrict__ perm,
                                                             const V* __restrict__ in,
                                                             V* __restrict__ out)
{
    int64_t r, c;
    if (rows_per_group > 0) {
        const int t = threadIdx.x;
        const int64_t local = t / w;
        if (local >= rows_per_group) return;
        r = (int64_t)blockIdx.x * rows_per_group + local;
        c = t - local * w;
    } else {
        r = (int64_t)blockIdx.x / groups_per_row;
        c = ((int64_t)blockIdx.x - r * groups_per_row) * kThreads + threadIdx.x;
        if (c >= w) return;
    }
    if (r >= M) return;
    const int64_t dst = (int64_t)perm[r];
    if (dst < 0 || dst >= M) return;
    out[dst * w + c] = in[r * w + c];
}

template <typename V, typename I>
void launch_unpermute(const V* in, V* out, const I* perm, int64_t M, int64_t w, hipStream_t s)
{
    int64_t rpg = 0, gpr = 1, groups;
    if (w <= kThreads) {
        rpg = kThreads / w;
        groups = (M + rpg - 1) / rpg;
    } else {
        gpr = (w + kThreads - 1) / kThreads;
        groups = M * gpr;
    }
    if (groups > 0x7fffffffLL) throw std::invalid_argument("unpermute: matrix too large.");
    hipLaunchKernelGGL((unpermute_kernel<V, I>), dim3((unsigned)groups), dim3(kThreads), 0, s, M,
                       w, rpg, gpr, perm, in, out);
    XSPMM_LAUNCH_CHECK();
}

}  // namespace

template <typename T, typename I>
void apply_permutation(int64_t M, int64_t nnz, const I* rp, const I* ci, const T* vals,
                       const I* perm, I* nrp, I* nci, T* nvals, hipStream_t s)
{
    if (M < 0 || nnz < 0) throw std::invalid_argument("CSR dimensions must be non-negative.");
    device_exclusive_scan(PermutedRowLength<I>{rp, perm, M, nnz}, M, nrp, s);
    if (M == 0 || nnz == 0) return;
    const int64_t groups = (M + kRowsPerGroup - 1) / kRowsPerGroup;
    hipLaunchKernelGGL((gather_rows_kernel<T, I>), dim3((unsigned)groups), dim3(kThreads), 0, s, M,
                       nnz, rp, ci, vals, perm, nrp, nci, nvals);
    XSPMM_LAUNCH_CHECK();
}

template <typename I>
void unpermute_dense(const float* in, float* out, const I* perm, int64_t M, int64_t N,
                     hipStream_t s)
{
    if (M < 0 || N < 0) throw std::invalid_argument("unpermute: negative size.");
    if (M == 0 || N == 0) return;
    const bool vec = (N % 4 == 0) && ((reinterpret_cast<uintptr_t>(in) & 15) == 0) &&
                     ((reinterpret_cast<uintptr_t>(out) & 15) == 0);
    if (vec)
        launch_unpermute(reinterpret_cast<const float4*>(in), reinterpret_cast<float4*>(out), perm,
                         M, N / 4, s);
    else
        launch_unpermute(in, out, perm, M, N, s);
}

#define XSPMM_INST_PERM(T, I)                                                                 \
    template void apply_permutation<T, I>(int64_t, int64_t, const I*, const I*, const T*,    \
                                          const I*, I*, I*, T*, hipStream_t);
XSPMM_INST_PERM(uint16_t, int32_t)
XSPMM_INST_PERM(uint16_t, int64_t)
XSPMM_INST_PERM(float, int32_t)
XSPMM_INST_PERM(float, int64_t)
#undef XSPMM_INST_PERM
template void unpermute_dense<int32_t>(const float*, float*, const int32_t*, int64_t, int64_t,
                                       hipStream_t);
template void unpermute_dense<int64_t>(const float*, float*, const int64_t*, int64_t, int64_t,
                                       hipStream_t);

}  // namespace detail
}  // namespace xspmm
