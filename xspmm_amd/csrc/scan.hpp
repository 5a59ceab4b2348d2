// scan.hpp -- device-wide exclusive prefix sum of n values produced by a
// functor, written as out[0..n] (out[n] = total).  Reduce-then-scan over
// 2048-element tiles: tile sums -> one-workgroup scan of the sums -> tile scan.
// Used for bcsr_row_ptr (block counts per strip) and for the permuted
// row_ptr (row lengths gathered through perm).
#pragma once

#include "internal.hpp"

namespace xspmm {
namespace detail {

constexpr int kScanThreads = 256;
constexpr int kScanItems = 8;
constexpr int kScanTile = kScanThreads * kScanItems;

__device__ __forceinline__ int64_t wave_inclusive_scan(int64_t v)
{
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t t = __shfl_up(v, d, 64);
        if (lane >= d) v += t;
    }
    return v;
}

// Exclusive scan across a 256-thread workgroup; *total gets the sum.
// `red` is shared scratch of >= 4 int64.  Contains two barriers.
__device__ __forceinline__ int64_t block_exclusive_scan(int64_t v, int64_t* total, int64_t* red)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t incl = wave_inclusive_scan(v);
    if (lane == 63) red[wave] = incl;
    __syncthreads();
    int64_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kScanThreads / 64; ++w) {
        const int64_t x = red[w];
        if (w < wave) before += x;
        all += x;
    }
    __syncthreads();
    *total = all;
    return before + incl - v;
}

__device__ __forceinline__ int64_t block_sum(int64_t v, int64_t* red)
{
    int64_t total;
    (void)block_exclusive_scan(v, &total, red);
    return total;
}

template <typename F>
__global__ __launch_bounds__(kScanThreads) void scan_reduce_kernel(F f, int64_t n,
                                                                    int64_t* partials)
{
    __shared__ int64_t red[kScanThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kScanTile;
    int64_t sum = 0;
    for (int i = threadIdx.x; i < kScanTile; i += kScanThreads) {
        const int64_t idx = base + i;
        if (idx < n) sum += f(idx);
    }
    const int64_t total = block_sum(sum, red);
    if (threadIdx.x == 0) partials[blockIdx.x] = total;
}

// Exclusive scan of partials[0..nt) in place; partials[nt] = total.
// (A template so that every translation unit including this header shares
// one definition.)
template <int kUnused = 0>
__global__ __launch_bounds__(kScanThreads) void scan_partials_kernel(int64_t* partials,
                                                                      int64_t nt)
{
    __shared__ int64_t red[kScanThreads / 64];
    int64_t carry = 0;
    for (int64_t c = 0; c < nt; c += kScanThreads) {
        const int64_t idx = c + threadIdx.x;
        const int64_t v = idx < nt ? partials[idx] : 0;
        int64_t tot;
        const int64_t ex = block_exclusive_scan(v, &tot, red);
        if (idx < nt) partials[idx] = carry + ex;
        carry += tot;
    }
    if (threadIdx.x == 0) partials[nt] = carry;
}

template <typename F, typename I>
__global__ __launch_bounds__(kScanThreads) void scan_final_kernel(F f, int64_t n,
                                                                   const int64_t* partials, I* out)
{
    __shared__ int64_t red[kScanThreads / 64];
    const int64_t base = (int64_t)blockIdx.x * kScanTile + (int64_t)threadIdx.x * kScanItems;
    int64_t v[kScanItems];
    int64_t sum = 0;
#pragma unroll
    for (int e = 0; e < kScanItems; ++e) {
        v[e] = (base + e < n) ? f(base + e) : 0;
        sum += v[e];
    }
    int64_t tot;
    int64_t run = block_exclusive_scan(sum, &tot, red) + partials[blockIdx.x];
#pragma unroll
    for (int e = 0; e < kScanItems; ++e) {
        if (base + e < n) out[base + e] = (I)run;
        run += v[e];
    }
    if (blockIdx.x == gridDim.x - 1 && threadIdx.x == 0) out[n] = (I)partials[gridDim.x];
}

template <typename I>
__global__ void set_value_kernel(I* p, I v)
{
    if (threadIdx.x == 0 && blockIdx.x == 0) *p = v;
}

template <typename I>
struct ArrayValue {
    const I* a;
    __device__ int64_t operator()(int64_t i) const { return (int64_t)a[i]; }
};

// out[0..n] = exclusive prefix sums of f(0..n-1), out[n] = total.
template <typename F, typename I>
void device_exclusive_scan(F f, int64_t n, I* out, hipStream_t s)
{
    if (n <= 0) {
        hipLaunchKernelGGL(set_value_kernel<I>, dim3(1), dim3(64), 0, s, out, (I)0);
        XSPMM_LAUNCH_CHECK();
        return;
    }
    const int64_t nt = (n + kScanTile - 1) / kScanTile;
    Scratch partials((size_t)(nt + 1) * sizeof(int64_t), s);
    hipLaunchKernelGGL(scan_reduce_kernel<F>, dim3((unsigned)nt), dim3(kScanThreads), 0, s, f, n,
                       partials.as<int64_t>());
    XSPMM_LAUNCH_CHECK();
    hipLaunchKernelGGL(scan_partials_kernel<0>, dim3(1), dim3(kScanThreads), 0, s,
                       partials.as<int64_t>(), nt);
    XSPMM_LAUNCH_CHECK();
    hipLaunchKernelGGL((scan_final_kernel<F, I>), dim3((unsigned)nt), dim3(kScanThreads), 0, s, f,
                       n, partials.as<int64_t>(), out);
    XSPMM_LAUNCH_CHECK();
}

}  // namespace detail
}  // namespace xspmm
