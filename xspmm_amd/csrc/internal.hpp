// internal.hpp -- shared declarations of libxspmm.so (not installed).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>

#include "xspmm/core/executor.hpp"

#define XSPMM_HIP_CHECK(call)                                                          \
    do {                                                                               \
        hipError_t xspmm_err_ = (call);                                                \
        if (xspmm_err_ != hipSuccess) {                                                \
            throw std::runtime_error(std::string("HIP Error: ") +                      \
                                     hipGetErrorString(xspmm_err_) + " at " +          \
                                     __FILE__ + ":" + std::to_string(__LINE__));       \
        }                                                                              \
    } while (0)

// Check the launch status of the kernel just enqueued.
#define XSPMM_LAUNCH_CHECK() XSPMM_HIP_CHECK(hipGetLastError())

namespace xspmm {
namespace detail {

// Stream-ordered device scratch: allocated with hipMallocAsync on `s` and
// released with hipFreeAsync on `s` when it goes out of scope, so it may be
// dropped right after the kernels that use it are enqueued.
class Scratch {
public:
    Scratch() = default;
    Scratch(size_t bytes, hipStream_t s) : s_(s) {
        if (bytes) XSPMM_HIP_CHECK(hipMallocAsync(&p_, bytes, s));
    }
    ~Scratch() {
        if (p_) (void)hipFreeAsync(p_, s_);
    }
    Scratch(const Scratch&) = delete;
    Scratch& operator=(const Scratch&) = delete;
    Scratch(Scratch&& o) noexcept : p_(o.p_), s_(o.s_) { o.p_ = nullptr; }
    Scratch& operator=(Scratch&& o) noexcept {
        if (this != &o) {
            if (p_) (void)hipFreeAsync(p_, s_);
            p_ = o.p_;
            s_ = o.s_;
            o.p_ = nullptr;
        }
        return *this;
    }
    template <typename T>
    T* as() const { return static_cast<T*>(p_); }
    void* get() const { return p_; }

private:
    void* p_ = nullptr;
    hipStream_t s_ = nullptr;
};

// Keeps freed stream-ordered memory in the device pool instead of returning
// it to the driver at every synchronization (called once per device).
void init_device_pool(int device);

// ---------------------------------------------------------------------------
// Kernel launchers (all enqueue on `s`; none synchronizes unless stated).
// Index type I in {int32_t, int64_t}; value type tags: uint16_t = fp16 bits,
// float = fp32.
// ---------------------------------------------------------------------------

// Tier-1 BCSR SpMM with 16x16 blocks.  C[M x N] = A * B[K x N].
template <typename T, typename I>
void bcsr_spmm(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
               const I* bci, const T* bvals, const T* B, float* C, int64_t N, hipStream_t s);

// Tier-1 fp16 SpMM for a fully populated block grid (nnzb == Mb * Kb).
// Returns false (and launches nothing) when the shape is not covered.
bool bcsr_spmm_dense_f16(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb,
                         const uint16_t* bvals, const uint16_t* B, float* C, int64_t N,
                         hipStream_t s);

// CSR -> BCSR.  count writes brp[Mb+1] and returns nnzb (synchronizes `s`);
// it throws std::invalid_argument on an out-of-range column index.
template <typename I>
int64_t csr_to_bcsr_count(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                          int64_t rb, int64_t cb, I* brp, hipStream_t s);
template <typename T, typename I>
void csr_to_bcsr_fill(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                      const T* vals, int64_t rb, int64_t cb, const I* brp, I* bci, T* bvals,
                      hipStream_t s);

// Row permutation new row i = old row perm[i] (outputs caller-allocated).
template <typename T, typename I>
void apply_permutation(int64_t M, int64_t nnz, const I* rp, const I* ci, const T* vals,
                       const I* perm, I* nrp, I* nci, T* nvals, hipStream_t s);

// out[perm[r], :] = in[r, :] (M x N fp32).
template <typename I>
void unpermute_dense(const float* in, float* out, const I* perm, int64_t M, int64_t N,
                     hipStream_t s);

// Host Jaccard clustering (exact restatement of the reference's greedy).
template <typename I>
void jaccard_clustering_host(int64_t M, int64_t K, const I* rp, const I* ci, float dist_thresh,
                             int64_t block_width, I* perm, int nthreads);

// GPU Jaccard clustering on device CSR arrays; writes perm[M] on the device.
// The same permutation as jaccard_clustering_host.  Synchronizes `s`.
// engine_used (nullable, host) receives 0 (closed form), 1 (scan) or 2 (index).
template <typename I>
void jaccard_clustering_device(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                               float dist_thresh, int64_t block_width, I* perm, hipStream_t s,
                               int* engine_used);
// Whether the GPU engine covers the shape (M < 2^31, at most 524288 column
// blocks, row bitmaps within 16 GiB).
bool clustering_device_supported(int64_t M, int64_t K, int64_t block_width);

// Clustering of device CSR arrays into the device array d_perm: the host
// greedy on copies (the reference's placement), or the GPU engine when
// XSPMM_CLUSTER_DEVICE=gpu and the shape is within its limits.  Both give the
// same permutation.  Synchronizes `s`.
template <typename I>
void jaccard_clustering_dispatch(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                                 float dist_thresh, int64_t block_width, I* d_perm, hipStream_t s);

// Tier-2 pipeline on raw device pointers.  `timings` may be null; it points
// at six doubles laid out like SpMMTimings.
template <typename T, typename I>
void spmm_pipeline(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const T* vals,
                   const T* B, float* C, int64_t N, int64_t hw_block_size, bool optimize_pattern,
                   double* timings, hipStream_t s);

}  // namespace detail
}  // namespace xspmm
