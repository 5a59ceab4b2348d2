// internal.hpp -- shared declarations of libxspmm.so (not installed).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <stdexcept>
#include <string>
#include <vector>

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

// Keeps freed stream-ordered memory in the device pool instead of returning
// it to the driver at every synchronization (the default pool's release
// threshold; set once per device, before its first stream-ordered
// allocation).
void init_device_pool(int device);

// Stream-ordered device scratch: allocated with hipMallocAsync on `s` and
// released with hipFreeAsync on `s` when it goes out of scope, so it may be
// dropped right after the kernels that use it are enqueued.
class Scratch {
public:
    Scratch() = default;
    Scratch(size_t bytes, hipStream_t s) : s_(s) {
        if (bytes) {
            int dev = 0;
            XSPMM_HIP_CHECK(hipGetDevice(&dev));
            init_device_pool(dev);
            XSPMM_HIP_CHECK(hipMallocAsync(&p_, bytes, s));
        }
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

// Offsets of 256-byte aligned pieces of one allocation (one stream-ordered
// allocation costs less host time than several).
struct Carve {
    size_t end = 0;
    size_t take(size_t bytes)
    {
        const size_t at = (end + 255) & ~size_t(255);
        end = at + bytes;
        return at;
    }
};

// A piece of such an allocation
struct Piece {
    char* p;
    template <typename U>
    U* as() const { return reinterpret_cast<U*>(p); }
};

// A HIP event without timing, destroyed with its scope.
class EventHandle {
public:
    EventHandle() { XSPMM_HIP_CHECK(hipEventCreateWithFlags(&e_, hipEventDisableTiming)); }
    ~EventHandle() {
        if (e_) (void)hipEventDestroy(e_);
    }
    EventHandle(const EventHandle&) = delete;
    EventHandle& operator=(const EventHandle&) = delete;
    hipEvent_t get() const { return e_; }

private:
    hipEvent_t e_ = nullptr;
};

// Device memory for a launcher's temporaries.  Without a region it makes
// stream-ordered allocations (Scratch, released when the arena goes out of
// scope); given a fixed region (the allocation-free entry point's scratch
// array) it hands out 256-byte aligned pieces of it and throws
// std::invalid_argument when a request does not fit.  Launchers take every
// piece before they enqueue the first kernel that uses one, so a request
// that does not fit leaves nothing half done.
class TempArena {
public:
    explicit TempArena(hipStream_t s) : s_(s) {}
    TempArena(void* base, size_t bytes, hipStream_t s)
        : s_(s), base_(static_cast<char*>(base)), cap_(bytes) {}
    TempArena(const TempArena&) = delete;
    TempArena& operator=(const TempArena&) = delete;
    bool fixed() const { return base_ != nullptr; }
    size_t capacity() const { return cap_; }
    void* take(size_t bytes) {
        if (bytes == 0) return nullptr;
        if (!base_) {
            owned_.emplace_back(bytes, s_);
            return owned_.back().get();
        }
        const size_t at = (used_ + 255) & ~size_t(255);
        if (at > cap_ || bytes > cap_ - at)
            throw std::invalid_argument(
                "xSpMM: this product needs " + std::to_string(at + bytes) +
                " bytes of scratch; the allocation-free entry point has " + std::to_string(cap_) +
                " (use the allocating entry point for it).");
        used_ = at + bytes;
        return base_ + at;
    }
    template <typename T>
    T* take_as(size_t count) { return static_cast<T*>(take(count * sizeof(T))); }

private:
    hipStream_t s_;
    char* base_ = nullptr;
    size_t cap_ = 0, used_ = 0;
    std::vector<Scratch> owned_;
};

// Elapsed times of stages bracketed by HIP events on stream s.  start() and
// stop() only record the events, so the host goes on to the next stage
// while the GPU runs this one; finish() waits for the last stop and writes
// each stage's milliseconds (brackets stopped into one slot add up).  Host
// work inside a bracket still counts: the stop event is recorded after it,
// and the stream idles meanwhile.  A disabled timer does nothing.
class StageTimer {
public:
    StageTimer(bool on, hipStream_t s) : on_(on), s_(s) {}
    ~StageTimer() {
        for (auto& st : stages_) {
            (void)hipEventDestroy(st.a);
            (void)hipEventDestroy(st.b);
        }
    }
    StageTimer(const StageTimer&) = delete;
    StageTimer& operator=(const StageTimer&) = delete;
    void start() {
        if (!on_) return;
        Stage st;
        XSPMM_HIP_CHECK(hipEventCreate(&st.a));
        if (hipEventCreate(&st.b) != hipSuccess) {
            (void)hipEventDestroy(st.a);
            XSPMM_HIP_CHECK(hipGetLastError());
            throw std::runtime_error("HIP Error: hipEventCreate failed");
        }
        stages_.push_back(st);
        XSPMM_HIP_CHECK(hipEventRecord(st.a, s_));
    }
    void stop(double* out) {
        if (!on_ || stages_.empty()) return;
        Stage& st = stages_.back();
        XSPMM_HIP_CHECK(hipEventRecord(st.b, s_));
        st.out = out;
    }
    void finish() {
        for (auto& st : stages_)
            if (st.out) *st.out = 0.0;
        for (auto& st : stages_) {
            if (!st.out) continue;
            XSPMM_HIP_CHECK(hipEventSynchronize(st.b));
            float ms = 0.f;
            XSPMM_HIP_CHECK(hipEventElapsedTime(&ms, st.a, st.b));
            *st.out += (double)ms;
        }
    }

private:
    struct Stage {
        hipEvent_t a = nullptr, b = nullptr;
        double* out = nullptr;
    };
    bool on_;
    hipStream_t s_;
    std::vector<Stage> stages_;
};

// ---------------------------------------------------------------------------
// Kernel launchers (all enqueue on `s`; none synchronizes unless stated).
// Index type I in {int32_t, int64_t}; value type tags: uint16_t = fp16 bits,
// float = fp32.
// ---------------------------------------------------------------------------

// Tier-1 BCSR SpMM with 16x16 blocks.  C[M x N] = A * B[K x N].
template <typename T, typename I>
void bcsr_spmm(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
               const I* bci, const T* bvals, const T* B, float* C, int64_t N, hipStream_t s);

// Tier-1 with a precomputed dispatch order (null: built here when useful, see
// spmm_order_wanted) and an optional output row map: product row r is stored
// in C row row_map[r] (row_map a permutation of [0, M)).  Returns false and
// launches nothing when row_map is given but the selected kernel stores rows
// in place; the caller then un-permutes a temporary.
template <typename T, typename I>
bool bcsr_spmm_ex(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
                  const I* bci, const T* bvals, const T* B, float* C, int64_t N,
                  const int32_t* order, const I* row_map, hipStream_t s);
// Tier-1 with the band kernel of T (uint16_t: fp16, float: fp32) where its
// shape conditions hold, else as bcsr_spmm_ex with no order.  The band
// kernels are only correct when every block-row is one contiguous run of
// block columns (spmm_band_wanted checks).
template <typename T, typename I>
void bcsr_spmm_band(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp, const I* bci,
                    const T* bvals, const T* B, float* C, int64_t N, hipStream_t s);
// Tier-1 without any allocation: the temporaries come from a fixed device
// array of kNoAllocScratchBytes (one copy per GPU, shared by every call on
// it).  Throws std::invalid_argument when a product needs more.
constexpr size_t kNoAllocScratchBytes = size_t(8) << 20;
template <typename T, typename I>
void bcsr_spmm_noalloc(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
                       const I* bci, const T* bvals, const T* B, float* C, int64_t N,
                       hipStream_t s);
// Dispatch order of the column-batch kernels (fp16 and fp32), Mb block-row
// ids.  spmm_order_wanted: a grid long enough (more than 2048 block-rows)
// that Tier-1 orders it on every call that is given no order;
// spmm_dispatch_order writes that order (longest rows first).
// spmm_order_cols_wanted: a grid for which an order computed once per
// matrix may pay (at least 256 block-rows); spmm_dispatch_order_cols writes
// it into order[0 .. Mb] (Mb + 1 entries) and returns whether to use it:
// longest rows first above 2048 block-rows (true, asynchronous), else, from
// the block columns, a contiguous range of block-rows per XCD when the rows
// are short and neighbouring rows alike (true) or the identity (false,
// order not worth passing); below 2048 block-rows it synchronizes s.
bool spmm_order_wanted(int64_t Mb);
bool spmm_order_cols_wanted(int64_t Mb);
template <typename I>
void spmm_dispatch_order(const I* brp, int64_t Mb, int32_t* order, hipStream_t s);
template <typename I>
bool spmm_dispatch_order_cols(const I* brp, const I* bci, int64_t Mb, int32_t* order, hipStream_t s);

// Packed column batches (fp16): the batches the Tier-1 batch kernel forms
// for each (block-row, wave) -- their A' operands (1 KB each) and B-row
// indices (32 per batch) -- stored once so that later products stream them
// instead of the BCSR blocks.  count writes Mb * 4 batch counts (wave-major
// per row); fill writes the batches at the exclusive-scan offsets of those
// counts (Mb * 4 + 1 entries) into a (batches x 1 KB) and rows (batches x 32).
// spmm_f16_packed multiplies them (same C as bcsr_spmm_ex on the BCSR matrix,
// with the same order / row_map meaning); it returns false when N is not
// covered (N % 8 != 0 or too large).
bool spmm_f16_pack_supported(int64_t K, int64_t Mb, int64_t Kb);
// Waves per workgroup of the batch kernels: the batch counts and offsets
// hold this many entries per block-row.
int spmm_batch_waves();
// offsets[0..n] = exclusive scan of counts[0..n-1]; returns offsets[n]
// (synchronizes s).
int64_t spmm_f16_pack_offsets(const int32_t* counts, int64_t n, int64_t* offsets, hipStream_t s);
template <typename I>
void spmm_f16_pack_count(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                         const uint16_t* bvals, int32_t* counts, hipStream_t s);
template <typename I>
void spmm_f16_pack_fill(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                        const uint16_t* bvals, const int64_t* offsets, void* a, uint32_t* rows,
                        hipStream_t s);
template <typename I>
bool spmm_f16_packed(int64_t M, int64_t K, int64_t Mb, const int64_t* offsets, const void* a,
                     const uint32_t* rows, const uint16_t* B, float* C, int64_t N,
                     const int32_t* order, const I* row_map, hipStream_t s);

// Tier-1 fp32 column-batch SpMM (spmm_f32.hip): covers N % 4 == 0 with B and
// C 16-byte aligned, K * N * 4 <= 2^31 and Kb < 2^21 (XSPMM_F32_KERNEL=tile
// declines it); order and row_map as for bcsr_spmm_ex.
bool spmm_f32_batch_covers(int64_t K, int64_t Kb, int64_t N, const void* B, const void* C);
template <typename I>
void bcsr_spmm_f32_batch(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                         const float* bvals, const float* B, float* C, int64_t N,
                         const int32_t* order, const I* row_map, hipStream_t s);
// Packed fp32 column batches (csr_pack_emit with V = uint32_t): strip br's
// batches [offsets[br], offsets[br + 1]) (a multiple of 4), A' in a and row
// indices in rows; order and row_map as for bcsr_spmm_ex.  Returns false
// when the shape is not covered (N % 4 != 0, B, C or a not 16-byte aligned,
// K * N * 4 > 2^31).
template <typename I>
bool spmm_f32_packed(int64_t M, int64_t K, int64_t Mb, const int64_t* offsets, const void* a,
                     const uint32_t* rows, const float* B, float* C, int64_t N, const int32_t* order,
                     const I* row_map, hipStream_t s);

// Tier-1 fp16 SpMM for a fully populated block grid (nnzb == Mb * Kb);
// row_map (null: rows in place) as for bcsr_spmm_ex.  Each tile checks that
// its block-rows hold the canonical layout (block br * Kb + c has column c)
// and otherwise multiplies its blocks in stored order, so any block order
// gives the right C.  Returns false (and launches nothing) when the shape is
// not covered; spmm_dense_f16_covers tells in advance.
bool spmm_dense_f16_covers(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, int64_t N);
template <typename I>
bool bcsr_spmm_dense_f16(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb,
                         const I* brp, const I* bci, const uint16_t* bvals, const uint16_t* B,
                         float* C, int64_t N, hipStream_t s, const I* row_map);

// Tier-1 fp16 SpMM for grids whose block-rows are contiguous runs of block
// columns (banded grids): four neighbouring block-rows share each B tile.
// Only correct when every block-row is contiguous; spmm_band_f16_covers tells
// whether the shape is covered (false: nothing launched).
bool spmm_band_f16_covers(int64_t K, int64_t Kb, int64_t Mb, int64_t N);
// Tier-1 fp32 SpMM for banded grids (contiguous block-rows): four
// neighbouring block-rows per workgroup share each B load in registers.
// Grids of at most 4096 groups where one group per workgroup is predicted to
// leave CUs idle long enough run the balanced launch (a plan kernel, then
// equal shares of the groups' blocks per workgroup, cut groups summed in part
// order; stream-ordered scratch).  False (nothing
// launched) when the shape is not covered (N % 4 != 0, B or C not 16-byte
// aligned, K * N * 4 > 2^31).
bool spmm_band_f32_covers(int64_t K, int64_t Kb, int64_t Mb, int64_t N, const void* B, const void* C);
template <typename I>
bool bcsr_spmm_band_f32(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                        const float* bvals, const float* B, float* C, int64_t N, const I* row_map,
                        int64_t nnzb, hipStream_t s);
// Whether Tier-1 should take a band kernel for this grid of fp16
// (value_bytes 2) or fp32 (4) blocks: every block-row contiguous, the grid not
// full, the groups' spans gathering fewer B rows than the column-batch kernel
// would (nnz: CSR entries behind the grid, 0 if not known; N: a typical column
// count, 0 for 128), and for fp32 at least 16 blocks per block-row on average.
// Reads two counters back (synchronizes `s`).
template <typename I>
bool spmm_band_wanted(const I* brp, const I* bci, int64_t M, int64_t K, int64_t Mb, int64_t Kb,
                      int64_t nnz, int64_t nnzb, int64_t N, int value_bytes, hipStream_t s);
template <typename I>
bool bcsr_spmm_band_f16(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                        const uint16_t* bvals, const uint16_t* B, float* C, int64_t N,
                        const I* row_map, hipStream_t s);

// CSR -> BCSR.  count writes brp[Mb+1] and returns nnzb (synchronizes `s`);
// it throws std::invalid_argument on an out-of-range column index.
template <typename I>
int64_t csr_to_bcsr_count(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                          int64_t rb, int64_t cb, I* brp, hipStream_t s);
// The same count without waiting: brp[Mb+1] and the device flag *err (0 for a
// valid CSR) are written on `s`; csr_to_bcsr_result later reads nnzb and the
// flag back (synchronizing `s`) and throws as csr_to_bcsr_count does.
template <typename I>
void csr_to_bcsr_count_async(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                             int64_t rb, int64_t cb, I* brp, int* err, hipStream_t s);
template <typename I>
int64_t csr_to_bcsr_result(const I* brp, int64_t Mb, const int* err, hipStream_t s);
// Fill of bci[nnzb] and bvals[nnzb * rb * cb].  err (nullable): the count's
// flag; when set the fill writes nothing (used when the outputs are sized
// from the bound min(nnz, Mb * Kb) before nnzb is known).
template <typename T, typename I>
void csr_to_bcsr_fill(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                      const T* vals, int64_t rb, int64_t cb, const I* brp, I* bci, T* bvals,
                      hipStream_t s, const int* err = nullptr);

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

// Prepared Tier-2 product: clustering, permutation and conversion done once
// (plan.cpp); execute() runs the Tier-1 SpMM with the un-permutation fused
// or through a kept workspace.  Value type erased for the C ABI.
class PlanBase {
public:
    virtual ~PlanBase() = default;
    virtual void execute(const void* B, float* C, int64_t N, hipStream_t s) = 0;
    virtual int64_t num_blocks() const = 0;
    virtual int64_t num_block_rows() const = 0;
    virtual int64_t num_packed_batches() const = 0;  // -1 when not packed
    virtual bool clustered() const = 0;
    virtual const void* permutation() const = 0;  // device perm[M], or null
};
// Builds a plan on stream s (synchronizes it).  timings: null, or six doubles
// laid out like SpMMTimings; the clustering, permutation, conversion and total
// fields receive the preparation times.
template <typename T, typename I>
PlanBase* make_plan(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const T* vals,
                    int64_t hw_block_size, bool optimize_pattern, double* timings, hipStream_t s);

// MatrixMarket coordinate file read as the reference's reader does
// (mtx.cpp): CSR with int indices, float values.
struct MtxError : std::runtime_error {
    using std::runtime_error::runtime_error;
};
struct MtxData {
    int rows = 0, cols = 0;
    std::vector<int> row_ptr, col_ind;
    std::vector<float> values;
    std::vector<int> r, c;  // entries before sorting (emptied afterwards)
    std::vector<float> v;
};
MtxData read_matrix_market(const std::string& path);

// CSR -> packed column batches (convert.hip), formed from the CSR strips
// without padded blocks.  V = uint16_t: the fp16 batches that
// spmm_f16_packed multiplies (per (block-row, wave) chains, 1152 B per
// batch); V = uint32_t: the fp32 batches that spmm_f32_packed multiplies
// (one count per strip, a multiple of 4 batches, 272 B per batch).
// csr_pack_analyse: per strip its block count (bcounts[Mb]) and their
// exclusive scan (brp, Mb + 1 entries: the BCSR row_ptr), the batch counts
// (counts: Mb * spmm_batch_waves() for fp16, Mb for fp32) and their exclusive
// scan (offsets, one more entry), err (set for an invalid row_ptr or
// column), flags (2: a strip's row is not strictly increasing; 4, fp16 only:
// an Inf or NaN value) and status[5] = {batches, blocks, err, flags, go}:
// go is decided on the device (valid and sorted input, fp16 finite, not a
// fully populated grid, 1 .. cap batches that take at most three quarters of
// the padded blocks' bytes).  csr_pack_emit writes the batches (A' operands,
// then B-row indices, in a and rows, each holding cap batches) when go is
// set and nothing otherwise, so it can be queued before the host reads the
// status.  csr_pack_status copies the status to the host (one
// synchronization).  csr_pack_covers: the strip kernels' LDS holds
// ceil(K / 16) column blocks.  csr_pack_batch_bound: an upper bound on the
// batch count (fp16: the smaller of 2 nnz / 33 + min(Mb * waves, nnz) and
// Mb * ceil(Kb / 2); fp32: the smaller of nnz / 4 + 4 Mb and Mb (4 Kb + 4)).
struct PackStatus {
    int64_t nbatches, nnzb;
    int err;
    unsigned int flags;
    bool go;
};
bool csr_pack_covers(int64_t K);
int64_t csr_pack_batch_bound(int64_t M, int64_t K, int64_t nnz, int value_bytes);
template <typename I, typename V>
void csr_pack_analyse(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const V* vals,
                      I* bcounts, I* brp, int32_t* counts, int64_t* offsets, int* err,
                      unsigned int* flags, int64_t cap, int64_t* status, hipStream_t s);
PackStatus csr_pack_status(const int64_t* status, hipStream_t s);
template <typename I, typename V>
void csr_pack_emit(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const V* vals,
                   const int64_t* offsets, const int64_t* status, int64_t cap, void* a, uint32_t* rows,
                   hipStream_t s);

// Device bytes of the temporaries the last spmm_pipeline call on this thread
// took (0 before any call).
size_t last_pipeline_temp_bytes();
// Whether the last spmm_pipeline call on this thread multiplied packed column
// batches (else BCSR blocks).
bool last_pipeline_packed();

// Tier-2 pipeline on raw device pointers.  `timings` may be null; it points
// at six doubles laid out like SpMMTimings.
template <typename T, typename I>
void spmm_pipeline(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const T* vals,
                   const T* B, float* C, int64_t N, int64_t hw_block_size, bool optimize_pattern,
                   double* timings, hipStream_t s);

}  // namespace detail
}  // namespace xspmm
