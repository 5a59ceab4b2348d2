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
#include <algorithm>

#include "internal.hpp"
#include "scan.hpp"

namespace xspmm {
namespace detail {

namespace {

constexpr int kThreads = 256;
constexpr int64_t kMaxStripRows = 1024;
constexpr size_t kMaxLds = 64 * 1024;
constexpr int kEntryUnroll = 4;  // CSR entries per thread per loop step

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

    // kEntryUnroll entries per thread in flight; a bit already set is not
    // set again (in a dense block every bit is met once per row); the row
    // search runs only where the next column does not increase
    const int64_t e0 = sv.bounds[0];
    const int64_t e1 = sv.bounds[sv.nr];
    for (int64_t i0 = e0 + threadIdx.x; i0 < e1; i0 += (int64_t)kThreads * kEntryUnroll) {
        int64_t c[kEntryUnroll], cn[kEntryUnroll];
#pragma unroll
        for (int u = 0; u < kEntryUnroll; ++u) {
            const int64_t idx = i0 + (int64_t)u * kThreads;
            c[u] = idx < e1 ? (int64_t)ci[idx] : 0;
            cn[u] = idx + 1 < e1 ? (int64_t)ci[idx + 1] : 0;
        }
#pragma unroll
        for (int u = 0; u < kEntryUnroll; ++u) {
            const int64_t idx = i0 + (int64_t)u * kThreads;
            if (idx >= e1) continue;
            if (c[u] < 0 || c[u] >= K) {
                *s_bad = 1;
                continue;
            }
            const int64_t bc = cb == 16 ? c[u] >> 4 : c[u] / cb;
            const uint32_t bit = 1u << (bc & 31);
            if (!(bitmap[bc >> 5] & bit)) atomicOr(&bitmap[bc >> 5], bit);
            if (idx + 1 < e1 && cn[u] <= c[u] && !row_starts_at(sv, idx + 1)) *s_unsorted = 1;
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


// ---------------------------------------------------------------------------
// CSR -> packed column batches (the Tier-2 pipeline's fp16 form).
//
// The fp16 column-batch SpMM (spmm.hip) turns each block-row's BCSR blocks
// into column batches, and its pack mode stores them for
// spmm_f16_packed_kernel: per (block-row, wave) the batches the wave forms,
// each an A' operand (64 lanes x 16 bytes) and 32 B-row indices.  What the
// batches hold is fixed by A alone: block-row br's blocks are its distinct
// column blocks in ascending order, block pair j is blocks (2j, 2j+1), wave
// w takes pairs w, w + W, ... in order, a pair's set columns (a column is set
// when any of its 16 entries has non-zero fp16 bits) take slots in the pair
// mask's bit order, and a pair that does not fit the open batch's 32 slots
// closes it.  Two kernels form the same batches straight from the CSR
// strips, one workgroup per strip, with every per-block quantity in LDS:
//   pack_analyse_kernel  the strip's column-block bitmap and its popcount
//                        prefix (a block's rank), the pair words (column
//                        masks of blocks 2j and 2j+1), then per wave the
//                        batch walk, counting batches;
//   pack_scan_kernel     (one workgroup) scans the block counts -> brp and
//                        the batch counts -> offsets, and decides on the
//                        device whether the packed form is taken;
//   pack_emit_kernel     the same analysis again, the walk recording each
//                        pair's batch and first slot, then the strip's A'
//                        operands and B-row indices: cleared, then every
//                        used slot's B row and every entry's value stored.
// The result equals the pack mode's byte for byte when every strip's rows
// hold strictly increasing columns and every value is finite (the flags
// below report strips and values outside that, and the caller then keeps
// the BCSR path): A' then holds each set column's exact values, with +0.0
// where the pack mode's compaction turns -0.0 into +0.0.
//
// Batch count bound.  In one wave's walk with m batches of s_1 .. s_m slots
// (S in all), batch i closed because the next pair did not fit, so
// s_i + s_{i+1} >= 33 for i < m; summed, 2 S - s_1 - s_m >= 33 (m - 1), so
// m <= (2 S - 2) / 33 + 1.  Each slot holds a non-zero entry, so over all
// walks the batches number at most 2 nnz / 33 plus the walks with a batch
// (at most min(Mb * W, nnz)), and at most the pair count Mb * ceil(Kb / 2)
// (a batch holds at least one pair): csr_pack_batch_bound.

constexpr uint32_t kPackFlagUnsorted = 2;   // a strip's row is not strictly increasing
constexpr uint32_t kPackFlagNonFinite = 4;  // an Inf or NaN value
constexpr int kPackWalkUnroll = 8;

// the batch kernel's pair-mask bit of pair column pc (0 .. 31): lane group
// g = pc / 8 holds pair columns 8g .. 8g+7 as halves e; half 2d goes to bit
// 4g + d, half 2d + 1 to bit 16 + 4g + d
__device__ __forceinline__ uint32_t pair_bit(uint32_t pc)
{
    const uint32_t g = pc >> 3, e = pc & 7u;
    return 16u * (e & 1u) + 4u * g + (e >> 1);
}

// the pair column of pair-mask bit b (inverse of pair_bit)
__device__ __forceinline__ uint32_t bit_pair_col(uint32_t b)
{
    const uint32_t hb = b >> 4, g = (b >> 2) & 3u, d = b & 3u;
    return 8u * g + 2u * d + hb;
}

// the even bits of x (bit 2i -> bit i)
__device__ __forceinline__ uint32_t even_bits(uint32_t x)
{
    x &= 0x55555555u;
    x = (x | (x >> 1)) & 0x33333333u;
    x = (x | (x >> 2)) & 0x0f0f0f0fu;
    x = (x | (x >> 4)) & 0x00ff00ffu;
    return (x | (x >> 8)) & 0x0000ffffu;
}

// pair mask of a pair word m (bit c: column c of block 2j; bit 16 + c:
// column c of block 2j + 1): pair column pc = 8g + e has pair_bit(pc), which
// is bit 4g + e/2 of the even-e or the odd-e half.  A bit permutation, so
// popc(pair_mask(m)) == popc(m).
__device__ __forceinline__ uint32_t pair_mask(uint32_t m)
{
    return even_bits(m) | (even_bits(m >> 1) << 16);
}

// MFMA K position that carries batch slot s (inverse of the batch kernel's
// kslot: k = 8 (s' >> 2) + 4 h + (s' & 3), s = 16 h + s')
__device__ __forceinline__ uint32_t slot_kpos(uint32_t s)
{
    const uint32_t h = s >> 4, sp = s & 15u;
    return 8u * (sp >> 2) + 4u * h + (sp & 3u);
}

// LDS of the packed-form strip kernels (byte offsets): the strip's row
// bounds, the column-block bitmap and its per-word popcount prefix, the pair
// words; pack_emit_kernel adds each pair's batch info, the waves' first
// batch and each block's column block.
struct PackLds {
    uint32_t bitmap, prefix, pw, analyse_bytes, pinfo, ob, bcl, emit_bytes, sb, emit32_bytes;
};

__host__ __device__ inline PackLds pack_lds(int64_t Kb, int nw)
{
    const uint32_t nwords = (uint32_t)(Kb > 0 ? (Kb + 31) / 32 : 1);
    const uint32_t npc = (uint32_t)((Kb + 1) / 2 + 1);  // pair capacity
    PackLds L;
    L.bitmap = 17 * 8;
    L.prefix = L.bitmap + 4 * nwords;
    L.pw = L.prefix + 4 * nwords;
    L.analyse_bytes = L.pw + 4 * npc;
    L.pinfo = L.analyse_bytes;
    L.ob = (L.pinfo + 4 * npc + 7) & ~7u;
    L.bcl = L.ob + 8 * (uint32_t)(nw + 1);
    L.emit_bytes = (L.bcl + 2 * (uint32_t)(Kb > 0 ? Kb : 1) + 15) & ~15u;
    // fp32 emit: each block's first slot (one more entry for an odd count)
    L.sb = L.analyse_bytes;
    L.emit32_bytes = (L.sb + 4 * (uint32_t)((Kb > 0 ? Kb : 1) + 2) + 15) & ~15u;
    return L;
}

// Value bits of the packed forms: V = uint16_t (fp16) or uint32_t (fp32).
// A column of a block is set when one of its entries is: for fp16 when its
// bits are not 0 (the fp16 batch kernel's rule: -0.0 counts), for fp32 when
// it is not +-0 (a +-0 entry adds an exact zero to an fp32 sum that starts
// at +0).  Non-finite values are flagged for fp16 only (the fp16 form must
// equal the BCSR kernel's compaction bit for bit).
__device__ __forceinline__ bool pack_set(uint16_t v) { return v != 0u; }
__device__ __forceinline__ bool pack_set(uint32_t v) { return (v & 0x7fffffffu) != 0u; }
__device__ __forceinline__ bool pack_nonfinite(uint16_t v) { return (v & 0x7c00u) == 0x7c00u; }
__device__ __forceinline__ bool pack_nonfinite(uint32_t) { return false; }

// One strip's analysis, shared by the strip kernels: bitmap, prefix, *nb (the
// strip's block count) and the pair words (column masks of blocks 2j, 2j+1).
// Leaves *s_bad / *s_unsorted set for an invalid or unsorted strip (the pair
// words are then not formed) and *s_nonfinite for a flagged value.  Ends with
// a barrier.
template <typename I, typename V>
__device__ void pack_strip(int64_t M, int64_t K, int64_t nnz, const I* __restrict__ rp,
                           const I* __restrict__ ci, const V* __restrict__ vals,
                           int64_t nwords, unsigned char* smem, const PackLds& L, StripView& sv,
                           int* s_unsorted, int* s_bad, int* s_nonfinite, int64_t* red, int64_t* nb)
{
    uint32_t* bitmap = reinterpret_cast<uint32_t*>(smem + L.bitmap);
    uint32_t* prefix = reinterpret_cast<uint32_t*>(smem + L.prefix);
    uint32_t* pw = reinterpret_cast<uint32_t*>(smem + L.pw);
    sv.bounds = reinterpret_cast<int64_t*>(smem);
    if (threadIdx.x == 0) *s_nonfinite = 0;
    build_strip_bitmap(M, K, nnz, rp, ci, 16, 16, nwords, sv, bitmap, s_unsorted, s_bad);
    *nb = 0;
    if (*s_bad) return;  // uniform
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
    *nb = total;
    if (*s_unsorted) return;  // uniform (set before build_strip_bitmap's last barrier)
    const int64_t npairs = (total + 1) >> 1;
    for (int64_t j = threadIdx.x; j < npairs; j += kThreads) pw[j] = 0u;
    __syncthreads();  // prefix and cleared pair words before the ORs
    const int64_t e0 = sv.bounds[0];
    const int64_t e1 = sv.bounds[sv.nr];
    bool nonfinite = false;
    for (int64_t i0 = e0 + threadIdx.x; i0 < e1; i0 += (int64_t)kThreads * kEntryUnroll) {
        V v[kEntryUnroll];
        uint32_t c[kEntryUnroll];
#pragma unroll
        for (int u = 0; u < kEntryUnroll; ++u) {
            const int64_t idx = i0 + (int64_t)u * kThreads;
            v[u] = idx < e1 ? vals[idx] : (V)0;
            c[u] = idx < e1 ? (uint32_t)ci[idx] : 0u;
        }
#pragma unroll
        for (int u = 0; u < kEntryUnroll; ++u) {
            if (pack_nonfinite(v[u])) nonfinite = true;
            if (!pack_set(v[u])) continue;  // also the entries past the strip
            const uint32_t bc = c[u] >> 4;
            const uint32_t w = bc >> 5;
            const uint32_t rank = prefix[w] + (uint32_t)__popc(bitmap[w] & ((1u << (bc & 31u)) - 1u));
            const uint32_t bit = 1u << (16u * (rank & 1u) + (c[u] & 15u));
            if (!(pw[rank >> 1] & bit)) atomicOr(&pw[rank >> 1], bit);
        }
    }
    if (nonfinite) *s_nonfinite = 1;
    __syncthreads();
}

// One wave's batch walk over pairs t, t + nw, ... (< npairs): returns the
// wave's batch count; with Record, pinfo[j] = (batch << 6) | first slot for
// every pair with a set column.  The pair words are read kPackWalkUnroll
// ahead so that the LDS latency is paid once per group.
template <bool Record>
__device__ __forceinline__ uint32_t pack_walk(const uint32_t* pw, uint32_t* pinfo, int64_t t, int nw,
                                              int64_t npairs)
{
    uint32_t pending = 0, nbatch = 0;
    for (int64_t j0 = t; j0 < npairs; j0 += (int64_t)kPackWalkUnroll * nw) {
        uint32_t cnt[kPackWalkUnroll];
#pragma unroll
        for (int u = 0; u < kPackWalkUnroll; ++u) {
            const int64_t j = j0 + (int64_t)u * nw;
            cnt[u] = j < npairs ? (uint32_t)__popc(pw[j]) : 0u;
        }
#pragma unroll
        for (int u = 0; u < kPackWalkUnroll; ++u) {
            if (cnt[u] == 0u) continue;
            if (pending + cnt[u] > 32u) {
                ++nbatch;
                pending = 0;
            }
            if (Record) pinfo[j0 + (int64_t)u * nw] = (nbatch << 6) | pending;
            pending += cnt[u];
        }
    }
    return nbatch + (pending > 0u ? 1u : 0u);
}

// err: set for an invalid row_ptr or column (as the count pass does);
// bcounts[br] = the strip's block count; counts[br * nw + w] = wave w's
// batch count (0 for an unsorted strip); flags as above.
template <typename I>
__global__ __launch_bounds__(kThreads) void pack_analyse_kernel(
    int64_t M, int64_t K, int64_t nnz, const I* __restrict__ rp, const I* __restrict__ ci,
    const uint16_t* __restrict__ vals, int64_t nwords, int64_t Kb, int nw, I* __restrict__ bcounts,
    int32_t* __restrict__ counts, int* __restrict__ err, unsigned int* __restrict__ flags)
{
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int s_unsorted, s_bad, s_nonfinite;
    __shared__ int64_t red[kThreads / 64];
    const PackLds L = pack_lds(Kb, nw);
    StripView sv;
    int64_t nb;
    pack_strip(M, K, nnz, rp, ci, vals, nwords, smem, L, sv, &s_unsorted, &s_bad, &s_nonfinite, red, &nb);
    const int64_t br = blockIdx.x;
    if (threadIdx.x == 0) {
        bcounts[br] = (I)nb;
        if (s_bad) atomicOr(err, 1);
        else if (s_unsorted) atomicOr(flags, kPackFlagUnsorted);
        else if (s_nonfinite) atomicOr(flags, kPackFlagNonFinite);
    }
    if (threadIdx.x < nw) {
        uint32_t n = 0;
        if (!s_bad && !s_unsorted)
            n = pack_walk<false>(reinterpret_cast<const uint32_t*>(smem + L.pw), nullptr, threadIdx.x, nw,
                                 (nb + 1) >> 1);
        counts[br * nw + threadIdx.x] = (int32_t)n;
    }
}

// status[0..4] = {batches, blocks, err, flags, go}: go (the packed form is
// taken) when the input is valid, sorted (and for fp16 finite), the grid is
// not fully populated, there is a batch, the batches fit the cap of the
// arrays they are written to and take at most three quarters of the BCSR
// blocks' bytes: num * batches <= den * blocks (fp16: 1152 B per batch
// against 512 B per block, num / den = 3 / 1; fp32: 272 B against 1024 B,
// 17 / 48).
__device__ __forceinline__ void pack_decide(int64_t nbat, int64_t nnzb, int e, unsigned int f, int64_t Mb,
                                            int64_t Kb, int64_t cap, int64_t num, int64_t den,
                                            int64_t* __restrict__ status)
{
    const bool go = e == 0 && f == 0u && nbat > 0 && nbat <= cap && nnzb != Mb * Kb &&
                    num * nbat <= den * nnzb;
    status[0] = nbat;
    status[1] = nnzb;
    status[2] = (int64_t)e;
    status[3] = (int64_t)f;
    status[4] = go ? 1 : 0;
}

template <typename I>
__global__ void pack_decide_kernel(const int64_t* __restrict__ off_end, const I* __restrict__ brp_end,
                                   const int* __restrict__ err, const unsigned int* __restrict__ flags,
                                   int64_t Mb, int64_t Kb, int64_t cap, int64_t num, int64_t den,
                                   int64_t* __restrict__ status)
{
    if (threadIdx.x == 0 && blockIdx.x == 0)
        pack_decide(*off_end, (int64_t)*brp_end, *err, *flags, Mb, Kb, cap, num, den, status);
}

// One workgroup scans both count arrays and decides (one launch instead of
// two device-wide scans and pack_decide_kernel) while the batch counts fit
// one pass of the workgroup (kPackScanMax); longer arrays take the
// device-wide scans (at gnn, 32768 counts: 41 us in four passes of one
// workgroup against 13 us).
constexpr int kPackScanThreads = 1024;
constexpr int kPackScanItems = 8;
constexpr int64_t kPackScanMax = (int64_t)kPackScanThreads * kPackScanItems;

__device__ __forceinline__ int64_t wg_exclusive_scan_1024(int64_t v, int64_t* total, int64_t* red)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t incl = wave_inclusive_scan(v);
    if (lane == 63) red[wave] = incl;
    __syncthreads();
    int64_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kPackScanThreads / 64; ++w) {
        const int64_t x = red[w];
        if (w < wave) before += x;
        all += x;
    }
    __syncthreads();
    *total = all;
    return before + incl - v;
}

// out[0..n] = exclusive prefix sums of in[0..n), out[n] = total (returned)
template <typename T, typename O>
__device__ int64_t wg_scan_array(const T* __restrict__ in, int64_t n, O* __restrict__ out, int64_t* red)
{
    int64_t carry = 0;
    for (int64_t c0 = 0; c0 < n; c0 += (int64_t)kPackScanThreads * kPackScanItems) {
        const int64_t base = c0 + (int64_t)threadIdx.x * kPackScanItems;
        int64_t v[kPackScanItems];
        int64_t sum = 0;
#pragma unroll
        for (int e = 0; e < kPackScanItems; ++e) {
            v[e] = base + e < n ? (int64_t)in[base + e] : 0;
            sum += v[e];
        }
        int64_t tot;
        int64_t run = carry + wg_exclusive_scan_1024(sum, &tot, red);
#pragma unroll
        for (int e = 0; e < kPackScanItems; ++e) {
            if (base + e < n) out[base + e] = (O)run;
            run += v[e];
        }
        carry += tot;
    }
    if (threadIdx.x == 0) out[n] = (O)carry;
    return carry;
}

template <typename I>
__global__ __launch_bounds__(kPackScanThreads) void pack_scan_kernel(
    const I* __restrict__ bcounts, int64_t Mb, const int32_t* __restrict__ counts, int nw,
    I* __restrict__ brp, int64_t* __restrict__ offsets, const int* __restrict__ err,
    const unsigned int* __restrict__ flags, int64_t Kb, int64_t cap, int64_t num, int64_t den,
    int64_t* __restrict__ status)
{
    __shared__ int64_t red[kPackScanThreads / 64];
    const int64_t nnzb = wg_scan_array(bcounts, Mb, brp, red);
    const int64_t nbat = wg_scan_array(counts, Mb * nw, offsets, red);
    if (threadIdx.x == 0) pack_decide(nbat, nnzb, *err, *flags, Mb, Kb, cap, num, den, status);
}

// Writes strip br's batches [offsets[br * nw], offsets[br * nw + nw]) when
// status[4] (go) is set: A' operands (1 KB each; lane (r, g) holds
// A'[r][4g .. 4g+3] and A'[r][16 + 4g .. 16 + 4g + 3]) and B-row indices
// (32 per batch, 0xffffffff for an unused slot).  Batches at or above cap
// are never written.
template <typename I>
__global__ __launch_bounds__(kThreads) void pack_emit_kernel(
    int64_t M, int64_t K, int64_t nnz, const I* __restrict__ rp, const I* __restrict__ ci,
    const uint16_t* __restrict__ vals, int64_t nwords, int64_t Kb, int nw,
    const int64_t* __restrict__ offsets, const int64_t* __restrict__ status, int64_t cap,
    uint16_t* __restrict__ a, uint32_t* __restrict__ rows)
{
    if (status[4] == 0) return;  // uniform: before any barrier
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int s_unsorted, s_bad, s_nonfinite;
    __shared__ int64_t red[kThreads / 64];
    const PackLds L = pack_lds(Kb, nw);
    StripView sv;
    int64_t nb;
    pack_strip(M, K, nnz, rp, ci, vals, nwords, smem, L, sv, &s_unsorted, &s_bad, &s_nonfinite, red, &nb);
    if (s_bad || s_unsorted || s_nonfinite) return;  // uniform; excluded by go
    const uint32_t* bitmap = reinterpret_cast<const uint32_t*>(smem + L.bitmap);
    const uint32_t* prefix = reinterpret_cast<const uint32_t*>(smem + L.prefix);
    const uint32_t* pw = reinterpret_cast<const uint32_t*>(smem + L.pw);
    uint32_t* pinfo = reinterpret_cast<uint32_t*>(smem + L.pinfo);
    int64_t* ob = reinterpret_cast<int64_t*>(smem + L.ob);
    uint16_t* bcl = reinterpret_cast<uint16_t*>(smem + L.bcl);
    const int64_t br = blockIdx.x;
    const int64_t npairs = (nb + 1) >> 1;

    // each block's column block, by rank
    {
        const int64_t per = (nwords + kThreads - 1) / kThreads;
        const int64_t w0 = (int64_t)threadIdx.x * per;
        const int64_t w1 = (w0 + per < nwords) ? w0 + per : nwords;
        for (int64_t w = w0; w < w1; ++w) {
            uint32_t bits = bitmap[w];
            uint32_t o = prefix[w];
            while (bits) {
                bcl[o++] = (uint16_t)(w * 32 + (__ffs(bits) - 1));
                bits &= bits - 1;
            }
        }
    }
    if (threadIdx.x <= nw) ob[threadIdx.x] = offsets[br * nw + threadIdx.x];
    // clear the strip's batches (A' zero, indices unused) while the walk runs
    {
        const int64_t q0 = offsets[br * nw];
        int64_t q1 = offsets[br * nw + nw];
        if (q1 > cap) q1 = cap;
        uint4* a4 = reinterpret_cast<uint4*>(a);
        uint4* r4 = reinterpret_cast<uint4*>(rows);
        for (int64_t i = q0 * 64 + threadIdx.x; i < q1 * 64; i += kThreads) a4[i] = make_uint4(0, 0, 0, 0);
        const uint32_t u = 0xffffffffu;
        for (int64_t i = q0 * 8 + threadIdx.x; i < q1 * 8; i += kThreads) r4[i] = make_uint4(u, u, u, u);
    }
    if (threadIdx.x < nw) (void)pack_walk<true>(pw, pinfo, threadIdx.x, nw, npairs);
    __syncthreads();  // clears complete; bcl, ob and pinfo visible

    // every used slot's B-row index: one thread per pair
    for (int64_t j = threadIdx.x; j < npairs; j += kThreads) {
        uint32_t pm = pair_mask(pw[j]);
        if (pm == 0u) continue;
        const uint32_t info = pinfo[j];
        const int64_t bi = ob[j % nw] + (int64_t)(info >> 6);
        if (bi >= cap) continue;
        uint32_t slot = info & 63u;
        while (pm) {
            const uint32_t b = (uint32_t)(__ffs(pm) - 1);
            pm &= pm - 1;
            const uint32_t pc = bit_pair_col(b);
            const uint32_t row = 16u * (uint32_t)bcl[2 * j + (pc >> 4)] + (pc & 15u);
            rows[bi * 32 + slot_kpos(slot)] = row;
            ++slot;
        }
    }
    // every non-zero entry's fp16 bits at its slot; -0.0 leaves the +0.0
    const int64_t e0 = sv.bounds[0];
    const int64_t e1 = sv.bounds[sv.nr];
    for (int64_t i0 = e0 + threadIdx.x; i0 < e1; i0 += (int64_t)kThreads * kEntryUnroll) {
        uint16_t v[kEntryUnroll];
        uint32_t c[kEntryUnroll];
#pragma unroll
        for (int u = 0; u < kEntryUnroll; ++u) {
            const int64_t idx = i0 + (int64_t)u * kThreads;
            v[u] = idx < e1 ? vals[idx] : (uint16_t)0;
            c[u] = idx < e1 ? (uint32_t)ci[idx] : 0u;
        }
#pragma unroll
        for (int u = 0; u < kEntryUnroll; ++u) {
            if ((v[u] & 0x7fffu) == 0u) continue;  // also the entries past the strip
            const int64_t idx = i0 + (int64_t)u * kThreads;
            const uint32_t bc = c[u] >> 4;
            const uint32_t w = bc >> 5;
            const uint32_t rank = prefix[w] + (uint32_t)__popc(bitmap[w] & ((1u << (bc & 31u)) - 1u));
            const uint32_t j = rank >> 1;
            const uint32_t pm = pair_mask(pw[j]);
            const uint32_t info = pinfo[j];
            const uint32_t bit = pair_bit(16u * (rank & 1u) + (c[u] & 15u));
            const uint32_t slot = (info & 63u) + (uint32_t)__popc(pm & ((1u << bit) - 1u));
            const int64_t bi = ob[j % (uint32_t)nw] + (int64_t)(info >> 6);
            if (bi >= cap) continue;
            const int64_t r = row_of(sv, idx);
            const uint32_t lane = ((slot & 15u) >> 2) * 16u + (uint32_t)r;
            const uint32_t t = (slot >> 4) * 4u + (slot & 3u);
            a[(bi * 64 + lane) * 8 + t] = v[u];
        }
    }
}
// ---------------------------------------------------------------------------
// CSR -> packed fp32 column batches (the Tier-2 pipeline's fp32 form,
// multiplied by spmm_f32_packed_kernel).  A strip's slots are its set
// columns (a column of a block is set when one of its entries is not +-0)
// in block order (ascending block column), then column order; slot s is
// K position s % 4 of batch s / 4.  A batch's A' operand is 16 rows x 4
// slots of fp32 values (zeros where a row has no entry), and its B-row
// indices are the slots' columns (0xffffffff for a slot past the last).  A
// strip's batch count is rounded up to a multiple of 4; four consecutive
// batches form a group, stored so that one 16-byte load per lane reads the
// group: A' value of batch 4G + c, row i, slot k at float (64 G + 16 k + i)
// * 4 + c, B row of its slot k at word (4 G + k) * 4 + c.  Per strip:
//   pack32_analyse_kernel  the strip's block count and batch count (and the
//                          flags of pack_analyse_kernel);
//   pack_scan_kernel       as for fp16, one batch count per strip;
//   pack32_emit_kernel     clears the strip's groups, then stores every set
//                          entry's value and its column as the slot's B row.
// Batch count bound: a strip's S slots make at most S / 4 + 4 batches
// after rounding, so at most nnz / 4 + 4 Mb in all, and at most
// 4 Kb + 4 per strip.

template <typename I>
__global__ __launch_bounds__(kThreads) void pack32_analyse_kernel(
    int64_t M, int64_t K, int64_t nnz, const I* __restrict__ rp, const I* __restrict__ ci,
    const uint32_t* __restrict__ vals, int64_t nwords, int64_t Kb, I* __restrict__ bcounts,
    int32_t* __restrict__ counts, int* __restrict__ err, unsigned int* __restrict__ flags)
{
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int s_unsorted, s_bad, s_nonfinite;
    __shared__ int64_t red[kThreads / 64];
    const PackLds L = pack_lds(Kb, 1);
    StripView sv;
    int64_t nb;
    pack_strip(M, K, nnz, rp, ci, vals, nwords, smem, L, sv, &s_unsorted, &s_bad, &s_nonfinite, red, &nb);
    const int64_t br = blockIdx.x;
    if (s_bad || s_unsorted) {  // uniform
        if (threadIdx.x == 0) {
            bcounts[br] = (I)nb;
            counts[br] = 0;
            if (s_bad) atomicOr(err, 1);
            else atomicOr(flags, kPackFlagUnsorted);
        }
        return;
    }
    const uint32_t* pw = reinterpret_cast<const uint32_t*>(smem + L.pw);
    const int64_t npairs = (nb + 1) >> 1;
    int64_t mine = 0;
    for (int64_t j = threadIdx.x; j < npairs; j += kThreads) mine += __popc(pw[j]);
    const int64_t slots = block_sum(mine, red);
    if (threadIdx.x == 0) {
        bcounts[br] = (I)nb;
        counts[br] = (int32_t)((((slots + 3) / 4) + 3) / 4 * 4);
    }
}

// Writes strip br's batches [offsets[br], offsets[br + 1]) when status[4]
// (go) is set; batches at or above cap are never written.
template <typename I>
__global__ __launch_bounds__(kThreads) void pack32_emit_kernel(
    int64_t M, int64_t K, int64_t nnz, const I* __restrict__ rp, const I* __restrict__ ci,
    const uint32_t* __restrict__ vals, int64_t nwords, int64_t Kb, const int64_t* __restrict__ offsets,
    const int64_t* __restrict__ status, int64_t cap, uint32_t* __restrict__ a, uint32_t* __restrict__ rows)
{
    if (status[4] == 0) return;  // uniform: before any barrier
    extern __shared__ __align__(16) unsigned char smem[];
    __shared__ int s_unsorted, s_bad, s_nonfinite;
    __shared__ int64_t red[kThreads / 64];
    const PackLds L = pack_lds(Kb, 1);
    StripView sv;
    int64_t nb;
    pack_strip(M, K, nnz, rp, ci, vals, nwords, smem, L, sv, &s_unsorted, &s_bad, &s_nonfinite, red, &nb);
    if (s_bad || s_unsorted) return;  // uniform; excluded by go
    const uint32_t* bitmap = reinterpret_cast<const uint32_t*>(smem + L.bitmap);
    const uint32_t* prefix = reinterpret_cast<const uint32_t*>(smem + L.prefix);
    const uint32_t* pw = reinterpret_cast<const uint32_t*>(smem + L.pw);
    uint32_t* sb = reinterpret_cast<uint32_t*>(smem + L.sb);
    const int64_t br = blockIdx.x;
    const int64_t npairs = (nb + 1) >> 1;

    // each block's first slot: exclusive scan of the column counts by rank
    {
        const int64_t per = (npairs + kThreads - 1) / kThreads;
        const int64_t j0 = (int64_t)threadIdx.x * per;
        const int64_t j1 = (j0 + per < npairs) ? j0 + per : npairs;
        int64_t mine = 0;
        for (int64_t j = j0; j < j1; ++j) mine += __popc(pw[j]);
        int64_t total;
        int64_t run = block_exclusive_scan(mine, &total, red);
        for (int64_t j = j0; j < j1; ++j) {
            const uint32_t w = pw[j];
            sb[2 * j] = (uint32_t)run;
            run += __popc(w & 0xffffu);
            sb[2 * j + 1] = (uint32_t)run;
            run += __popc(w >> 16);
        }
    }
    // clear the strip's groups (A' zero, indices unused)
    const int64_t q0 = offsets[br];
    int64_t q1 = offsets[br + 1];
    if (q1 > cap) q1 = cap;
    {
        uint4* a4 = reinterpret_cast<uint4*>(a);
        uint4* r4 = reinterpret_cast<uint4*>(rows);
        for (int64_t i = q0 * 16 + threadIdx.x; i < q1 * 16; i += kThreads) a4[i] = make_uint4(0, 0, 0, 0);
        const uint32_t u = 0xffffffffu;
        for (int64_t i = q0 + threadIdx.x; i < q1; i += kThreads) r4[i] = make_uint4(u, u, u, u);
    }
    __syncthreads();  // clears complete; slot bases visible

    const int64_t e0 = sv.bounds[0];
    const int64_t e1 = sv.bounds[sv.nr];
    for (int64_t i0 = e0 + threadIdx.x; i0 < e1; i0 += (int64_t)kThreads * kEntryUnroll) {
        uint32_t v[kEntryUnroll], c[kEntryUnroll];
#pragma unroll
        for (int u = 0; u < kEntryUnroll; ++u) {
            const int64_t idx = i0 + (int64_t)u * kThreads;
            v[u] = idx < e1 ? vals[idx] : 0u;
            c[u] = idx < e1 ? (uint32_t)ci[idx] : 0u;
        }
#pragma unroll
        for (int u = 0; u < kEntryUnroll; ++u) {
            if (!pack_set(v[u])) continue;  // also the entries past the strip
            const int64_t idx = i0 + (int64_t)u * kThreads;
            const uint32_t bc = c[u] >> 4;
            const uint32_t w = bc >> 5;
            const uint32_t rank = prefix[w] + (uint32_t)__popc(bitmap[w] & ((1u << (bc & 31u)) - 1u));
            const uint32_t m = (pw[rank >> 1] >> (16u * (rank & 1u))) & 0xffffu;
            const uint32_t slot = sb[rank] + (uint32_t)__popc(m & ((1u << (c[u] & 15u)) - 1u));
            const int64_t t = q0 + (int64_t)(slot >> 2);  // the batch (q0 is a multiple of 4)
            if (t >= cap) continue;
            const uint32_t k = slot & 3u;
            const int64_t G = t >> 2;
            const uint32_t cc = (uint32_t)(t & 3);
            const int64_t r = row_of(sv, idx);
            a[((G * 64) + 16 * k + r) * 4 + cc] = v[u];
            rows[(G * 4 + k) * 4 + cc] = c[u];
        }
    }
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

bool csr_pack_covers(int64_t K)
{
    const int64_t Kb = (K + 15) / 16;
    if (Kb <= 0) return false;
    const PackLds L16 = pack_lds(Kb, spmm_batch_waves()), L32 = pack_lds(Kb, 1);
    return L16.emit_bytes <= kMaxLds && L32.emit32_bytes <= kMaxLds;
}

int64_t csr_pack_batch_bound(int64_t M, int64_t K, int64_t nnz, int value_bytes)
{
    const int64_t Mb = (M + 15) / 16, Kb = (K + 15) / 16;
    if (value_bytes == 4) return std::min<int64_t>(nnz / 4 + 4 * Mb, Mb * (4 * Kb + 4));
    const int64_t by_slots = 2 * nnz / 33 + std::min<int64_t>(Mb * spmm_batch_waves(), nnz);
    return std::min<int64_t>(by_slots, Mb * ((Kb + 1) / 2));  // a batch holds a pair
}

template <typename I, typename V>
void csr_pack_analyse(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const V* vals,
                      I* bcounts, I* brp, int32_t* counts, int64_t* offsets, int* err,
                      unsigned int* flags, int64_t cap, int64_t* status, hipStream_t s)
{
    constexpr bool f32 = sizeof(V) == 4;
    const ConvGeometry g = conv_geometry(M, K, nnz, 16, 16);
    if (!csr_pack_covers(K)) throw std::invalid_argument("csr_pack_analyse: K above the packed form's limit.");
    const int nw = f32 ? 1 : spmm_batch_waves();  // batch counts per strip
    const PackLds L = pack_lds(g.Kb, nw);
    const int64_t num = f32 ? 17 : 3, den = f32 ? 48 : 1;
    hipLaunchKernelGGL(set_value_kernel<int>, dim3(1), dim3(64), 0, s, err, 0);
    XSPMM_LAUNCH_CHECK();
    hipLaunchKernelGGL(set_value_kernel<unsigned int>, dim3(1), dim3(64), 0, s, flags, 0u);
    XSPMM_LAUNCH_CHECK();
    if (g.Mb > 0) {
        if constexpr (f32)
            hipLaunchKernelGGL(pack32_analyse_kernel<I>, dim3((unsigned)g.Mb), dim3(kThreads), L.analyse_bytes,
                               s, M, K, nnz, rp, ci, vals, g.nwords, g.Kb, bcounts, counts, err, flags);
        else
            hipLaunchKernelGGL(pack_analyse_kernel<I>, dim3((unsigned)g.Mb), dim3(kThreads), L.analyse_bytes,
                               s, M, K, nnz, rp, ci, vals, g.nwords, g.Kb, nw, bcounts, counts, err, flags);
        XSPMM_LAUNCH_CHECK();
    }
    if (g.Mb * nw <= kPackScanMax) {
        hipLaunchKernelGGL(pack_scan_kernel<I>, dim3(1), dim3(kPackScanThreads), 0, s, bcounts, g.Mb, counts,
                           nw, brp, offsets, err, flags, g.Kb, cap, num, den, status);
        XSPMM_LAUNCH_CHECK();
        return;
    }
    device_exclusive_scan(ArrayValue<I>{bcounts}, g.Mb, brp, s);
    device_exclusive_scan(ArrayValue<int32_t>{counts}, g.Mb * nw, offsets, s);
    hipLaunchKernelGGL(pack_decide_kernel<I>, dim3(1), dim3(64), 0, s, offsets + g.Mb * nw, brp + g.Mb,
                       err, flags, g.Mb, g.Kb, cap, num, den, status);
    XSPMM_LAUNCH_CHECK();
}

PackStatus csr_pack_status(const int64_t* status, hipStream_t s)
{
    int64_t h[5] = {0, 0, 0, 0, 0};
    XSPMM_HIP_CHECK(hipMemcpyAsync(h, status, sizeof(h), hipMemcpyDeviceToHost, s));
    XSPMM_HIP_CHECK(hipStreamSynchronize(s));
    return PackStatus{h[0], h[1], (int)h[2], (unsigned)h[3], h[4] != 0};
}

template <typename I, typename V>
void csr_pack_emit(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci, const V* vals,
                   const int64_t* offsets, const int64_t* status, int64_t cap, void* a, uint32_t* rows,
                   hipStream_t s)
{
    constexpr bool f32 = sizeof(V) == 4;
    const ConvGeometry g = conv_geometry(M, K, nnz, 16, 16);
    if (g.Mb == 0 || cap <= 0) return;
    if (!csr_pack_covers(K)) throw std::invalid_argument("csr_pack_emit: K above the packed form's limit.");
    if constexpr (f32) {
        const PackLds L = pack_lds(g.Kb, 1);
        hipLaunchKernelGGL(pack32_emit_kernel<I>, dim3((unsigned)g.Mb), dim3(kThreads), L.emit32_bytes, s, M,
                           K, nnz, rp, ci, vals, g.nwords, g.Kb, offsets, status, cap,
                           static_cast<uint32_t*>(a), rows);
    } else {
        const int nw = spmm_batch_waves();
        const PackLds L = pack_lds(g.Kb, nw);
        hipLaunchKernelGGL(pack_emit_kernel<I>, dim3((unsigned)g.Mb), dim3(kThreads), L.emit_bytes, s, M, K,
                           nnz, rp, ci, vals, g.nwords, g.Kb, nw, offsets, status, cap,
                           static_cast<uint16_t*>(a), rows);
    }
    XSPMM_LAUNCH_CHECK();
}

#define XSPMM_INST_PACK(I, V)                                                                     \
    template void csr_pack_analyse<I, V>(int64_t, int64_t, int64_t, const I*, const I*, const V*, \
                                         I*, I*, int32_t*, int64_t*, int*, unsigned int*,         \
                                         int64_t, int64_t*, hipStream_t);                         \
    template void csr_pack_emit<I, V>(int64_t, int64_t, int64_t, const I*, const I*, const V*,    \
                                      const int64_t*, const int64_t*, int64_t, void*, uint32_t*, \
                                      hipStream_t);
XSPMM_INST_PACK(int32_t, uint16_t)
XSPMM_INST_PACK(int64_t, uint16_t)
XSPMM_INST_PACK(int32_t, uint32_t)
XSPMM_INST_PACK(int64_t, uint32_t)
#undef XSPMM_INST_PACK

}  // namespace detail
}  // namespace xspmm
