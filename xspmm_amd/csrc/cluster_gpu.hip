// cluster_gpu.hip -- exact 1-D Jaccard ("Sylos Labini") row clustering on the GPU.
//
// Same greedy, same visiting order and same float comparison as the
// reference (src/cpu/clustering_sylos_labini.cpp:51-120) and as the host
// engines in cluster.cpp, so the permutation is identical bit for bit:
//   q_r = set of block_width-wide column blocks row r touches (:13-33);
//   unclustered = [0..M-1]; while non-empty: seed = pop_back(); p = q_seed;
//   for i = size-1 down to 0: cand = unclustered[i];
//     d = |p|q| == 0 ? 0 : 1 - (float)|p&q| / (float)|p|q|          (:35-46)
//     if d <= dist_thresh: join, p |= q_cand, swap-remove position i (:97-104)
//
// The greedy is sequential in its commits: whether a candidate joins depends
// on every join before it.  It runs in ONE workgroup of 1024 threads, which
// evaluates many candidates at once against the current pattern and commits
// the first joiner in visiting order (the highest position), then goes on
// below it -- the candidates above it were tested against the right pattern.
// All threads keep the loop state (counts, positions) in registers as
// identical copies: every decision comes out of a block reduction.  Thread 0
// writes a single commit to the shared arrays (permutation, positions); a
// run of commits is written by all threads, each its own entries.
//
// Two engines, picked from the pattern statistics (or XSPMM_CLUSTER_ENGINE):
//  * scan:  each step tests 1024 consecutive positions below the last commit
//           with popcounts of the row bitmaps (a popcount bound first), and
//           commits every joiner down to the first one that grows the
//           pattern (joiners whose rows lie inside it leave it unchanged);
//  * index: only rows that share a block with the pattern can join (d = 1
//           otherwise, and dist_thresh < 1), so the workgroup keeps
//           |p & q_r| per row, raised through per-block row lists whenever a
//           block enters the pattern, and tests only those rows;
//           |p | q_r| = |p| + |q_r| - |p & q_r|.
// Every loop of the clustering kernel ends: each commit removes a row and
// lowers the scan limit, and each step without a commit lowers it by 1024.
//
// Preparation (all rows in parallel): row bitmaps by atomic OR (in LDS up to
// 64 words per row), their popcounts, each row's block list, the per-block
// row lists (counts, exclusive scan, scatter) and each row's partners --
// the rows close enough to join it while the pattern is still its own, by
// all pairs on the int8 matrix cores or through the row lists.  A seed whose partners are
// all clustered forms a cluster of one without a scan, and any other seed
// starts its scan at its highest-positioned partner.
#include <cstdlib>
#include <cstring>
#include <string>
#include <vector>

#include "internal.hpp"
#include "scan.hpp"

namespace xspmm {
namespace detail {

namespace {

constexpr int kClThreads = 1024;
constexpr int kClWaves = kClThreads / 64;
constexpr int kPatternWords32 = 16384;        // LDS pattern bitmap: 64 KB
constexpr int64_t kMaxGpuBlocks = 32LL * kPatternWords32;  // 524288 column blocks
constexpr int kPrepThreads = 256;
constexpr int kEngineAuto = 0, kEngineScan = 1, kEngineIndex = 2;

// Jaccard distance exactly as the reference evaluates it: int -> float
// conversions and an IEEE division (round to nearest).
__device__ __forceinline__ float jaccard_distance(int inter, int uni)
{
    if (uni == 0) return 0.0f;
    return 1.0f - __fdiv_rn((float)inter, (float)uni);
}

// The reference's test d(inter, uni) <= thr, decided without the division
// away from the threshold.  With x = inter / uni (exact), the float value
// d = RN(1 - RN(x)) is within 2^-23 of 1 - x.  So d <= thr whenever
// x >= 1 - thr + 2^-23, and d > thr whenever x < 1 - thr - 2^-23.  The
// factors a_hi / a_lo add 2^-20 of margin on either side, which covers the
// rounding of the products a * uni (uni < 2^24, so int -> float is exact).
// Inside that band the division decides, exactly as the reference.
struct JaccardTest {
    float thr, a_hi, a_lo;
    __device__ explicit JaccardTest(float t) : thr(t)
    {
        const float a = 1.0f - t;
        a_hi = a + 0x1p-20f;
        a_lo = a - 0x1p-20f;
    }
    __device__ __forceinline__ bool close(int inter, int uni) const
    {
        if (uni == 0) return 0.0f <= thr;
        const float fi = (float)inter, fu = (float)uni;
        if (fi >= a_hi * fu) return true;
        if (fi < a_lo * fu) return false;
        return jaccard_distance(inter, uni) <= thr;
    }
    // false when no pair of rows with popcounts mn <= mx can be close:
    // |p & q| <= mn and |p | q| >= mx, so x <= mn / mx
    __device__ __forceinline__ bool may_close(int mn, int mx) const
    {
        return !((float)mn < a_lo * (float)mx);
    }
};

// Phase boundary of the clustering workgroup: every wave waits until its
// global stores and atomics are acknowledged, then the barrier.  All waves
// share one CU, so plain loads after the barrier see plain stores from
// before it; the counters (cnt) live at L2 and are only touched by L2
// atomics and L1-bypassing atomic loads/stores.  (An agent-scope fence
// would also write back and invalidate the L2 -- far slower, and not
// needed inside one workgroup.)
__device__ __forceinline__ void phase_sync()
{
    __builtin_amdgcn_s_waitcnt(0);
    __syncthreads();
}

__device__ __forceinline__ int wave_max(int v)
{
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v = max(v, __shfl_xor(v, d, 64));
    return v;
}

__device__ __forceinline__ int64_t wave_sum64(int64_t v)
{
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) v += __shfl_xor(v, d, 64);
    return v;
}

// Block-wide reductions over the 1024 threads (two barriers each).
__device__ __forceinline__ int block_max(int v, int* red)
{
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    int m = red[0];
#pragma unroll
    for (int w = 1; w < kClWaves; ++w) m = max(m, red[w]);
    __syncthreads();
    return m;
}

__device__ __forceinline__ int64_t block_sum64(int64_t v, int64_t* red)
{
    v = wave_sum64(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    int64_t s = 0;
#pragma unroll
    for (int w = 0; w < kClWaves; ++w) s += red[w];
    __syncthreads();
    return s;
}

// Exclusive scan over the 1024 threads; *total gets the sum (two barriers).
__device__ __forceinline__ int64_t block_exscan64(int64_t v, int64_t* total, int64_t* red)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int64_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    if (lane == 63) red[wave] = incl;
    __syncthreads();
    int64_t before = 0, all = 0;
#pragma unroll
    for (int w = 0; w < kClWaves; ++w) {
        const int64_t x = red[w];
        if (w < wave) before += x;
        all += x;
    }
    __syncthreads();
    *total = all;
    return before + incl - v;
}

// --- preparation kernels (one wave per row) ---------------------------------

// column block of column c: a shift when the block width is a power of two
// (sh >= 0), else a division
__device__ __forceinline__ int64_t column_block(int64_t c, int64_t bw, int sh)
{
    return sh >= 0 ? c >> sh : c / bw;
}

template <typename I>
__global__ __launch_bounds__(kPrepThreads) void pattern_bits_kernel(const I* __restrict__ rp,
                                                                    const I* __restrict__ ci,
                                                                    int64_t M, int64_t K,
                                                                    int64_t nnz, int64_t bw, int sh,
                                                                    int64_t W, uint64_t* bits,
                                                                    int* bad)
{
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * (kPrepThreads / 64);
    for (int64_t r = ((int64_t)blockIdx.x * kPrepThreads + threadIdx.x) >> 6; r < M; r += nw) {
        int64_t s = (int64_t)rp[r], e = (int64_t)rp[r + 1];
        s = s < 0 ? 0 : s;
        e = e > nnz ? nnz : e;
        uint64_t* q = bits + r * W;
        for (int64_t j = s + lane; j < e; j += 64) {
            const int64_t c = (int64_t)ci[j];
            if (c < 0 || c >= K) {
                *bad = 1;
                continue;
            }
            const int64_t b = column_block(c, bw, sh);
            atomicOr((unsigned long long*)(q + (b >> 6)), 1ULL << (b & 63));
        }
    }
}

// Row bitmaps of at most 64 words and their popcounts in one pass: each wave
// ORs its row's bits into a bitmap in LDS (a wave's LDS operations complete
// in order), then stores its W words and the popcount -- no global atomics
// and no separate count pass.
template <typename I>
__global__ __launch_bounds__(kPrepThreads) void pattern_bits_lds_kernel(const I* __restrict__ rp,
                                                                        const I* __restrict__ ci,
                                                                        int64_t M, int64_t K,
                                                                        int64_t nnz, int64_t bw, int sh,
                                                                        int W, uint64_t* __restrict__ bits,
                                                                        int32_t* __restrict__ count,
                                                                        int* bad)
{
    __shared__ unsigned long long lbits[kPrepThreads / 64][64];
    const int lane = threadIdx.x & 63;
    unsigned long long* const q = lbits[threadIdx.x >> 6];
    const int64_t nw = (int64_t)gridDim.x * (kPrepThreads / 64);
    for (int64_t r = ((int64_t)blockIdx.x * kPrepThreads + threadIdx.x) >> 6; r < M; r += nw) {
        if (lane < W) q[lane] = 0ULL;
        __builtin_amdgcn_wave_barrier();
        int64_t s = (int64_t)rp[r], e = (int64_t)rp[r + 1];
        s = s < 0 ? 0 : s;
        e = e > nnz ? nnz : e;
        for (int64_t j = s + lane; j < e; j += 64) {
            const int64_t c = (int64_t)ci[j];
            if (c < 0 || c >= K) {
                *bad = 1;
                continue;
            }
            const int64_t b = column_block(c, bw, sh);
            atomicOr(q + (b >> 6), 1ULL << (b & 63));
        }
        __builtin_amdgcn_wave_barrier();
        int64_t n = 0;
        if (lane < W) {
            const uint64_t v = q[lane];
            bits[r * W + lane] = v;
            n = __popcll(v);
        }
        n = wave_sum64(n);
        if (lane == 0) count[r] = (int32_t)n;
        __builtin_amdgcn_wave_barrier();
    }
}

__global__ __launch_bounds__(kPrepThreads) void pattern_count_kernel(const uint64_t* __restrict__ bits,
                                                                     int64_t M, int64_t W,
                                                                     int32_t* count)
{
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * (kPrepThreads / 64);
    for (int64_t r = ((int64_t)blockIdx.x * kPrepThreads + threadIdx.x) >> 6; r < M; r += nw) {
        int64_t n = 0;
        for (int64_t w = lane; w < W; w += 64) n += __popcll(bits[r * W + w]);
        n = wave_sum64(n);
        if (lane == 0) count[r] = (int32_t)n;
    }
}

// Row r's blocks, ascending, at rb[rb_start[r] ...]; counts rows per block.
__global__ __launch_bounds__(kPrepThreads) void row_lists_kernel(const uint64_t* __restrict__ bits,
                                                                 int64_t M, int64_t W,
                                                                 const int64_t* __restrict__ rb_start,
                                                                 int32_t* rb, int32_t* bl_count)
{
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * (kPrepThreads / 64);
    for (int64_t r = ((int64_t)blockIdx.x * kPrepThreads + threadIdx.x) >> 6; r < M; r += nw) {
        int64_t at = rb_start[r];
        for (int64_t w0 = 0; w0 < W; w0 += 64) {
            const int64_t w = w0 + lane;
            uint64_t x = w < W ? bits[r * W + w] : 0ULL;
            const int64_t n = __popcll(x);
            int64_t incl = n;
#pragma unroll
            for (int d = 1; d < 64; d <<= 1) {
                const int64_t t = __shfl_up(incl, d, 64);
                if (lane >= d) incl += t;
            }
            int64_t o = at + incl - n;
            for (; x; x &= x - 1) {
                const int32_t b = (int32_t)(w * 64 + __builtin_ctzll(x));
                rb[o++] = b;
                atomicAdd(&bl_count[b], 1);
            }
            at += __shfl(incl, 63, 64);
        }
    }
}

// Rows per column block, v_b, from the bitmaps without building any list:
// thread b of grid.x counts bit b over its grid.y slice of rows (the 64
// threads of a wave read the same word), then adds once.
__global__ __launch_bounds__(kPrepThreads) void block_counts_kernel(const uint64_t* __restrict__ bits,
                                                                    int64_t M, int64_t W, int64_t Kb,
                                                                    int32_t* bl_count)
{
    const int64_t b = (int64_t)blockIdx.x * kPrepThreads + threadIdx.x;
    if (b >= Kb) return;
    const int64_t per = (M + gridDim.y - 1) / gridDim.y;
    const int64_t r0 = (int64_t)blockIdx.y * per;
    const int64_t r1 = r0 + per < M ? r0 + per : M;
    const int64_t w = b >> 6;
    const int sh = (int)(b & 63);
    int32_t c = 0;
    for (int64_t r = r0; r < r1; ++r) c += (int32_t)((bits[r * W + w] >> sh) & 1u);
    if (c) atomicAdd(&bl_count[b], c);
}

// Row lists per block: bl_rows[bl_start[b] ...] (order within a list is free).
// Per-block row lists, each entry with its row's block count beside it
// (bl_cnt), so that a walk over a list reads both contiguously.
__global__ __launch_bounds__(kPrepThreads) void block_lists_kernel(int64_t M,
                                                                   const int64_t* __restrict__ rb_start,
                                                                   const int32_t* __restrict__ rb,
                                                                   const int64_t* __restrict__ bl_start,
                                                                   int32_t* bl_fill, int32_t* bl_rows,
                                                                   int32_t* bl_cnt)
{
    const int lane = threadIdx.x & 63;
    const int64_t nw = (int64_t)gridDim.x * (kPrepThreads / 64);
    for (int64_t r = ((int64_t)blockIdx.x * kPrepThreads + threadIdx.x) >> 6; r < M; r += nw) {
        const int64_t r0 = rb_start[r], r1 = rb_start[r + 1];
        for (int64_t k = r0 + lane; k < r1; k += 64) {
            const int32_t b = rb[k];
            const int32_t at = atomicAdd(&bl_fill[b], 1);
            bl_rows[bl_start[b] + at] = (int32_t)r;
            bl_cnt[bl_start[b] + at] = (int32_t)(r1 - r0);
        }
    }
}

template <typename I>
__global__ void reversed_perm_kernel(I* perm, int64_t M)
{
    const int64_t stride = (int64_t)gridDim.x * blockDim.x;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < M; i += stride)
        perm[i] = (I)(M - 1 - i);
}

// The row list total and the bad-column flag side by side, for one copy to
// the host.
__global__ void status_kernel(const int64_t* __restrict__ total, const int* __restrict__ bad,
                              int64_t* __restrict__ status)
{
    if (threadIdx.x == 0) {
        status[0] = *total;
        status[1] = *bad;
    }
}

// --- partner lists -------------------------------------------------------------
// Row j is a partner of row i (j != i) when d(q_i, q_j) <= dist_thresh.  Until
// the first join of a cluster the pattern is exactly q_seed, so its first
// joiner is the highest-position unclustered partner of the seed, and a seed
// without one stays alone.  Lists hold up to kPartnerCap rows; pn[i] = -1
// marks a row whose list was not computed or overflowed (it then takes the
// full path).  Partnership is symmetric and fixed, so the lists are computed
// for all rows at once, in parallel.  pn[i] > kPartnerCap also means
// "overflowed": such a row takes the full path too.

constexpr int kPartnerCap = 32;
constexpr int kPairRows = 64;    // bitmap method: rows i per workgroup
constexpr int kPairTile = 128;   // rows j per LDS tile
constexpr int kHashSlots = 8192;

// The partner counts of a close pair (i, j) as they stand (relaxed loads,
// possibly stale), and the appends.  pn[i] counts row i's partners and the
// first kPartnerCap are listed; a count past the cap only marks the list
// overflowed, so a row whose count already reads past it is not added to
// again (stale reads just let an add happen).  Rows with thousands of
// partners would otherwise serialize on their counters.
__device__ __forceinline__ int partner_count(const int32_t* pn, int i)
{
    return __hip_atomic_load(pn + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void add_partner(int32_t* pn, int32_t* partners, int i, int j)
{
    const int k = atomicAdd(&pn[i], 1);
    if (k < kPartnerCap) partners[(int64_t)i * kPartnerCap + k] = j;
}

// All pairs by bitmap popcounts (row bitmaps of at most MAXW words).
// 256 threads: 64 rows i, four threads per row splitting each tile; the
// row tiles j are dealt over gridDim.y workgroups.  Each pair is tested once, as
// j > i, and a close pair is listed for both rows.  pn[i] (zeroed first)
// ends as the number of partners of row i; the first kPartnerCap are listed.
template <int MAXW>
__global__ __launch_bounds__(256) void partners_bitmap_kernel(const uint64_t* __restrict__ bits,
                                                              const int32_t* __restrict__ count,
                                                              int M, int W, float thr,
                                                              int32_t* pn, int32_t* partners)
{
    __shared__ uint64_t tile[kPairTile * MAXW];
    __shared__ int32_t tcount[kPairTile];
    const int t = threadIdx.x;
    const int li = t & (kPairRows - 1);
    const int part = t / kPairRows;
    const int i = blockIdx.x * kPairRows + li;
    const bool vi = i < M;
    uint64_t q[MAXW];
#pragma unroll
    for (int w = 0; w < MAXW; ++w) q[w] = (vi && w < W) ? bits[(int64_t)i * W + w] : 0ULL;
    const int qc = vi ? count[i] : 0;
    const int tiles = (M + kPairTile - 1) / kPairTile;
    const int jend = M;
    const JaccardTest jt(thr);
    const int ibase = blockIdx.x * kPairRows;
    // tiles of rows j dealt to the gridDim.y workgroups of a row block in
    // turn, so that each gets its share of the tiles above the block
    for (int tt = (int)blockIdx.y; tt < tiles; tt += (int)gridDim.y) {
        const int j0 = tt * kPairTile;
        // each pair once, as (i, j) with j > i: tiles wholly at or below this
        // workgroup's first row hold none (a uniform skip)
        if (j0 + kPairTile - 1 <= ibase) continue;
        __syncthreads();
        for (int x = t; x < kPairTile * MAXW; x += 256) {
            const int jj = x / MAXW, w = x % MAXW;
            const int j = j0 + jj;
            tile[x] = (j < M && w < W) ? bits[(int64_t)j * W + w] : 0ULL;
        }
        for (int jj = t; jj < kPairTile; jj += 256) tcount[jj] = j0 + jj < M ? count[j0 + jj] : 0;
        __syncthreads();
        if (!vi) continue;
        for (int jj = part; jj < kPairTile; jj += 256 / kPairRows) {
            const int j = j0 + jj;
            if (j >= jend || j <= i) continue;
            const int qj = tcount[jj];
            const int mn = qj < qc ? qj : qc, mx = qj < qc ? qc : qj;
            if (!jt.may_close(mn, mx)) continue;
            // |q_i | q_j| = |q_i| + |q_j| - |q_i & q_j| (counts are the popcounts)
            int inter = 0;
#pragma unroll
            for (int w = 0; w < MAXW; ++w) inter += __popcll(q[w] & tile[jj * MAXW + w]);
            if (jt.close(inter, qc + qj - inter)) {  // partnership is symmetric
                if (partner_count(pn, i) <= kPartnerCap) add_partner(pn, partners, i, j);
                if (partner_count(pn, j) <= kPartnerCap) add_partner(pn, partners, j, i);
            }
        }
    }
}

// All pairs on the int8 matrix cores: |q_i & q_j| is entry (i, j) of the
// Gram matrix Q Q^T of the 0/1 row bitmaps, an exact integer dot product.
// A workgroup of four waves takes a 128 x 128 tile (rows i of tile ti, rows
// j of tile tj >= ti: the upper triangle, numbered row by row), each wave a
// 64 x 64 quarter as 4 x 4 products v_mfma_i32_16x16x64_i8.  The tile's
// 256 bitmap rows and their counts are staged in LDS first (rows padded to
// 4 NQ + 1 words for W <= 4 NQ, the words past W zero; the odd stride
// spreads a read's 16 rows over the banks).  Lane group g of a wave reads word 4q + g
// of its rows for word quad q and spreads 16 of its bits per product into
// 16 bytes 0 / -1.  The A and B operands of a product come from the same
// spreading of the same word, so whatever K order the instruction's lane
// layout implies, it pairs equal bits of q_i and q_j, and (-1)(-1) = 1.
// Every pair j > i of the tile whose product passes a cheap bound (below)
// gets the exact Jaccard test in the accumulator layout (lane (l, g) holds
// rows 4g .. 4g+3 of column l of each 16 x 16 block), and a close pair is
// listed for both rows, as in the popcount kernel.
constexpr int kGramTile = 128;
typedef int i32x4_t __attribute__((ext_vector_type(4)));


// bits 15-s, 31-s, 47-s and 63-s of w (0 <= s < 16) as four bytes 0 or -1:
// v_perm_b32 selectors 8..11 replicate the top bits of bytes 1, 3, 5 and 7.
// One 64-bit shift per dword (the compiler would split it into two 32-bit
// operations).
template <int S>
__device__ __forceinline__ int spread_bits(uint64_t w)
{
    static_assert(S >= 0 && S < 16, "shift of 0 .. 15");
    uint64_t y = w;
    if constexpr (S != 0) asm("v_lshlrev_b64 %0, %1, %2" : "=v"(y) : "i"(S), "v"(w));
    return (int)__builtin_amdgcn_perm((uint32_t)(y >> 32), (uint32_t)y, 0x0b0a0908u);
}
// the 16 bytes of bits 16 C .. 16 C + 15 of the spreading order
template <int C>
__device__ __forceinline__ i32x4_t spread_chunk(uint64_t w)
{
    return i32x4_t{spread_bits<4 * C>(w), spread_bits<4 * C + 1>(w), spread_bits<4 * C + 2>(w),
                   spread_bits<4 * C + 3>(w)};
}

// NQ: word quads per row (W <= 4 NQ)
template <int NQ>
__global__ __launch_bounds__(256, 3) void partners_gram_kernel(const uint64_t* __restrict__ bits,
                                                             const int32_t* __restrict__ count,
                                                             int M, int W, int T, float thr,
                                                             int32_t* pn, int32_t* partners)
{
    constexpr int wp = 4 * NQ + 1;
    __shared__ uint64_t gram_lds[2 * kGramTile * wp + kGramTile];  // words, then 256 counts
    // tile (ti, tj): row t of the triangle holds T - t tiles, so the rows
    // above t hold start(t) = t T - t (t - 1) / 2; ti is the largest t with
    // start(t) <= id (the smaller root of start(t) = id, then corrected)
    const int64_t id = blockIdx.x;
    auto start = [&](int64_t t) { return t * T - t * (t - 1) / 2; };
    const double b2 = 2.0 * T + 1.0;
    int64_t ti = (int64_t)((b2 - sqrt(fmax(b2 * b2 - 8.0 * (double)id, 0.0))) * 0.5);
    ti = min(max(ti, (int64_t)0), (int64_t)T - 1);
    while (ti > 0 && start(ti) > id) --ti;
    while (ti + 1 < T && start(ti + 1) <= id) ++ti;
    const int64_t tj = ti + (id - start(ti));

    // stage rows i (local 0..127) and rows j (local 128..255): four threads
    // per row, each taking every fourth word; rows past M read as zeros
    int32_t* const lcount = reinterpret_cast<int32_t*>(gram_lds + 2 * kGramTile * wp);
    {
        const int t = threadIdx.x;
        for (int rr = t >> 2; rr < 2 * kGramTile; rr += 64) {
            const int64_t row = rr < kGramTile ? ti * kGramTile + rr : tj * kGramTile + rr - kGramTile;
            const bool valid = row < M;
            const uint64_t* src = bits + (valid ? row : 0) * W;
#pragma unroll
            for (int u = 0; u < NQ; ++u) {
                const int w = 4 * u + (t & 3);
                gram_lds[rr * wp + w] = valid && w < W ? src[w] : 0ULL;
            }
        }
        const int64_t row = t < kGramTile ? ti * kGramTile + t : tj * kGramTile + t - kGramTile;
        lcount[t] = row < M ? count[row] : 0;
    }
    __syncthreads();

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int li = lane & 15, g = lane >> 4;
    const int il0 = (wave >> 1) * 64;               // local row of the quarter's first i
    const int jl0 = kGramTile + (wave & 1) * 64;    // and of its first j
    const int64_t i0 = ti * kGramTile + il0;
    const int64_t j0 = tj * kGramTile + jl0 - kGramTile;
    // a quarter wholly on or below the diagonal, or past the last row, holds
    // no pair j > i (no barrier follows: the wave may leave)
    if (j0 + 63 <= i0 || i0 >= M || j0 >= M) return;

    // Candidates.  close() holds only if inter >= RN(a_lo uni) >= a' uni
    // with a' = a_lo (1 - 2^-24) and uni = c_i + c_j - inter, that is only if
    // inter >= a' / (1 + a') (c_i + c_j).  beta rounds that factor down by
    // 2^-16 (more than its float roundings), so f = floor(beta c) gives
    // f_i + f_j <= a' / (1 + a') (c_i + c_j): each accumulator starts at
    // -(f_i + f_j), and a pair whose product ends below zero is not close.
    const JaccardTest jt(thr);
    const float beta = jt.a_lo > 0.0f ? jt.a_lo / (1.0f + jt.a_lo) * (1.0f - 0x1p-16f) : 0.0f;
    int fi[4][4], fj[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
        // rows il0 + 16 m + 4 g + r (r = 0..3) and row jl0 + 16 m + li
        const int4 c4 = *reinterpret_cast<const int4*>(lcount + il0 + 16 * m + 4 * g);
        fi[m][0] = (int)(beta * (float)c4.x);
        fi[m][1] = (int)(beta * (float)c4.y);
        fi[m][2] = (int)(beta * (float)c4.z);
        fi[m][3] = (int)(beta * (float)c4.w);
        fj[m] = (int)(beta * (float)lcount[jl0 + 16 * m + li]);
    }
    i32x4_t acc[4][4];
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[m][n][r] = -(fi[m][r] + fj[n]);

    const uint64_t* const wi = gram_lds + (il0 + li) * wp + g;
    const uint64_t* const wj = gram_lds + (jl0 + li) * wp + g;
    // (eight quads unrolled would need more than 256 registers)
#pragma unroll(NQ > 4 ? 4 : NQ)
    for (int q = 0; q < NQ; ++q) {
        uint64_t a[4], b[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) {
            a[m] = wi[16 * m * wp + 4 * q];
            b[m] = wj[16 * m * wp + 4 * q];
        }
        auto chunk = [&]<int C>() __attribute__((always_inline)) {
            i32x4_t A[4], B[4];
#pragma unroll
            for (int m = 0; m < 4; ++m) {
                A[m] = spread_chunk<C>(a[m]);
                B[m] = spread_chunk<C>(b[m]);
            }
#pragma unroll
            for (int m = 0; m < 4; ++m)
#pragma unroll
                for (int n = 0; n < 4; ++n)
                    acc[m][n] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[m], B[n], acc[m][n], 0, 0, 0);
        };
        chunk.template operator()<0>();
        chunk.template operator()<1>();
        chunk.template operator()<2>();
        chunk.template operator()<3>();
    }

    // no candidate in the whole quarter (the usual case): done
    bool any = false;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) any |= acc[m][n][r] >= 0;
    if (!__any(any)) return;
    // the partner counts of the quarter's rows as the epilogue starts (they
    // only grow): pairs whose two lists had overflowed by then are skipped
    // without a read; the others read the count again before an add
    int pn_i[4][4], pn_j[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
#pragma unroll
        for (int r = 0; r < 4; ++r) pn_i[m][r] = partner_count(pn, min((int)i0 + 16 * m + 4 * g + r, M - 1));
        pn_j[m] = partner_count(pn, min((int)j0 + 16 * m + li, M - 1));
    }
    // every pair of the quarter has i < j < M (uniform)
    const bool interior = j0 >= i0 + 64 && j0 + 64 <= M;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int n = 0; n < 4; ++n) {
                if (acc[m][n][r] < 0) continue;
                const int inter = acc[m][n][r] + fi[m][r] + fj[n];
                // row numbers fit 31 bits (M < 2^31)
                const int i = (int)i0 + 16 * m + 4 * g + r;
                const int j = (int)j0 + 16 * n + li;
                if (!interior && (i >= M || j >= M || j <= i)) continue;
                // both lists already overflowed: nothing to add
                const int ni = pn_i[m][r], nj = pn_j[n];
                if (ni > kPartnerCap && nj > kPartnerCap) continue;
                const int ci = lcount[il0 + 16 * m + 4 * g + r], cj = lcount[jl0 + 16 * n + li];
                if (jt.close(inter, ci + cj - inter)) {  // partnership is symmetric
                    if (ni <= kPartnerCap && partner_count(pn, i) <= kPartnerCap) add_partner(pn, partners, i, j);
                    if (nj <= kPartnerCap && partner_count(pn, j) <= kPartnerCap) add_partner(pn, partners, j, i);
                }
            }
}

// Pairs through the per-block row lists: one workgroup per row i counts
// |q_i & q_j| for the rows j it meets in an LDS hash table, each wave
// walking the row lists of every 16th block of row i.  Only rows whose
// popcount bound allows a join are inserted; a row whose table would pass
// half full, and empty rows (their partners are the other empty rows, which
// share no block), get pn = -1.  The filled slots are listed, so a row reads
// and clears only those.
__global__ __launch_bounds__(1024) void partners_index_kernel(int M, const int64_t* __restrict__ rb_start,
                                                             const int32_t* __restrict__ rb,
                                                             const int64_t* __restrict__ bl_start,
                                                             const int32_t* __restrict__ bl_rows,
                                                             const int32_t* __restrict__ bl_cnt,
                                                             const int32_t* __restrict__ count,
                                                             float thr, int32_t* pn, int32_t* partners)
{
    __shared__ int32_t hkey[kHashSlots];
    __shared__ int32_t hval[kHashSlots];
    __shared__ uint16_t s_used[kHashSlots / 2];  // the slots a row filled, while it fits
    __shared__ int s_n, s_over, s_np;
    const int t = threadIdx.x;
    const JaccardTest jt(thr);
    // the table starts empty and each row leaves it empty: through its list
    // of filled slots, or wholly when the row overflowed
    for (int h = t; h < kHashSlots; h += 1024) {
        hkey[h] = -1;
        hval[h] = 0;
    }
    for (int i = blockIdx.x; i < M; i += gridDim.x) {
        const int qi = count[i];
        if (qi == 0) {
            if (t == 0) pn[i] = -1;
            continue;
        }
        if (t == 0) {
            s_n = 0;
            s_over = 0;
            s_np = 0;
        }
        __syncthreads();
        // each wave takes every 16th block of the row and walks its row list
        // with its lanes (contiguous reads of bl_rows)
        const int64_t rs = rb_start[i];
        const int wave = t >> 6, lane = t & 63;
        for (int c = wave; c < qi; c += kClWaves) {
            const int32_t b = rb[rs + c];
            const int64_t b0 = bl_start[b], b1 = bl_start[b + 1];
            for (int64_t e = b0 + lane; e < b1; e += 64) {
                const int32_t j = bl_rows[e];
                const int qj = bl_cnt[e];
                if (j == i || s_over) continue;
                const int mn = qj < qi ? qj : qi, mx = qj < qi ? qi : qj;
                if (!jt.may_close(mn, mx)) continue;
                uint32_t h = ((uint32_t)j * 2654435761u) & (kHashSlots - 1);
                for (int probe = 0; probe < kHashSlots; ++probe) {
                    const int32_t old = atomicCAS(&hkey[h], -1, j);
                    if (old == -1 || old == j) {
                        if (old == -1) {
                            const int k = atomicAdd(&s_n, 1);
                            if (k < kHashSlots / 2) s_used[k] = (uint16_t)h;
                            else s_over = 1;
                        }
                        atomicAdd(&hval[h], 1);
                        break;
                    }
                    h = (h + 1) & (kHashSlots - 1);
                }
            }
        }
        __syncthreads();
        if (!s_over) {
            for (int k = t; k < s_n; k += 1024) {
                const int h = s_used[k];
                const int32_t j = hkey[h];
                const int inter = hval[h];
                hkey[h] = -1;
                hval[h] = 0;
                if (jt.close(inter, qi + count[j] - inter)) {
                    const int np = atomicAdd(&s_np, 1);
                    if (np < kPartnerCap) partners[(int64_t)i * kPartnerCap + np] = j;
                }
            }
        } else {
            for (int h = t; h < kHashSlots; h += 1024) {
                hkey[h] = -1;
                hval[h] = 0;
            }
        }
        __syncthreads();
        if (t == 0) pn[i] = (s_over || s_np > kPartnerCap) ? -1 : s_np;
        __syncthreads();
    }
}

struct ClusterArgs {
    int64_t M, W, Kb;
    float thresh;
    int engine;
    const uint64_t* bits;     // M x W row bitmaps (scan engine)
    const int32_t* count;     // |q_r|
    const int64_t* rb_start;  // M + 1
    const int32_t* rb;        // row block lists
    const int64_t* bl_start;  // Kb + 1
    const int32_t* bl_rows;   // block row lists
    int32_t* un;              // unclustered rows by position
    int32_t* pos;             // position of each row, -1 once clustered
    int32_t* cnt;             // |p & q_r| (index engine), zero between clusters
    int32_t* log;             // rows with cnt > 0
    int32_t* cand_a;          // candidate lists (compacted each round)
    int32_t* cand_b;
    int32_t* plist;           // blocks of the pattern
    const int32_t* pn;        // partner counts (-1: unknown), or null
    const int32_t* partners;  // M x kPartnerCap partner rows
    int* engine_used;
};

// --- the clustering kernel ----------------------------------------------------

template <typename I>
__global__ __launch_bounds__(kClThreads) void cluster_kernel(ClusterArgs a, I* __restrict__ perm)
{
    __shared__ uint32_t p32[kPatternWords32];  // pattern bitmap
    __shared__ int red[kClWaves];
    __shared__ int64_t red64[kClWaves];
    __shared__ int s_cnt[4];                   // append counters: log, candidates, pattern
    __shared__ int32_t s_blk[kClThreads];      // touch: blocks of the current chunk
    __shared__ int64_t s_pre[kClThreads + 1];  // touch: their list offsets
    __shared__ uint8_t s_flag[kClThreads];
    __shared__ int32_t s_rank[kClThreads];     // commit: visiting rank of each window position
    __shared__ int32_t s_nxt[kClThreads];      // commit: move chains over the positions past the new end
    __shared__ int32_t s_val[kClThreads];

    const int t = threadIdx.x;
    const int M = (int)a.M;
    const int W = (int)a.W;  // 64-bit words per row bitmap
    const float thr = a.thresh;
    const JaccardTest jt(thr);
    uint64_t* p64 = reinterpret_cast<uint64_t*>(p32);

    for (int i = t; i < M; i += kClThreads) {
        a.un[i] = i;
        a.pos[i] = i;
    }
    for (int i = t; i < kPatternWords32; i += kClThreads) p32[i] = 0u;
    if (t < 4) s_cnt[t] = 0;

    int engine = a.engine;
    if (engine == kEngineAuto) {
        // work estimates: scan ~ M^2 * W / 2 word tests, index ~ 3 * sum over
        // blocks of (rows in the block)^2 counter updates
        int64_t sq = 0;
        for (int64_t b = t; b < a.Kb; b += kClThreads) {
            const int64_t v = a.bl_start[b + 1] - a.bl_start[b];
            sq += v * v;
        }
        const double s = (double)block_sum64(sq, red64);
        engine = 3.0 * s < 0.5 * (double)M * (double)M * (double)W ? kEngineIndex : kEngineScan;
    }
    if (t == 0) *a.engine_used = engine;
    phase_sync();

    int n_un = M;  // every thread holds the same loop state
    int out = 0;

    // Clusters of one, up to 4096 at a time.  The next seeds are un[n_un-1],
    // un[n_un-2], ... for as long as each stays alone, and the partner lists
    // decide that up front: the seed at position `at` is alone iff it has a
    // list and none of its partners is unclustered below `at` (partners above
    // `at` are the seeds before it, clustered by its turn).  The longest run
    // of such seeds is committed at once.  Each thread takes kRunSeeds seeds
    // per round (offsets t + 1024 u from the end) and reads their rows and
    // partner counts before any partner list.
    constexpr int kRunSeeds = 4;
    constexpr int kRun = kRunSeeds * kClThreads;
    auto singleton_runs = [&]() {
        if (!a.pn) return;
        while (n_un > 0) {
            int s[kRunSeeds], np[kRunSeeds];
#pragma unroll
            for (int u = 0; u < kRunSeeds; ++u) {
                const int at = n_un - 1 - (t + kClThreads * u);
                s[u] = at >= 0 ? a.un[at] : -1;
            }
#pragma unroll
            for (int u = 0; u < kRunSeeds; ++u) np[u] = s[u] >= 0 ? a.pn[s[u]] : -1;
            int first = kRun;  // this thread's first offset whose seed is not alone
#pragma unroll
            for (int u = 0; u < kRunSeeds; ++u) {
                const int k = t + kClThreads * u, at = n_un - 1 - k;
                bool alone = s[u] >= 0 && np[u] >= 0 && np[u] <= kPartnerCap;
                for (int e = 0; alone && e < np[u]; ++e) {
                    const int pr = a.pos[a.partners[(int64_t)s[u] * kPartnerCap + e]];
                    if (pr >= 0 && pr < at) alone = false;
                }
                if (!alone && k < first) first = k;
            }
            const int run = -block_max(-first, red);  // the first seed not alone
#pragma unroll
            for (int u = 0; u < kRunSeeds; ++u) {
                const int k = t + kClThreads * u;
                if (k < run) {
                    perm[out + k] = (I)s[u];
                    a.pos[s[u]] = -1;
                }
            }
            out += run;
            n_un -= run;
            phase_sync();
            if (run < kRun) return;
        }
    };

    // Highest position of an unclustered partner of `seed` (-1: none), or
    // -2 when the seed's partner list is unknown.  Two barriers.
    auto first_partner = [&](int seed) -> int {
        const int np = a.pn ? a.pn[seed] : -1;
        if (np < 0 || np > kPartnerCap) return -2;
        int key = -1;
        if (t < np) {
            const int pr = a.pos[a.partners[(int64_t)seed * kPartnerCap + t]];
            if (pr >= 0) key = pr;
        }
        return block_max(key, red);
    };

    // Commit the rows at the window positions hi - t with `flag` set, in
    // visiting order (descending position), with the reference's
    // swap-removes -- the j-th commit (j = 1, 2, ...) moves the row then at
    // position n0 - j, the end of `un`, into the freed position -- computed
    // in parallel.  With k commits the new end is nf = n0 - k, every move
    // source lies in [nf, n0), and a freed position below nf ends up with
    // the row its source held at that time: the source's own row if it was
    // not committed, else (it was freed earlier, as the j'-th commit) the row
    // that came from n0 - j', and so on up.  Those chains climb [nf, n0),
    // so pointer jumping over k slots resolves them in log2(k) + 1 rounds.
    auto commit_flagged = [&](int hi, bool flag) {
        const int at = hi - t;
        int64_t total;
        const int rank = (int)block_exscan64(flag ? 1 : 0, &total, red64);  // t ascending = position descending
        const int k = (int)total;
        if (k == 0) return;
        const int n0 = n_un, nf = n0 - k;
        int32_t row = -1;
        if (flag) {
            row = a.un[at];
            perm[out + rank] = (I)row;
            s_rank[t] = rank;
        }
        s_flag[t] = flag ? 1 : 0;
        __syncthreads();
        if (t < k) {  // slot t: position q = nf + t
            const int q = nf + t;
            const int tw = hi - q;  // its window slot, when q <= hi (q >= nf > hi - kClThreads)
            int nx = -1;
            if (tw >= 0 && s_flag[tw]) {
                const int src = n0 - 1 - s_rank[tw];  // the source of q's own commit
                nx = src == q ? -1 : src - nf;         // src == q: q was the end itself, popped
            } else {
                s_val[t] = a.un[q];
            }
            s_nxt[t] = nx;
        }
        __syncthreads();
        for (int len = 1; len <= k; len <<= 1) {
            int nx = -1, v = 0;
            if (t < k) {
                nx = s_nxt[t];
                if (nx >= 0) {
                    v = s_val[nx];
                    nx = s_nxt[nx];
                }
            }
            __syncthreads();
            if (t < k && s_nxt[t] >= 0) {
                s_val[t] = v;
                s_nxt[t] = nx;
            }
            __syncthreads();
        }
        if (flag && at < nf) {
            const int32_t v = s_val[n0 - 1 - rank - nf];  // from the source of this commit
            a.un[at] = v;
            a.pos[v] = at;
        }
        if (flag) a.pos[row] = -1;
        out += k;
        n_un = nf;
        phase_sync();
    };

    if (engine == kEngineScan) {
        while (n_un > 0) {
            singleton_runs();
            if (n_un == 0) break;
            const int seed = a.un[n_un - 1];
            --n_un;
            if (t == 0) {
                perm[out] = (I)seed;
                a.pos[seed] = -1;
            }
            ++out;
            // positions above the first partner cannot join: start there
            const int fp = first_partner(seed);
            if (fp == -1) {
                phase_sync();
                continue;  // no unclustered partner: a cluster of one
            }
            for (int w = t; w < W; w += kClThreads) p64[w] = a.bits[(int64_t)seed * W + w];
            int pc = a.count[seed];
            int hi = fp >= 0 ? fp : n_un - 1;  // highest position not yet visited
            phase_sync();
            while (hi >= 0) {
                const int at = hi - t;
                // joiners: 2 at + 1 when q lies inside the pattern (joining
                // leaves it unchanged), 2 at when q grows it
                int key = -1;
                if (at >= 0) {
                    const int c = a.un[at];
                    const int qc = a.count[c];
                    const int mn = qc < pc ? qc : pc, mx = qc < pc ? pc : qc;
                    if (jt.may_close(mn, mx)) {  // |p&q| <= mn, |p|q| >= mx
                        const uint64_t* q = a.bits + (int64_t)c * W;
                        int inter = 0, uni = 0;
                        for (int w = 0; w < W; ++w) {
                            const uint64_t x = q[w], y = p64[w];
                            inter += __popcll(x & y);
                            uni += __popcll(x | y);
                        }
                        if (jt.close(inter, uni)) key = 2 * at + (inter == qc ? 1 : 0);
                    }
                }
                const int top = block_max(key, red);
                int best = top < 0 ? -1 : top >> 1;  // the first joiner in visiting order
                if (top >= 0 && (top & 1)) {
                    // Joiners inside the pattern leave it as it is, so every joiner
                    // down to the first one that grows it (best, or the window's
                    // end) was tested against the pattern it meets: thread 0
                    // commits those inside it in visiting order, with the
                    // reference's swap-removes (a row from above moves into each
                    // freed position), and best, if any, is committed below.
                    best = block_max((key >= 0 && !(key & 1)) ? key >> 1 : -1, red);
                    commit_flagged(hi, key >= 0 && (key & 1) && (key >> 1) > best);
                }
                if (best < 0) {
                    hi -= kClThreads;
                    continue;
                }
                const int c = a.un[best];
                int64_t add = 0;
                for (int w = t; w < W; w += kClThreads) {
                    const uint64_t q = a.bits[(int64_t)c * W + w], o = p64[w];
                    add += __popcll(q & ~o);
                    p64[w] = o | q;
                }
                pc += (int)block_sum64(add, red64);
                if (t == 0) {
                    perm[out] = (I)c;
                    const int moved = a.un[n_un - 1];
                    a.un[best] = moved;
                    a.pos[moved] = best;
                    a.pos[c] = -1;
                }
                ++out;
                --n_un;
                hi = best - 1;
                phase_sync();
            }
            __syncthreads();
        }
        return;
    }

    // ---- index engine (0 <= dist_thresh < 1) ----
    // Raise cnt of the not-yet-visited rows of the lists of plist[b0, b1);
    // rows whose cnt leaves zero are logged and appended to `cand`.
    auto touch = [&](int b0, int b1, int limit, int32_t* cand) {
        for (int c0 = b0; c0 < b1; c0 += kClThreads) {
            const int nb = b1 - c0 < kClThreads ? b1 - c0 : kClThreads;
            int64_t len = 0;
            if (t < nb) {
                const int32_t b = a.plist[c0 + t];
                s_blk[t] = b;
                len = a.bl_start[b + 1] - a.bl_start[b];
            }
            int64_t total;
            const int64_t ex = block_exscan64(len, &total, red64);
            if (t < nb) s_pre[t] = ex;
            if (t == 0) s_pre[nb] = total;
            __syncthreads();
            for (int64_t e = t; e < total; e += kClThreads) {
                int lo = 0, hi = nb - 1;  // last j with s_pre[j] <= e
                while (lo < hi) {
                    const int mid = (lo + hi + 1) >> 1;
                    if (s_pre[mid] <= e) lo = mid;
                    else hi = mid - 1;
                }
                const int32_t r = a.bl_rows[a.bl_start[s_blk[lo]] + (e - s_pre[lo])];
                const int pr = a.pos[r];
                if (pr < 0 || pr >= limit) continue;  // clustered or already visited
                if (atomicAdd(&a.cnt[r], 1) == 0) {
                    a.log[atomicAdd(&s_cnt[0], 1)] = r;
                    cand[atomicAdd(&s_cnt[1], 1)] = r;
                }
            }
            __syncthreads();
        }
    };

    while (n_un > 0) {
        singleton_runs();
        if (n_un == 0) break;
        const int seed = a.un[n_un - 1];
        --n_un;
        if (t == 0) {
            perm[out] = (I)seed;
            a.pos[seed] = -1;
        }
        ++out;
        phase_sync();

        if (a.count[seed] == 0) {
            // Empty pattern: the remaining empty rows join, in descending
            // position order, and the pattern stays empty.  A swap-remove at
            // position i moves in a row from above i, already visited.
            for (int hi = n_un - 1; hi >= 0; hi -= kClThreads) {
                const int at = hi - t;
                commit_flagged(hi, at >= 0 && a.count[a.un[at]] == 0);
            }
            continue;
        }

        const int fp = first_partner(seed);
        if (fp == -1) continue;  // no unclustered partner: a cluster of one

        // pattern := blocks of the seed
        {
            const int64_t rs = a.rb_start[seed];
            const int n = (int)(a.rb_start[seed + 1] - rs);
            for (int k = t; k < n; k += kClThreads) {
                const int32_t b = a.rb[rs + k];
                a.plist[k] = b;
                atomicOr(&p32[b >> 5], 1u << (b & 31));
            }
        }
        int pc = a.count[seed];
        // positions below limit are not yet visited; those above the first
        // partner cannot join and are skipped
        int limit = fp >= 0 ? fp + 1 : n_un;
        int32_t* cur = a.cand_a;
        int32_t* nxt = a.cand_b;
        phase_sync();
        touch(0, pc, limit, cur);
        phase_sync();

        for (;;) {
            const int ncand = s_cnt[1];
            __syncthreads();
            if (t == 0) s_cnt[1] = 0;
            __syncthreads();
            // test the candidates, keeping those still below the limit
            int key = -1;
            for (int k = t; k < ncand; k += kClThreads) {
                const int32_t r = cur[k];
                const int pr = a.pos[r];
                if (pr < 0 || pr >= limit) continue;
                nxt[atomicAdd(&s_cnt[1], 1)] = r;
                const int inter = __hip_atomic_load(&a.cnt[r], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                const int uni = pc + a.count[r] - inter;
                if (pr > key && jt.close(inter, uni)) key = pr;
            }
            const int best = block_max(key, red);
            int32_t* sw = cur;
            cur = nxt;
            nxt = sw;
            if (best < 0) break;
            const int r = a.un[best];
            if (t == 0) {
                perm[out] = (I)r;
                const int moved = a.un[n_un - 1];
                a.un[best] = moved;
                a.pos[moved] = best;
                a.pos[r] = -1;
            }
            ++out;
            --n_un;
            limit = best;
            if (t == 0) s_cnt[2] = pc;
            phase_sync();
            // blocks of r not yet in the pattern
            const int64_t rs = a.rb_start[r];
            const int n = (int)(a.rb_start[r + 1] - rs);
            for (int k = t; k < n; k += kClThreads) {
                const int32_t b = a.rb[rs + k];
                const uint32_t bit = 1u << (b & 31);
                if ((atomicOr(&p32[b >> 5], bit) & bit) == 0u) a.plist[atomicAdd(&s_cnt[2], 1)] = b;
            }
            phase_sync();
            const int pc_new = s_cnt[2];
            touch(pc, pc_new, limit, cur);  // new candidates join the compacted list
            pc = pc_new;
            phase_sync();
        }

        // reset the counters and the pattern
        const int nlog = s_cnt[0];
        for (int k = t; k < nlog; k += kClThreads)
            __hip_atomic_store(&a.cnt[a.log[k]], 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        for (int k = t; k < pc; k += kClThreads) {
            const int32_t b = a.plist[k];
            p32[b >> 5] = 0u;
        }
        phase_sync();
        if (t < 4) s_cnt[t] = 0;
        __syncthreads();
    }
}

}  // namespace

template <typename I>
void jaccard_clustering_device(int64_t M, int64_t K, int64_t nnz, const I* rp, const I* ci,
                               float dist_thresh, int64_t block_width, I* perm, hipStream_t s,
                               int* engine_used)
{
    if (M < 0 || K < 0 || nnz < 0) throw std::invalid_argument("CSR dimensions must be non-negative.");
    if (M == 0) return;  // reference :63
    if (block_width <= 0) throw std::invalid_argument("clustering: block_width must be positive.");
    const int64_t Kb = (K + block_width - 1) / block_width;
    if (!clustering_device_supported(M, K, block_width))
        throw std::invalid_argument("clustering: shape beyond the GPU engine's limits.");
    const int64_t W = Kb > 0 ? (Kb + 63) / 64 : 1;

    // One allocation for the fixed-size temporaries (a stream-ordered
    // allocation costs host time; the call makes two).  The pieces cleared
    // before use -- flags, the greedy's counters, partner counts and the row
    // bitmaps -- come first and are cleared by one memset.
    const int64_t nb = Kb > 0 ? Kb : 1;
    Carve cv;
    const size_t o_flags = cv.take(2 * sizeof(int));
    const size_t o_cnt = cv.take((size_t)M * sizeof(int32_t));
    const size_t o_pn = cv.take((size_t)M * sizeof(int32_t));
    const size_t o_bits = cv.take((size_t)(M * W) * sizeof(uint64_t));
    const size_t zeroed = cv.end;
    const size_t o_count = cv.take((size_t)M * sizeof(int32_t));
    const size_t o_rbs = cv.take((size_t)(M + 1) * sizeof(int64_t));
    const size_t o_blc = cv.take((size_t)nb * sizeof(int32_t));
    const size_t o_un = cv.take((size_t)M * sizeof(int32_t));
    const size_t o_pos = cv.take((size_t)M * sizeof(int32_t));
    const size_t o_logb = cv.take((size_t)M * sizeof(int32_t));
    const size_t o_ca = cv.take((size_t)M * sizeof(int32_t));
    const size_t o_cb = cv.take((size_t)M * sizeof(int32_t));
    const size_t o_plist = cv.take((size_t)nb * sizeof(int32_t));
    const size_t o_partners = cv.take((size_t)M * kPartnerCap * sizeof(int32_t));
    const size_t o_status = cv.take(2 * sizeof(int64_t));
    Scratch tmp(cv.end, s);
    char* const base = tmp.as<char>();
    XSPMM_HIP_CHECK(hipMemsetAsync(base, 0, zeroed, s));
    int* const bad = reinterpret_cast<int*>(base + o_flags);  // [0] bad column, [1] engine used
    uint64_t* const bits = reinterpret_cast<uint64_t*>(base + o_bits);
    int32_t* const count = reinterpret_cast<int32_t*>(base + o_count);
    int64_t* const rb_start = reinterpret_cast<int64_t*>(base + o_rbs);
    int32_t* const bl_count = reinterpret_cast<int32_t*>(base + o_blc);
    int32_t* const pn = reinterpret_cast<int32_t*>(base + o_pn);
    int32_t* const partners = reinterpret_cast<int32_t*>(base + o_partners);

    const unsigned grid = (unsigned)std::min<int64_t>((M + 3) / 4, 65536);
    const int sh = (block_width & (block_width - 1)) == 0 ? __builtin_ctzll((unsigned long long)block_width) : -1;
    // bitmaps of up to 64 words come with their popcounts
    const bool lds_bits = W <= 64;
    if (lds_bits)
        hipLaunchKernelGGL(pattern_bits_lds_kernel<I>, dim3(grid), dim3(kPrepThreads), 0, s, rp, ci, M, K,
                           nnz, block_width, sh, (int)W, bits, count, bad);
    else
        hipLaunchKernelGGL(pattern_bits_kernel<I>, dim3(grid), dim3(kPrepThreads), 0, s, rp, ci, M, K,
                           nnz, block_width, sh, W, bits, bad);
    XSPMM_LAUNCH_CHECK();
    // an out-of-range column (skipped by the kernel) is reported before
    // anything writes perm: here on the closed-form path, else with the row
    // list total below
    int h_bad = 0;
    auto check_bad = [&] {
        if (h_bad) throw std::invalid_argument("clustering: column index out of range.");
    };

    // d <= t never holds for t < 0 (or NaN) and always holds for t >= 1:
    // no row joins, or every row joins the first cluster in visiting order;
    // either way perm = [M-1, ..., 0].
    if (!(dist_thresh >= 0.0f && dist_thresh < 1.0f)) {
        XSPMM_HIP_CHECK(hipMemcpyAsync(&h_bad, bad, sizeof(int), hipMemcpyDeviceToHost, s));
        XSPMM_HIP_CHECK(hipStreamSynchronize(s));
        check_bad();
        hipLaunchKernelGGL(reversed_perm_kernel<I>, dim3((unsigned)std::min<int64_t>((M + 255) / 256, 4096)),
                           dim3(256), 0, s, perm, M);
        XSPMM_LAUNCH_CHECK();
        if (engine_used) *engine_used = 0;
        return;
    }

    if (!lds_bits) {
        hipLaunchKernelGGL(pattern_count_kernel, dim3(grid), dim3(kPrepThreads), 0, s, bits, M, W, count);
        XSPMM_LAUNCH_CHECK();
    }

    // Engine and partner method, decided here so that the per-row and
    // per-block lists are built only when a step reads them: the index
    // engine and the row-list partner pass do, the scan engine and the
    // bitmap partner pass do not.  The engine estimate needs only v_b.
    int engine = kEngineAuto;
    if (const char* e = std::getenv("XSPMM_CLUSTER_ENGINE")) {
        if (std::strcmp(e, "scan") == 0) engine = kEngineScan;
        else if (std::strcmp(e, "index") == 0) engine = kEngineIndex;
    }
    // XSPMM_CLUSTER_PARTNERS: off (every seed on the full path) or popcount
    // (all-pairs lists by VALU popcounts instead of the matrix cores)
    bool use_partners = true, popcount_partners = false;
    if (const char* e = std::getenv("XSPMM_CLUSTER_PARTNERS")) {
        use_partners = std::strcmp(e, "off") != 0;
        popcount_partners = std::strcmp(e, "popcount") == 0;
    }
    const bool bitmap_partners = W <= 32 && (double)M * (double)M * (double)W <= 6.4e10;
    // row list offsets: their total, sum_b v_b = sum_i |q_i|, bounds the
    // engine estimate: (sum v_b)^2 / Kb <= sum v_b^2 <= sum v_b * min(M, sum v_b)
    device_exclusive_scan(ArrayValue<int32_t>{count}, M, rb_start, s);
    int64_t* const status = reinterpret_cast<int64_t*>(base + o_status);
    hipLaunchKernelGGL(status_kernel, dim3(1), dim3(64), 0, s, rb_start + M, bad, status);
    XSPMM_LAUNCH_CHECK();
    // pinned, so that the copy does not hold the host: 16 bytes allocated
    // once per host thread and never freed (a call reads them before it
    // returns, so calls on one thread never share them)
    thread_local int64_t* h_status = nullptr;
    if (!h_status) XSPMM_HIP_CHECK(hipHostMalloc((void**)&h_status, 2 * sizeof(int64_t), hipHostMallocDefault));
    XSPMM_HIP_CHECK(hipMemcpyAsync(h_status, status, 2 * sizeof(int64_t), hipMemcpyDeviceToHost, s));
    EventHandle copied;
    XSPMM_HIP_CHECK(hipEventRecord(copied.get(), s));

    // Partner lists (XSPMM_CLUSTER_PARTNERS=off leaves every seed on the
    // full path); pn starts at zero.  The all-pairs passes need only the
    // bitmaps and counts: they are enqueued before the host waits for the
    // copy of the row list total, so the host decides and enqueues the rest
    // while they run.  The row-list pass runs after the lists are built.
    if (use_partners && bitmap_partners) {
        const int Mi = (int)M, Wi = (int)W;
        if (bitmap_partners && !popcount_partners) {
            const int64_t T = (M + kGramTile - 1) / kGramTile;
            const dim3 g((unsigned)(T * (T + 1) / 2));
            auto kern = W <= 4 ? partners_gram_kernel<1> : W <= 8 ? partners_gram_kernel<2>
                      : W <= 16 ? partners_gram_kernel<4> : partners_gram_kernel<8>;
            hipLaunchKernelGGL(kern, g, dim3(256), 0, s, bits, count, Mi, Wi, (int)T, dist_thresh, pn,
                               partners);
        } else {
            // about 2048 workgroups: the rows j are split over grid.y
            const int64_t gx = (M + kPairRows - 1) / kPairRows;
            const int64_t tiles = (M + kPairTile - 1) / kPairTile;
            const dim3 g((unsigned)gx, (unsigned)std::max<int64_t>(1, std::min<int64_t>(tiles, 2048 / gx)));
            auto kern = W <= 8 ? partners_bitmap_kernel<8> : W <= 16 ? partners_bitmap_kernel<16>
                                                                      : partners_bitmap_kernel<32>;
            hipLaunchKernelGGL(kern, g, dim3(256), 0, s, bits, count, Mi, Wi, dist_thresh, pn, partners);
        }
        XSPMM_LAUNCH_CHECK();
    }

    XSPMM_HIP_CHECK(hipEventSynchronize(copied.get()));
    const int64_t nrb = h_status[0];
    h_bad = (int)h_status[1];
    check_bad();
    const double scan_work = 0.5 * (double)M * (double)M * (double)W;
    if (engine == kEngineAuto && Kb > 0) {
        const double sv = (double)nrb;
        if (3.0 * sv * sv / (double)Kb >= scan_work) engine = kEngineScan;
        else if (3.0 * sv * std::min(sv, (double)M) < scan_work) engine = kEngineIndex;
    }
    if (engine == kEngineAuto) {
        XSPMM_HIP_CHECK(hipMemsetAsync(bl_count, 0, (size_t)nb * sizeof(int32_t), s));
        const int64_t gy = std::max<int64_t>(1, std::min<int64_t>(1024, (M + 255) / 256));
        hipLaunchKernelGGL(block_counts_kernel, dim3((unsigned)((nb + kPrepThreads - 1) / kPrepThreads), (unsigned)gy),
                           dim3(kPrepThreads), 0, s, bits, M, W, Kb, bl_count);
        XSPMM_LAUNCH_CHECK();
        std::vector<int32_t> h_bl((size_t)nb);
        XSPMM_HIP_CHECK(hipMemcpyAsync(h_bl.data(), bl_count, (size_t)nb * sizeof(int32_t),
                                       hipMemcpyDeviceToHost, s));
        XSPMM_HIP_CHECK(hipStreamSynchronize(s));
        int64_t sq = 0;
        for (int64_t b = 0; b < Kb; ++b) sq += (int64_t)h_bl[(size_t)b] * h_bl[(size_t)b];
        // the same estimate as the host engines: index ~ 3 * sum v_b^2
        // counter updates, scan ~ M^2 * W / 2 word tests
        engine = 3.0 * (double)sq < scan_work ? kEngineIndex : kEngineScan;
    }
    const bool need_lists = engine == kEngineIndex || (use_partners && !bitmap_partners);

    // the per-row block lists and per-block row lists (nrb entries each)
    Scratch lists;
    int32_t* rb = nullptr;
    int64_t* bl_start = nullptr;
    int32_t* bl_rows = nullptr;
    int32_t* bl_cnt = nullptr;
    if (need_lists) {
        Carve lc;
        const size_t o_rb = lc.take((size_t)(nrb > 0 ? nrb : 1) * sizeof(int32_t));
        const size_t o_bls = lc.take((size_t)(nb + 1) * sizeof(int64_t));
        const size_t o_blr = lc.take((size_t)(nrb > 0 ? nrb : 1) * sizeof(int32_t));
        const size_t o_blc2 = lc.take((size_t)(nrb > 0 ? nrb : 1) * sizeof(int32_t));
        lists = Scratch(lc.end, s);
        bl_cnt = reinterpret_cast<int32_t*>(lists.as<char>() + o_blc2);
        rb = reinterpret_cast<int32_t*>(lists.as<char>() + o_rb);
        bl_start = reinterpret_cast<int64_t*>(lists.as<char>() + o_bls);
        bl_rows = reinterpret_cast<int32_t*>(lists.as<char>() + o_blr);
        XSPMM_HIP_CHECK(hipMemsetAsync(bl_count, 0, (size_t)nb * sizeof(int32_t), s));
        hipLaunchKernelGGL(row_lists_kernel, dim3(grid), dim3(kPrepThreads), 0, s, bits, M, W, rb_start,
                           rb, bl_count);
        XSPMM_LAUNCH_CHECK();
        device_exclusive_scan(ArrayValue<int32_t>{bl_count}, nb, bl_start, s);
        XSPMM_HIP_CHECK(hipMemsetAsync(bl_count, 0, (size_t)nb * sizeof(int32_t), s));
        hipLaunchKernelGGL(block_lists_kernel, dim3(grid), dim3(kPrepThreads), 0, s, M, rb_start, rb,
                           bl_start, bl_count, bl_rows, bl_cnt);
        XSPMM_LAUNCH_CHECK();
    }
    if (use_partners && !bitmap_partners) {
        hipLaunchKernelGGL(partners_index_kernel, dim3((unsigned)std::min<int64_t>(M, 1024)),
                           dim3(1024), 0, s, (int)M, rb_start, rb, bl_start, bl_rows, bl_cnt, count,
                           dist_thresh, pn, partners);
        XSPMM_LAUNCH_CHECK();
    }

    auto at = [&](size_t o) { return reinterpret_cast<int32_t*>(base + o); };
    ClusterArgs args{M, W, Kb, dist_thresh, engine, bits, count, rb_start, rb, bl_start, bl_rows,
                     at(o_un), at(o_pos), at(o_cnt), at(o_logb), at(o_ca), at(o_cb), at(o_plist),
                     use_partners ? pn : nullptr, partners, bad + 1};
    hipLaunchKernelGGL(cluster_kernel<I>, dim3(1), dim3(kClThreads), 0, s, args, perm);
    XSPMM_LAUNCH_CHECK();
    if (engine_used) {
        XSPMM_HIP_CHECK(hipMemcpyAsync(engine_used, bad + 1, sizeof(int), hipMemcpyDeviceToHost, s));
        XSPMM_HIP_CHECK(hipStreamSynchronize(s));
    }
}

bool clustering_device_supported(int64_t M, int64_t K, int64_t block_width)
{
    // row positions are doubled in the scan's joiner keys: M < 2^30
    if (block_width <= 0 || M >= (int64_t)1 << 30) return false;
    const int64_t Kb = (K + block_width - 1) / block_width;
    if (Kb > kMaxGpuBlocks) return false;
    const int64_t W = Kb > 0 ? (Kb + 63) / 64 : 1;
    return (double)M * (double)W * 8.0 <= 16.0 * (1ULL << 30);  // row bitmaps <= 16 GiB
}

template void jaccard_clustering_device<int32_t>(int64_t, int64_t, int64_t, const int32_t*,
                                                 const int32_t*, float, int64_t, int32_t*,
                                                 hipStream_t, int*);
template void jaccard_clustering_device<int64_t>(int64_t, int64_t, int64_t, const int64_t*,
                                                 const int64_t*, float, int64_t, int64_t*,
                                                 hipStream_t, int*);

}  // namespace detail
}  // namespace xspmm
