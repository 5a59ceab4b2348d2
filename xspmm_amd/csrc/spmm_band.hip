// spmm_band.hip -- Tier-1 BCSR SpMM (fp16) for grids whose block-rows are
// contiguous runs of block columns that neighbouring block-rows share: banded
// and block-banded matrices (the density sweep of the reference's
// examples/05_core_spmm_benchmark.cpp:56-77 is of this shape).
//
// In such a grid the column-batch kernel gathers the same B rows once for
// every block-row that meets them: at the 90 % band (16384^2, N = 128) that is
// 3 GB of B rows out of L2 for a 0.4 GB product, and the gathers bound it.
// Here a workgroup owns four consecutive block-rows (a group) and one
// 128-column chunk of C, and walks the union of their block columns once, in
// aligned pairs (block columns 2p and 2p + 1, i.e. B rows 32p .. 32p + 31).
// Eight waves, two per block-row, each with 64 of the columns (two waves per
// SIMD, so one hides the other's waits):
//   * each pair's 32 x 128 B tile is loaded once for the four rows -- each wave
//     loads 4 of its rows into registers L pairs ahead and writes them into
//     one of three LDS stages two pairs ahead, so a B row leaves L2 once per
//     group instead of once per block-row;
//   * each wave loads its row's two blocks of the pair straight into the
//     v_mfma_f32_16x16x32_f16 A operand (one 16-byte load per lane, L pairs
//     ahead); a block the row does not hold reads as zeros;
//   * each wave reads the next pair's tile back with the gfx950 transpose
//     read ds_read_b64_tr_b16 (the B operands of its 4 column tiles) while
//     this pair's 4 MFMAs run; one s_barrier per pair hands the stages over,
//     waiting only for the wave's LDS writes (its reads stay in flight);
//   * XCD x (workgroups go to the 8 XCDs round-robin) takes a contiguous range
//     of groups, so neighbouring groups, which walk the same B tiles a few
//     pairs apart, meet them in one L2.
// A row's block (br, c) sits at index row_ptr[br] + c - col_ind[row_ptr[br]]
// (the row is contiguous), so no column index is read inside the loop.  The
// Tier-1 entry points take this kernel only for grids checked to have
// contiguous rows (spmm_band_wanted); on any other grid every access still
// stays inside A and B (buffer resources with their sizes), but C would be
// wrong.
//
// Semantics are those of the tile kernel (reference
// src/common/spmm_math.hpp:20-146): each block a row holds multiplies all 16
// of its columns, and B rows meet a row only through the blocks it holds (so
// an Inf/NaN in B gives NaN exactly where the reference's would), fp32
// accumulators, C overwritten; rows >= M and columns >= N are not stored and
// B rows >= K contribute nothing.  A row's pairs accumulate in ascending
// column order, the same order on every call.
//
// The fp32 kernel (spmm_f32_band_kernel, below) shares each B load of a
// group in registers instead (v_mfma_f32_16x16x4f32 takes B rows as they lie
// in memory) and is bound by the matrix cores of each CU.  Where one group
// per workgroup would leave CUs idle (the band's edge groups hold half the
// centre's blocks; a small grid fills few workgroup slots), it runs a
// balanced launch: band_plan_kernel cuts the groups' blocks into one equal
// share per CU, and a group cut between shares is summed from its parts'
// partial tiles in part order by the part that arrives last.
#include <algorithm>
#include <atomic>
#include <cmath>
#include <cstdint>
#include <cstdlib>
#include <string>

#include "internal.hpp"

namespace xspmm {
namespace detail {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

constexpr int kBandRows = 4;        // block-rows per workgroup (a group)
constexpr int kBandTile = 32 * 256; // LDS stage: 32 B rows x 128 fp16 columns
constexpr uint32_t kOob = 0x80000000u;  // a buffer offset past every resource: reads zeros
// cache policy of a buffer access that is coherent across the XCDs (sc1: the
// policy of relaxed agent-scope atomic loads and stores)
constexpr int kAgentCoherent = 16;

#ifndef XSPMM_BAND_DEPTH
#define XSPMM_BAND_DEPTH 6
#endif
static_assert(XSPMM_BAND_DEPTH >= 6 && XSPMM_BAND_DEPTH <= 18, "band ring depth 6 .. 18");
#ifndef XSPMM_BAND_XCD
#define XSPMM_BAND_XCD 1
#endif
constexpr bool kBandXcd = XSPMM_BAND_XCD != 0;
#ifndef XSPMM_BAND_F32_DEPTH
#define XSPMM_BAND_F32_DEPTH 4
#endif
#ifndef XSPMM_BAND_WPR
#define XSPMM_BAND_WPR 2
#endif

constexpr int kRawBufferWord3 = 0x00020000;
__device__ __forceinline__ __amdgpu_buffer_rsrc_t band_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kRawBufferWord3);
}

// swizzle of tile row e (16-byte chunk c of the row is stored at chunk
// c ^ swz(e)): the 16 rows one transpose read touches spread over all banks
__device__ __forceinline__ uint32_t band_swz(uint32_t e)
{
    return 2u * ((e & 3u) | (((e >> 3) & 1u) << 2));
}

// The barrier that publishes a wave's LDS writes: every LDS access of this
// wave done, then the workgroup meets.  The memory clobber keeps the compiler
// from moving LDS accesses across it; outstanding global loads (the ring)
// stay in flight.
__device__ __forceinline__ void band_barrier()
{
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}
// The same when this wave issued its LDS writes before R >= 1 LDS reads (LDS
// operations of a wave complete in order): the writes are done once at most R
// operations are outstanding, and the reads may stay in flight across the
// barrier (their consumers wait for them).
template <int R>
__device__ __forceinline__ void band_barrier_writes()
{
    static_assert(R >= 1 && R <= 15, "lgkmcnt holds 0 .. 15");
    asm volatile("s_waitcnt lgkmcnt(%0)\n\ts_barrier" ::"n"(R) : "memory");
}

// WPR: waves per block-row (1: a wave owns its row's 128 columns; 2: two
// waves split them, 8 waves per workgroup, two per SIMD).
template <typename I, int L, int WPR>
__global__ __launch_bounds__(64 * kBandRows * WPR) void spmm_f16_band_kernel(
    const I* __restrict__ brp, const I* __restrict__ bci, const uint16_t* __restrict__ vals,
    const uint16_t* __restrict__ B, float* __restrict__ C, int64_t M, int64_t K, int64_t N,
    int64_t Mb, const I* __restrict__ row_map)
{
    static_assert(WPR == 1 || WPR == 2, "one or two waves per block-row");
    static_assert(L % 6 == 0, "ring depth a multiple of 6 (ring slot, stage and operand set align)");
    constexpr int W = kBandRows * WPR;  // waves per workgroup
    constexpr int NT = 8 / WPR;         // 16-column tiles per wave
    constexpr int LB = 8 / W;           // this wave's 1 KB B loads per pair (8 per tile)
    __shared__ __align__(16) unsigned char stage[3][kBandTile];
    // 8 rows of a tile, all zero: the transpose reads of a B-operand half
    // that a row's missing block would multiply come from here
    __shared__ __align__(16) unsigned char zeros[8 * 256];
    __shared__ int32_t s_first[kBandRows];
    __shared__ int32_t s_last[kBandRows];

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15;
    const int g = lane >> 4;
    const int row = wave % kBandRows;  // this wave's block-row in the group
    const int cs = wave / kBandRows;   // and its column slice (16 NT columns)
    // group of this workgroup: workgroups go to the 8 XCDs round-robin, and
    // XCD x takes a contiguous range of groups (start x * (G / 8) +
    // min(x, G % 8)), so neighbouring groups, which walk the same B tiles a
    // few pairs apart, meet them in one L2
    const uint32_t G = gridDim.x;
    const uint32_t x8 = blockIdx.x & 7u;
    const uint32_t grp = kBandXcd ? x8 * (G >> 3) + min(x8, G & 7u) + (blockIdx.x >> 3) : blockIdx.x;
    const int64_t br0 = (int64_t)grp * kBandRows;
    const int64_t n0 = (int64_t)blockIdx.y * 128;

    // this wave's row: its blocks, and first / last block column
    const int64_t br = br0 + row;
    int64_t rs = 0, re = 0;
    if (br < Mb) {
        rs = (int64_t)brp[br];
        re = (int64_t)brp[br + 1];
    }
    const int32_t nblk = (int32_t)(re - rs);
    if (cs == 0 && lane == 0) {
        s_first[row] = nblk > 0 ? (int32_t)bci[rs] : 0x7fffffff;
        s_last[row] = nblk > 0 ? (int32_t)bci[re - 1] : -1;
    }
    for (int i = threadIdx.x; i < 8 * 256 / 4; i += 64 * W) reinterpret_cast<uint32_t*>(zeros)[i] = 0u;
    __syncthreads();
    int32_t lo = 0x7fffffff, hi = -1;
#pragma unroll
    for (int w = 0; w < kBandRows; ++w) {
        lo = min(lo, s_first[w]);
        hi = max(hi, s_last[w]);
    }
    // pairs of the group's span (aligned block-column pairs)
    const int32_t p0 = hi >= 0 ? (lo >> 1) : 0;
    const int32_t steps = hi >= 0 ? (hi >> 1) - p0 + 1 : 0;

    // A of the row: lane (li, g) reads row li, columns 8 (g & 1) .. + 7 of
    // block 2p + (g >> 1); blocks outside the row read as zeros
    const __amdgpu_buffer_rsrc_t a_rsrc = band_rsrc(vals + rs * 256, (uint32_t)nblk * 512u);
    const int32_t r_rel0 = 2 * p0 - s_first[row];  // index in the row of block 2 p0 (uniform)
    const int32_t a_rel0 = r_rel0 + (g >> 1);       // this lane's block at pair 0
    const uint32_t a_lane = (uint32_t)(li * 32 + (g & 1) * 16);
    auto a_off = [&](int32_t t) __attribute__((always_inline)) -> uint32_t {
        const int32_t rel = a_rel0 + 2 * t;
        return (uint32_t)rel < (uint32_t)nblk ? (uint32_t)rel * 512u + a_lane : kOob;
    };

    // B rows of the tile: load v of this wave moves tile rows
    // 4 (LB wave + v) + lane / 16, chunk lane % 16 (written at chunk position
    // chunk ^ swz(row)).  Rows past K read as zeros (their offsets pass the
    // end of B).  A chunk past N (last column chunk, N % 128 != 0) loads the
    // row's last chunk instead: it only meets columns of C that are not
    // stored.
    const __amdgpu_buffer_rsrc_t b_rsrc = band_rsrc(B, (uint32_t)(K * N * 2));
    const uint32_t rowbytes = (uint32_t)(2 * N);
    uint32_t b_col[LB], b_row0[LB], st_w[LB];
#pragma unroll
    for (int v = 0; v < LB; ++v) {
        const uint32_t e = (uint32_t)(4 * (LB * wave + v) + (lane >> 4));
        const uint32_t ch = (uint32_t)(lane & 15);
        const int64_t col = n0 + 8 * (int64_t)ch;
        b_col[v] = (uint32_t)(2 * (col < N ? col : N - 8));
        b_row0[v] = (uint32_t)(32 * p0) + e;
        st_w[v] = e * 256u + 16u * (ch ^ band_swz(e));
    }
    auto b_off = [&](int32_t t, int v) __attribute__((always_inline)) -> uint32_t {
        return __umul24(b_row0[v] + 32u * (uint32_t)t, rowbytes) + b_col[v];
    };

    // transpose-read address of column tile j of the tile: tr_a0 ^ 32 j
    const uint32_t tr_e0 = (uint32_t)(8 * g + (li >> 2));
    const uint32_t tr_a0 = (tr_e0 * 256u + 16u * (uint32_t)((li & 3) >> 1) + 8u * (uint32_t)(li & 1)) ^
                           (band_swz(tr_e0) << 4);

    float4_t acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

    // ring of L pairs in flight (A operand and this wave's B rows per pair),
    // three LDS stages (pair t in stage t % 3) and the B operands of two
    // pairs (the one being multiplied and the next)
    half8_t ar[L];
    u32x4_t bq[L][LB];
    half8_t bop[2][NT];
    auto issue = [&](int slot, int32_t t) __attribute__((always_inline)) {
        ar[slot] = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, (int)a_off(t), 0, 0));
#pragma unroll
        for (int v = 0; v < LB; ++v)
            bq[slot][v] = __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)b_off(t, v), 0, 0));
    };
    auto put = [&](int slot, int st) __attribute__((always_inline)) {
#pragma unroll
        for (int v = 0; v < LB; ++v) *reinterpret_cast<u32x4_t*>(&stage[st][st_w[v]]) = bq[slot][v];
    };
    // Operands of pair t (tile in stage st) into operand set o.  With both
    // of the row's blocks of the pair present (the row's interior) they come
    // from the tile; otherwise the lanes of the half that a missing block
    // would multiply (lane group g >= 2 carries block 2p + 1) read the same
    // positions of `zeros` instead (a row holding neither block adds zeros).
    // So B rows meet a row only through blocks it holds, as in the
    // reference's tile product: an Inf or NaN in B gives NaN exactly where a
    // held block covers it, never through a neighbour's span.  Lane group g's
    // transpose reads touch tile rows 8g .. 8g + 7 only.
    const uint32_t z_base = (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)zeros -
                            (uint32_t)(8 * g * 256);
    auto fetch = [&](int st, int o, int32_t t) __attribute__((always_inline)) {
        const int32_t b0 = r_rel0 + 2 * t;
        const bool has0 = (uint32_t)b0 < (uint32_t)nblk;
        const bool has1 = (uint32_t)(b0 + 1) < (uint32_t)nblk;
        const bool keep = (g >= 2) ? has1 : has0;
        const uint32_t base =
            keep ? (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) unsigned char*)stage[st] : z_base;
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const uint32_t a = base + (tr_a0 ^ (uint32_t)(32 * (cs * NT + j)));
            typedef __attribute__((address_space(3))) short4_t* lp_t;
            const short4_t blo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp_t)(uintptr_t)a);
            const short4_t bhi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lp_t)(uintptr_t)(a + 4 * 256));
            bop[o][j] = __builtin_bit_cast(half8_t, __builtin_shufflevector(blo, bhi, 0, 1, 2, 3, 4, 5, 6, 7));
        }
    };
    auto multiply = [&](int slot, int o) __attribute__((always_inline)) {
#pragma unroll
        for (int j = 0; j < NT; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ar[slot], bop[o][j], acc[j], 0, 0, 0);
    };

    if (steps > 0) {
        // prologue: pairs 0 .. L-1 in flight, pairs 0 and 1 in stages 0 and
        // 1, pair 0's operands read
#pragma unroll
        for (int t = 0; t < L; ++t) issue(t, t);
        put(0, 0);
        put(1, 1);
        band_barrier();
        fetch(0, 0, 0);
        for (int32_t s0 = 0; s0 < steps; s0 += L) {
#pragma unroll
            for (int u = 0; u < L; ++u) {
                const int32_t s = s0 + u;
                // pair s + 2's rows into the stage pair s - 1 used (its
                // readers passed the barrier of pair s - 1), pair s's MFMAs
                // (operands read before the last barrier), pair s + 1's
                // operands out of its stage (written before the last
                // barrier) while they run, then pair s + L's loads into the
                // slot pair s used
                if (s + 2 < steps) put((u + 2) % L, (u + 2) % 3);
                if (s < steps) multiply(u, u & 1);
                asm volatile("" ::: "memory");
                if (s + 1 < steps) fetch((u + 1) % 3, (u + 1) & 1, s + 1);
                issue(u, s + L);
                // pair s + 2's writes (when made, pair s + 1's 2 NT reads
                // follow them) must land before the barrier; pair s + 1's
                // reads are consumed by its MFMAs before the next barrier
                band_barrier_writes<2 * NT < 15 ? 2 * NT : 14>();
            }
        }
    }

    // store: lane (li, g) holds rows 4g .. 4g + 3 of column 16 j + li of
    // the wave's tiles
    if (br < Mb) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int64_t grow = br * 16 + 4 * g + q;
            if (grow >= M) continue;
            const int64_t crow = row_map ? (int64_t)row_map[grow] : grow;
            const int64_t c0 = n0 + 16 * cs * NT + li;
            float* dst = C + crow * N + c0;
#pragma unroll
            for (int j = 0; j < NT; ++j)
                if (c0 + 16 * j < N) dst[16 * j] = acc[j][q];
        }
    }
}

// The balanced launch of the fp32 band kernel: the groups' block counts,
// laid end to end (S[g] = blocks of the spans of groups 0 .. g - 1, S[G] =
// all), are cut into P ranges of about equal size, one per workgroup slot
// and column chunk, so every CU gets the same number of MFMAs however the
// band's width varies along the diagonal.  A border that falls close to a
// group border moves onto it (a band of even width cuts no group).  A slot
// walks the groups its range meets: a group it holds whole is stored into
// C; a group cut by a border is summed from its parts: each part writes its
// partial tile, then counts itself in `arrivals`, and the part that arrives
// last adds the partial tiles in part order (part 0 + part 1 + ...) and
// stores C, so C is the same bit for bit whichever part arrives last.
struct BandSplit {
    const int64_t* S;      // G + 1: prefix of the groups' block counts
    const int64_t* bnd;    // P + 1: slot p's range is [bnd[p], bnd[p + 1])
    const int32_t* first;  // P: the first group slot p's range meets
    const int32_t* plo;    // G: the first slot meeting group g
    const int32_t* parts;  // G: the slots meeting group g (1: one holds it whole)
    int32_t* arrivals;     // chunks x P: parts counted of the cut group that slot starts
    float* tiles;          // chunks x 2 x P partial tiles of kBandPart32 floats
    int64_t G;             // groups
    int32_t P;             // slots, a multiple of 8
};
constexpr int kBandPart32 = 4 * 16 * 64;  // a group's 64 x 64 fp32 tile
constexpr int kPlanGroups = 4096;         // most groups a balanced launch plans
constexpr int kPlanSlots = 1024;          // most slots

// Blocks in the union of group grp's block-rows' spans (rows are contiguous
// runs, so a row spans col_ind[first] .. col_ind[last]); 0 when it holds none.
// The five row pointers load together, then the eight column indices (from
// indices clamped into [0, nnzb): the balanced launch is taken only for grids
// with blocks, nnzb >= 1, so nothing is read past col_ind).
template <typename I>
__device__ __forceinline__ int64_t band_group_blocks(const I* brp, const I* bci, int64_t Mb, int64_t nnzb,
                                                     int64_t grp)
{
    int64_t rp[5];
#pragma unroll
    for (int w = 0; w < 5; ++w) rp[w] = (int64_t)brp[min(grp * 4 + w, Mb)];
    int64_t f[4], l[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        f[w] = (int64_t)bci[min(max(rp[w], (int64_t)0), nnzb - 1)];
        l[w] = (int64_t)bci[min(max(rp[w + 1] - 1, (int64_t)0), nnzb - 1)];
    }
    int64_t lo = INT64_MAX, hi = -1;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        if (grp * 4 + w >= Mb || rp[w + 1] <= rp[w]) continue;
        lo = min(lo, f[w]);
        hi = max(hi, l[w]);
    }
    return hi >= 0 ? hi - lo + 1 : 0;
}

// The balanced launch's plan, one workgroup, in LDS: the prefix S, the slot
// borders, each slot's first group, each group's first slot and part count,
// and the arrival counts cleared.
template <typename I>
__global__ __launch_bounds__(1024) void band_plan_kernel(const I* __restrict__ brp, const I* __restrict__ bci,
                                                          int64_t Mb, int64_t nnzb, BandSplit sp, int32_t chunks)
{
    __shared__ int64_t s_S[kPlanGroups + 1];
    __shared__ int64_t s_b[kPlanSlots + 1];
    __shared__ int64_t red[16];
    const int32_t G = (int32_t)sp.G;
    const int32_t P = sp.P;
    for (int32_t g = threadIdx.x; g < G; g += 1024) s_S[g + 1] = band_group_blocks(brp, bci, Mb, nnzb, g);
    __syncthreads();
    // prefix: thread i scans a run of consecutive groups from the sum of the
    // runs before it
    const int32_t per = (G + 1023) / 1024;
    const int32_t a = min(G, (int32_t)threadIdx.x * per), b = min(G, a + per);
    int64_t own = 0;
    for (int32_t i = a; i < b; ++i) own += s_S[i + 1];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int64_t incl = own;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t t = __shfl_up(incl, d, 64);
        if (lane >= d) incl += t;
    }
    if (lane == 63) red[wave] = incl;
    __syncthreads();
    int64_t run = incl - own;
    for (int w = 0; w < wave; ++w) run += red[w];
    for (int32_t i = a; i < b; ++i) {
        run += s_S[i + 1];
        s_S[i + 1] = run;
    }
    if (threadIdx.x == 0) s_S[0] = 0;
    __syncthreads();
    const int64_t total = s_S[G];
    // lower bound: the first g in [0, G] with s_S[g] >= x
    auto lower = [&](int64_t x) {
        int32_t lo = 0, hi = G;
        while (lo < hi) {
            const int32_t m = (lo + hi) >> 1;
            if (s_S[m] >= x) hi = m; else lo = m + 1;
        }
        return lo;
    };
    // slot borders: ceil(p total / P), moved onto a group border within
    // total / (16 P) of it
    const int64_t tol = total / (16 * (int64_t)P);
    for (int32_t p = threadIdx.x; p <= P; p += 1024) {
        int64_t x = ((int64_t)p * total + P - 1) / P;
        if (p > 0 && p < P) {
            const int32_t j = lower(x);
            int64_t best = s_S[j];  // j <= G and s_S[G] = total >= x
            if (j > 0 && x - s_S[j - 1] < best - x) best = s_S[j - 1];
            if (best - x <= tol && x - best <= tol) x = best;
        }
        s_b[p] = x;
        const_cast<int64_t*>(sp.bnd)[p] = x;
    }
    __syncthreads();
    // slot p's first group: the first one holding a unit from bnd[p] on, or
    // an empty group there
    for (int32_t p = threadIdx.x; p < P; p += 1024) {
        const int64_t beg = s_b[p];
        int32_t lo = 0, hi = G;  // first g with S[g + 1] > beg
        while (lo < hi) {
            const int32_t m = (lo + hi) >> 1;
            if (s_S[m + 1] > beg) hi = m; else lo = m + 1;
        }
        const_cast<int32_t*>(sp.first)[p] = min(lower(beg), lo);
    }
    // the slot holding unit x: the last p with bnd[p] <= x (x < total)
    auto holder = [&](int64_t x) {
        int32_t lo = 0, hi = P;  // first p in [0, P] with bnd[p] > x
        while (lo < hi) {
            const int32_t m = (lo + hi) >> 1;
            if (s_b[m] > x) hi = m; else lo = m + 1;
        }
        return lo - 1;
    };
    for (int32_t g = threadIdx.x; g < G; g += 1024) {
        const int64_t s0 = s_S[g], s1 = s_S[g + 1];
        int32_t plo = 0, parts = 1;
        if (s1 > s0) {
            plo = holder(s0);
            parts = holder(s1 - 1) - plo + 1;
        }
        const_cast<int32_t*>(sp.plo)[g] = plo;
        const_cast<int32_t*>(sp.parts)[g] = parts;
    }
    for (int32_t i = threadIdx.x; i <= G; i += 1024) const_cast<int64_t*>(sp.S)[i] = s_S[i];
    for (int64_t i = threadIdx.x; i < (int64_t)P * chunks; i += 1024) sp.arrivals[i] = 0;
}

// ---------------------------------------------------------------------------
// fp32 banded grids: spmm_f32_band_kernel.  v_mfma_f32_16x16x4f32 takes one K
// index per lane group (lane (i, k) holds A[i][k] and B[k][i]), so B rows go
// from memory straight into MFMA operands and a wave can apply them to
// several block-rows.  A workgroup owns a group of four consecutive block-rows
// and 64 columns of C; its 4 waves split the group's block-column span
// (wave w takes columns lo + w, lo + w + 4, ...), and each wave multiplies
// every block it meets into all four rows:
//   * B: for block column c, lane (n, g) loads row 16c + 4g + s, columns
//     n0 + 4n .. + 3 (one 16-byte load, s = 0 .. 3); component j of load s
//     is the B operand of MFMA (s, j), K slot g <-> block column 4g + s;
//   * A: per row, lane (i, g) loads row i, columns 4g .. 4g + 3 of the row's
//     block at c (one 16-byte load); component s is the A operand of MFMA
//     (s, j) -- the same K order;
//   * so one block's 4 B loads per lane serve 4 rows x 16 MFMAs; loads run L
//     blocks ahead, every block issues the same loads (a row without the
//     block, or a column past the span, reads zeros), and the MFMAs of a
//     row that does not hold the block are skipped, so B meets a row only
//     through the blocks it holds (an Inf or NaN in B gives NaN where the
//     reference's tile product would);
//   * the waves' partial tiles are summed through LDS in wave order.
// Output tile j of a wave holds columns n0 + 4n + j (lane (n, g): rows
// 4g .. 4g + 3), as in the fp32 column-batch kernel.  Each block-row must be
// one contiguous run of block columns (spmm_band_wanted); N % 4 == 0, B and C
// 16-byte aligned.  SPLIT: the balanced launch (grid P x chunks, with the plan
// of band_plan_kernel); otherwise one group per workgroup.
template <typename I, int L, bool SPLIT>
__global__ __launch_bounds__(256, 2) void spmm_f32_band_kernel(
    const I* __restrict__ brp, const I* __restrict__ bci, const float* __restrict__ vals,
    const float* __restrict__ B, float* __restrict__ C, int64_t M, int64_t K, int64_t N, int64_t Mb,
    const I* __restrict__ row_map, BandSplit sp)
{
    typedef float float4v_t __attribute__((ext_vector_type(4)));
    __shared__ __align__(16) float red[4 * 4 * 16 * 64];  // [wave][row][16][64]
    __shared__ int32_t s_first[4];
    __shared__ int32_t s_last[4];
    __shared__ int32_t s_arrived;

    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int li = lane & 15;
    const int g = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.y * 64;
    const uint32_t a_lane = (uint32_t)(li * 64 + g * 16);
    // B: lane (n, g) of load s reads row 16c + 4g + s, columns n0 + 4n .. +3
    // (a quad past N reads the row's last quad: it only meets unstored
    // columns); rows past K read zeros
    const __amdgpu_buffer_rsrc_t b_rsrc = band_rsrc(B, (uint32_t)(K * N * 4));
    const uint32_t rowbytes = (uint32_t)(4 * N);
    const int64_t colq = n0 + 4 * li;
    const uint32_t b_lane = (uint32_t)(4 * (colq < N ? colq : N - 4)) + __umul24((uint32_t)(4 * g), rowbytes);

    // Blocks t0 .. t1 - 1 of group grp's span (clamped to the span), summed
    // over the waves into red (wave order), which the workgroup reads after
    // the closing barrier.
    auto group_blocks = [&](int64_t grp, int32_t t0, int32_t t1) __attribute__((always_inline)) {
        const int64_t br0 = grp * 4;
        __syncthreads();  // the previous group's readers of s_first, s_last and red are done
        {
            const int64_t br = br0 + wave;
            int32_t first = 0x7fffffff, last = -1;
            if (br < Mb) {
                const int64_t rs = (int64_t)brp[br], re = (int64_t)brp[br + 1];
                if (re > rs) {
                    first = (int32_t)bci[rs];
                    last = (int32_t)bci[re - 1];
                }
            }
            if (lane == 0) {
                s_first[wave] = first;
                s_last[wave] = last;
            }
        }
        __syncthreads();
        int32_t lo = 0x7fffffff, hi = -1;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            lo = min(lo, s_first[w]);
            hi = max(hi, s_last[w]);
        }
        const int32_t span = hi >= 0 ? hi - lo + 1 : 0;
        t1 = min(t1, span);
        t0 = min(t0, t1);
        const int32_t steps = t1 - t0;
        const int32_t nt = steps > wave ? (steps - wave + 3) >> 2 : 0;  // this wave's blocks
        const int32_t c0 = lo + t0 + wave;                               // its first block column

        // rows: block c of row r at index c - first_r, present when in [0, n_r)
        __amdgpu_buffer_rsrc_t a_rsrc[4];
        int32_t r_rel0[4], r_n[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t br = br0 + r;
            int64_t rs = 0, re = 0;
            if (br < Mb) {
                rs = (int64_t)brp[br];
                re = (int64_t)brp[br + 1];
            }
            r_n[r] = (int32_t)(re - rs);
            a_rsrc[r] = band_rsrc(vals + rs * 256, (uint32_t)r_n[r] * 1024u);
            r_rel0[r] = c0 - s_first[r];
        }
        auto a_off = [&](int r, int32_t t) __attribute__((always_inline)) -> uint32_t {
            const int32_t rel = r_rel0[r] + 4 * t;
            return (uint32_t)rel < (uint32_t)r_n[r] ? (uint32_t)rel * 1024u + a_lane : kOob;
        };
        auto b_off = [&](int32_t t, int sidx) __attribute__((always_inline)) -> uint32_t {
            const int32_t c = c0 + 4 * t;
            return t < nt ? __umul24((uint32_t)(16 * c + sidx), rowbytes) + b_lane : kOob;
        };

        float4v_t acc[4][4];
#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[r][j] = float4v_t{0.f, 0.f, 0.f, 0.f};

        float4v_t ar[L][4];  // A of the wave's block t, four rows (slot t % L)
        float4v_t bq[L][4];  // its four B loads
        auto issue = [&](int slot, int32_t t) __attribute__((always_inline)) {
#pragma unroll
            for (int sidx = 0; sidx < 4; ++sidx)
                bq[slot][sidx] = __builtin_bit_cast(
                    float4v_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)b_off(t, sidx), 0, 0));
#pragma unroll
            for (int r = 0; r < 4; ++r)
                ar[slot][r] = __builtin_bit_cast(
                    float4v_t, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc[r], (int)a_off(r, t), 0, 0));
        };
        auto multiply = [&](int slot, int32_t t) __attribute__((always_inline)) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                // uniform: does row r hold this block?
                if ((uint32_t)(r_rel0[r] + 4 * t) < (uint32_t)r_n[r]) {
#pragma unroll
                    for (int sidx = 0; sidx < 4; ++sidx)
#pragma unroll
                        for (int j = 0; j < 4; ++j)
                            acc[r][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(ar[slot][r][sidx], bq[slot][sidx][j],
                                                                             acc[r][j], 0, 0, 0);
                }
            }
        };

        if (nt > 0) {
#pragma unroll
            for (int t = 0; t < L; ++t) issue(t, t);
            for (int32_t q0 = 0; q0 < nt; q0 += L) {
#pragma unroll
                for (int u = 0; u < L; ++u) {
                    const int32_t t = q0 + u;
                    if (t < nt) multiply(u, t);
                    issue(u, t + L);
                }
            }
        }

#pragma unroll
        for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int q = 0; q < 4; ++q)
                *reinterpret_cast<float4v_t*>(red + ((wave * 4 + r) * 16 + 4 * g + q) * 64 + 4 * li) =
                    float4v_t{acc[r][0][q], acc[r][1][q], acc[r][2][q], acc[r][3][q]};
        __syncthreads();
    };
    // quad e of the group's tile: block-row e / 256, row (e / 16) % 16,
    // columns 4 (e % 16) .. + 3; its sum over the waves, in wave order
    auto tile_quad = [&](int e) __attribute__((always_inline)) -> float4v_t {
        const int o = e * 4;
        float4v_t v = *reinterpret_cast<const float4v_t*>(red + o);
#pragma unroll
        for (int w = 1; w < 4; ++w) v += *reinterpret_cast<const float4v_t*>(red + w * 4 * 16 * 64 + o);
        return v;
    };
    auto store_quad = [&](int64_t grp, int e, const float4v_t& v) __attribute__((always_inline)) {
        const int64_t br = grp * 4 + (e >> 8);
        const int64_t grow = br * 16 + ((e >> 4) & 15);
        const int64_t col = n0 + 4 * (e & 15);
        if (br >= Mb || grow >= M || col >= N) return;
        const int64_t crow = row_map ? (int64_t)row_map[grow] : grow;
        *reinterpret_cast<float4v_t*>(C + crow * N + col) = v;
    };

    if constexpr (!SPLIT) {
        const uint32_t G = gridDim.x;
        const uint32_t x8 = blockIdx.x & 7u;
        const uint32_t grp = kBandXcd ? x8 * (G >> 3) + min(x8, G & 7u) + (blockIdx.x >> 3) : blockIdx.x;
        group_blocks(grp, 0, 0x7fffffff);
        for (int e = threadIdx.x; e < 4 * 16 * 16; e += 256) store_quad(grp, e, tile_quad(e));
    } else {
        // slot of this workgroup: XCD x holds slots x P / 8 .. (x + 1) P / 8 - 1,
        // a contiguous stretch of groups
        const int32_t P = sp.P;
        const int32_t p = (int32_t)((blockIdx.x & 7u) * (uint32_t)(P >> 3) + (blockIdx.x >> 3));
        const int64_t beg = sp.bnd[p], end = sp.bnd[p + 1];
        // partial tiles of this column chunk, through agent-coherent accesses
        // (the cache policy of relaxed agent-scope atomics: no part writes
        // back or invalidates its XCD's whole L2): bank 1 holds a group's
        // first part (the last group of the slot holding it), bank 0 a later
        // part (the first group of its slot)
        const __amdgpu_buffer_rsrc_t part_rsrc = band_rsrc(
            sp.tiles + (int64_t)blockIdx.y * 2 * P * kBandPart32, (uint32_t)(2 * P * kBandPart32 * 4));
        auto part_at = [&](int32_t q, bool head) __attribute__((always_inline)) -> int {
            return (int)(((head ? P : 0) + q) * (uint32_t)(kBandPart32 * 4));
        };
        for (int64_t grp = sp.first[p]; grp < sp.G; ++grp) {
            const int64_t s0 = sp.S[grp], s1 = sp.S[grp + 1];
            // groups from `end` on are later slots' (the last slot also
            // takes the empty groups at the very end)
            if (s0 >= end && p != P - 1) break;
            group_blocks(grp, (int32_t)(max(beg, s0) - s0), (int32_t)(min(end, s1) - s0));
            const int32_t parts = sp.parts[grp];
            if (parts == 1) {
                for (int e = threadIdx.x; e < 4 * 16 * 16; e += 256) store_quad(grp, e, tile_quad(e));
                continue;
            }
            const int32_t plo = sp.plo[grp];
            const int32_t k = p - plo;
            const int mine = part_at(p, k == 0);
            for (int e = threadIdx.x; e < 4 * 16 * 16; e += 256)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, tile_quad(e)), part_rsrc,
                                                       e * 16, mine, kAgentCoherent);
            // the stores are complete before the part counts itself
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (threadIdx.x == 0)
                s_arrived = __hip_atomic_fetch_add(sp.arrivals + (int64_t)blockIdx.y * P + plo, 1,
                                                   __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __syncthreads();
            if (s_arrived != parts - 1) continue;
            // the last part: the group's tile is part 0 + part 1 + ... in
            // this order
            for (int e = threadIdx.x; e < 4 * 16 * 16; e += 256) {
                float4v_t v = __builtin_bit_cast(
                    float4v_t, __builtin_amdgcn_raw_buffer_load_b128(part_rsrc, e * 16, part_at(plo, true),
                                                                     kAgentCoherent));
                for (int32_t part = 1; part < parts; ++part)
                    v += __builtin_bit_cast(float4v_t,
                                            __builtin_amdgcn_raw_buffer_load_b128(
                                                part_rsrc, e * 16, part_at(plo + part, false), kAgentCoherent));
                store_quad(grp, e, v);
            }
        }
    }
}

// One thread per group of kBandRows block-rows: counts the block-rows that
// are not one contiguous run of block columns, and adds the group's span in
// aligned pairs (the pairs the band kernel walks for it).
template <typename I>
__global__ __launch_bounds__(256) void band_analyse_kernel(const I* __restrict__ brp,
                                                           const I* __restrict__ bci, int64_t Mb,
                                                           unsigned long long* __restrict__ out)
{
    const int64_t grp = (int64_t)blockIdx.x * 256 + threadIdx.x;
    unsigned long long gaps = 0, span = 0;
    if (grp * kBandRows < Mb) {
        int64_t lo = INT64_MAX, hi = -1;
        for (int w = 0; w < kBandRows; ++w) {
            const int64_t br = grp * kBandRows + w;
            if (br >= Mb) break;
            const int64_t rs = (int64_t)brp[br], re = (int64_t)brp[br + 1];
            if (re <= rs) continue;
            const int64_t first = (int64_t)bci[rs], last = (int64_t)bci[re - 1];
            if (last - first + 1 != re - rs) ++gaps;
            lo = min(lo, first);
            hi = max(hi, last);
        }
        if (hi >= 0) span = (unsigned long long)((hi >> 1) - (lo >> 1) + 1);
    }
    // one atomic per wave and counter
    for (int o = 32; o > 0; o >>= 1) {
        gaps += __shfl_down(gaps, o);
        span += __shfl_down(span, o);
    }
    if ((threadIdx.x & 63) == 0) {
        if (gaps) atomicAdd(&out[0], gaps);
        if (span) atomicAdd(&out[1], span);
    }
}

}  // namespace

template <typename I>
bool spmm_band_wanted(const I* brp, const I* bci, int64_t M, int64_t K, int64_t Mb, int64_t Kb,
                      int64_t nnz, int64_t nnzb, int64_t N, int value_bytes, hipStream_t s)
{
    (void)M;
    if (value_bytes != 2 && value_bytes != 4) return false;
    if (Mb < 1 || nnzb < 1 || !spmm_band_f16_covers(K, Kb, Mb, N > 0 ? N : 128)) return false;
    if (value_bytes == 4 && K * (N > 0 ? N : 128) * 4 > (int64_t(1) << 31)) return false;
    // fp32: the band kernel's waves split each group's blocks four ways, which
    // pays from about 16 blocks per block-row (the examples/05 bands from 5 %)
    if (value_bytes == 4 && nnzb < 16 * Mb) return false;
    if (nnzb == Mb * Kb) return false;  // every block present: the GEMM-tiled kernel's grid
    // a kernel forced by the diagnostic switches XSPMM_SPMM_KERNEL (fp16) or
    // XSPMM_F32_KERNEL (fp32) keeps its grids
    if (const char* e = std::getenv(value_bytes == 2 ? "XSPMM_SPMM_KERNEL" : "XSPMM_F32_KERNEL"); e && *e)
        return false;
    Scratch counters(2 * sizeof(unsigned long long), s);
    XSPMM_HIP_CHECK(hipMemsetAsync(counters.get(), 0, 2 * sizeof(unsigned long long), s));
    const int64_t groups = (Mb + kBandRows - 1) / kBandRows;
    hipLaunchKernelGGL((band_analyse_kernel<I>), dim3((unsigned)((groups + 255) / 256)), dim3(256), 0, s,
                       brp, bci, Mb, counters.as<unsigned long long>());
    XSPMM_LAUNCH_CHECK();
    unsigned long long h[2] = {0, 0};
    XSPMM_HIP_CHECK(hipMemcpyAsync(h, counters.get(), sizeof(h), hipMemcpyDeviceToHost, s));
    XSPMM_HIP_CHECK(hipStreamSynchronize(s));
    if (h[0] != 0) return false;  // a block-row with a gap: the kernel needs contiguous rows
    // B rows each kernel gathers per 128 columns: the band kernel 32 per pair
    // of a group's span; the column-batch kernel one per non-zero column of
    // each block (estimated for entries spread evenly over the blocks; all
    // 16 when the entry count is not known)
    const double f = nnz > 0 ? std::min(1.0, (double)nnz / (256.0 * (double)nnzb)) : 1.0;
    const double batch_rows = (double)nnzb * 16.0 * (1.0 - std::pow(1.0 - f, 16.0));
    return 32.0 * (double)h[1] <= batch_rows;
}

template bool spmm_band_wanted<int32_t>(const int32_t*, const int32_t*, int64_t, int64_t, int64_t,
                                        int64_t, int64_t, int64_t, int64_t, int, hipStream_t);
template bool spmm_band_wanted<int64_t>(const int64_t*, const int64_t*, int64_t, int64_t, int64_t,
                                        int64_t, int64_t, int64_t, int64_t, int, hipStream_t);

bool spmm_band_f16_covers(int64_t K, int64_t Kb, int64_t Mb, int64_t N)
{
    return Mb > 0 && N > 0 && N % 8 == 0 && K * N * 2 <= (int64_t(1) << 31) &&
           N < (int64_t(1) << 22) && Kb < (int64_t(1) << 20) && (N + 127) / 128 <= 65535;
}

template <typename I>
bool bcsr_spmm_band_f16(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                        const uint16_t* bvals, const uint16_t* B, float* C, int64_t N,
                        const I* row_map, hipStream_t s)
{
    if (!spmm_band_f16_covers(K, Kb, Mb, N)) return false;
    const dim3 grid((unsigned)((Mb + kBandRows - 1) / kBandRows), (unsigned)((N + 127) / 128));
    hipLaunchKernelGGL((spmm_f16_band_kernel<I, XSPMM_BAND_DEPTH, XSPMM_BAND_WPR>), grid,
                       dim3(64 * kBandRows * XSPMM_BAND_WPR), 0, s, brp, bci, bvals, B, C, M, K, N, Mb,
                       row_map);
    XSPMM_LAUNCH_CHECK();
    return true;
}

bool spmm_band_f32_covers(int64_t K, int64_t Kb, int64_t Mb, int64_t N, const void* B, const void* C)
{
    return Mb > 0 && N > 0 && N % 4 == 0 && K * N * 4 <= (int64_t(1) << 31) && N < (int64_t(1) << 22) &&
           Kb < (int64_t(1) << 20) && (N + 63) / 64 <= 65535 && (reinterpret_cast<uintptr_t>(B) & 15) == 0 &&
           (reinterpret_cast<uintptr_t>(C) & 15) == 0;
}

namespace {

// CUs of the current device, asked once per device
int band_device_cus()
{
    static std::atomic<int> cus[64];
    int dev = 0;
    XSPMM_HIP_CHECK(hipGetDevice(&dev));
    if (dev < 0 || dev >= 64) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n == 0) {
        XSPMM_HIP_CHECK(hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev));
        if (n <= 0) n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// The diagnostic switch XSPMM_BAND_SPLIT: "off" keeps one group per
// workgroup, "force" takes the balanced launch wherever it can run (for
// tests); otherwise the launcher's rule decides.
int band_split_mode()
{
    const char* e = std::getenv("XSPMM_BAND_SPLIT");
    if (e && std::string(e) == "off") return 0;
    if (e && std::string(e) == "force") return 2;
    return 1;
}

}  // namespace

template <typename I>
bool bcsr_spmm_band_f32(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                        const float* bvals, const float* B, float* C, int64_t N, const I* row_map,
                        int64_t nnzb, hipStream_t s)
{
    if (!spmm_band_f32_covers(K, Kb, Mb, N, B, C)) return false;
    const int64_t G = (Mb + 3) / 4;
    const int64_t chunks = (N + 63) / 64;
    const int64_t P = std::min<int64_t>(kPlanSlots, ((int64_t)band_device_cus() + 7) / 8 * 8);
    const size_t tile_bytes = (size_t)chunks * 2 * (size_t)P * kBandPart32 * sizeof(float);
    // The balanced launch (on grids of at most kPlanGroups groups) where the
    // one-group-per-workgroup launch is predicted to take 10 % longer:
    //   balanced:  W + 25 us (plan kernel, schedule loads, hand-off), with
    //              W = nnzb N / (850 per us and CU x CUs), the rate the
    //              balanced launch keeps on the 16384^2 90 % band;
    //   one group: W / (q s), q the share of the grid's workgroup rounds that
    //              its G x chunks workgroups fill (two per CU), s = 1 - f^2 / 2
    //              the average group's share of the widest span on a band of
    //              fill f = nnzb / (Mb Kb) (0.76 at the 90 % band, 0.90 at 50 %).
    // Measured rule: it picks the faster launch on every band of 4096^2 to
    // 16384^2 and N of 64 to 256 timed both ways.
    const int mode = band_split_mode();
    bool pays = false;
    if (mode == 1) {
        const double cus = (double)band_device_cus();
        const double W = (double)nnzb * (double)N / (850.0 * cus);
        const double wgs = (double)G * (double)chunks, cap = 2.0 * cus;
        const double q = wgs / (std::ceil(wgs / cap) * cap);
        const double f = (double)nnzb / ((double)Mb * (double)Kb);
        const double sp_share = 1.0 - f * f / 2.0;
        pays = W / (q * sp_share) > 1.1 * (W + 25.0);
    }
    if (mode > 0 && nnzb > 0 && (mode == 2 || pays) && G <= kPlanGroups && tile_bytes <= (size_t(512) << 20)) {
        Carve cv;
        const size_t o_S = cv.take((size_t)(G + 1) * sizeof(int64_t));
        const size_t o_bnd = cv.take((size_t)(P + 1) * sizeof(int64_t));
        const size_t o_first = cv.take((size_t)P * sizeof(int32_t));
        const size_t o_plo = cv.take((size_t)G * sizeof(int32_t));
        const size_t o_parts = cv.take((size_t)G * sizeof(int32_t));
        const size_t o_arr = cv.take((size_t)(P * chunks) * sizeof(int32_t));
        const size_t o_tiles = cv.take(tile_bytes);
        Scratch mem(cv.end, s);
        char* base = static_cast<char*>(mem.get());
        BandSplit sp;
        sp.S = reinterpret_cast<const int64_t*>(base + o_S);
        sp.bnd = reinterpret_cast<const int64_t*>(base + o_bnd);
        sp.first = reinterpret_cast<const int32_t*>(base + o_first);
        sp.plo = reinterpret_cast<const int32_t*>(base + o_plo);
        sp.parts = reinterpret_cast<const int32_t*>(base + o_parts);
        sp.arrivals = reinterpret_cast<int32_t*>(base + o_arr);
        sp.tiles = reinterpret_cast<float*>(base + o_tiles);
        sp.G = G;
        sp.P = (int32_t)P;
        hipLaunchKernelGGL((band_plan_kernel<I>), dim3(1), dim3(1024), 0, s, brp, bci, Mb, nnzb, sp,
                           (int32_t)chunks);
        XSPMM_LAUNCH_CHECK();
        hipLaunchKernelGGL((spmm_f32_band_kernel<I, XSPMM_BAND_F32_DEPTH, true>), dim3((unsigned)P, (unsigned)chunks),
                           dim3(256), 0, s, brp, bci, bvals, B, C, M, K, N, Mb, row_map, sp);
        XSPMM_LAUNCH_CHECK();
        return true;
    }
    const dim3 grid((unsigned)G, (unsigned)chunks);
    hipLaunchKernelGGL((spmm_f32_band_kernel<I, XSPMM_BAND_F32_DEPTH, false>), grid, dim3(256), 0, s, brp, bci,
                       bvals, B, C, M, K, N, Mb, row_map, BandSplit{});
    XSPMM_LAUNCH_CHECK();
    return true;
}
template bool bcsr_spmm_band_f32<int32_t>(int64_t, int64_t, int64_t, int64_t, const int32_t*,
                                          const int32_t*, const float*, const float*, float*, int64_t,
                                          const int32_t*, int64_t, hipStream_t);
template bool bcsr_spmm_band_f32<int64_t>(int64_t, int64_t, int64_t, int64_t, const int64_t*,
                                          const int64_t*, const float*, const float*, float*, int64_t,
                                          const int64_t*, int64_t, hipStream_t);

template bool bcsr_spmm_band_f16<int32_t>(int64_t, int64_t, int64_t, int64_t, const int32_t*,
                                          const int32_t*, const uint16_t*, const uint16_t*, float*,
                                          int64_t, const int32_t*, hipStream_t);
template bool bcsr_spmm_band_f16<int64_t>(int64_t, int64_t, int64_t, int64_t, const int64_t*,
                                          const int64_t*, const uint16_t*, const uint16_t*, float*,
                                          int64_t, const int64_t*, hipStream_t);

}  // namespace detail
}  // namespace xspmm
