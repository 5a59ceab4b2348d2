// spmm_f32.hip -- fp32 Tier-1 BCSR SpMM: column batches on v_mfma_f32_16x16x4f32.
//
// Semantics follow the reference tile kernel (src/common/spmm_math.hpp:20-146)
// as instantiated for float (src/xspmm.cpp:102-114, unstructured_mtx_mul.hip:
// 105-106): C[16 br : +16, :] = sum over the block-row's blocks of
// A_blk * B[16 col : +16, :], fp32 accumulation, C overwritten, block-rows
// without blocks give zeros.  Rows >= M are not stored; B rows >= K and
// columns >= N contribute nothing.
//
// A 16x16 block of a sparse matrix usually holds a few non-zero columns (1.7
// of 16 at the headline pattern), and only the B rows of those columns can
// change C.  The fp32 matrix-core step v_mfma_f32_16x16x4f32 takes one K
// index per 16-lane group (lane (i, k) holds A[i][k] and B[k][i]), so its four
// K slots can be filled with any four non-zero block columns of the
// block-row, from any blocks: all blocks of a block-row add into the same 16
// rows of C.  Each wave of a workgroup takes every W-th block of its
// block-row, D blocks per ring pass, and
//   1. streams the blocks (16 bytes per lane: lane (r, g) holds row r,
//      columns 4g .. 4g+3; each block's load issued one pass ahead) and, one
//      vector load per ring pass, their block columns;
//   2. forms the block's column mask from four ballots (one per column of a
//      lane's quad; a column counts when any of its 16 entries is not +-0,
//      so NaN and Inf count) and a few scalar operations;
//   3. queues the set columns in its LDS column queue: lane (r, g) writes
//      row r of each of its set columns to the column's slot (64 bytes of A'
//      per column, columns in block and column order), and lane (0, g) the
//      byte offset of the column's B row;
//   4. at the end of the pass, multiplies the batches taken at the previous
//      pass's end and takes up to F batches of four queued columns: lane
//      (r, k) reads A'[r][slot k] from the queue, and lane (n, k) loads
//      B[row(k)][n0 + 64 q + 4 n .. +3] as one 16-byte load per 64 columns,
//      straight into MFMA B operands.  So a pass's rows arrive while the next
//      pass streams its blocks.  The multiply issues one MFMA per float4
//      component j: component j of quad q covers C columns n0 + 64 q + 4 n + j.
// Every pass issues the same loads in the same order (window, D blocks,
// F * NQ B loads, unused ones at distinct offsets past B that read nothing),
// so the compiler's waits count exactly the loads they must: a block's wait
// never drains the blocks behind it or a batch's rows.
// A block whose 16 columns are all set is multiplied where it is met, after
// the batches in flight: four batches as it stands (batch s holding columns
// 4k + s, which lane (r, k) already holds) with their 4 x 16 B rows.
// The waves' partial tiles are summed through LDS in wave order and stored as
// 16-byte rows.  Skipped columns would add exact zeros (products of +-0 and
// finite B entries), so C equals the full product for finite B; a non-finite
// B entry meets only columns that hold a non-zero A entry (0 * Inf is not
// formed), as in the fp16 column-batch kernel.
// grid = (block-rows, ceil(N / (64 NQ))); N % 4 == 0, B 16-byte aligned,
// K * N * 4 <= 2^31, Kb < 2^21 (32-bit offsets within a row and into B).
//
// spmm_f32_packed_kernel (below) multiplies the same kind of batches stored
// once, from the Tier-2 pipeline's CSR conversion, instead of forming them
// from the blocks.
#include <cstdlib>
#include <string>

#include "internal.hpp"

namespace xspmm {
namespace detail {

namespace {

typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;
// Buffer resource word 3 for raw (untyped, unswizzled) dword access on gfx9.
constexpr int kRawBufferWord3 = 0x00020000;
// Cache-policy operand of the buffer-load builtins: non-temporal (nt).
constexpr int kNonTemporal = 2;
// Columns of the per-wave LDS column queue (a power of two): 64 bytes of A'
// and 4 bytes of B row offset each.  A pass queues at most 15 columns per
// block (a block with all 16 set is multiplied directly), and the pass end
// leaves at most kQueueCols - 15 D queued, so no unread slot is overwritten;
// LDS operations of one wave complete in order.
constexpr int kQueueCols = 128;
constexpr int kQueueBytes = kQueueCols * 68;
// column mask of a block whose 16 columns all hold a non-zero entry
constexpr uint64_t kAllColumns = 0x000f000f000f000full;

#ifndef XSPMM_F32_PRIO
#define XSPMM_F32_PRIO 1
#endif

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kRawBufferWord3);
}

__device__ __forceinline__ void set_prio(int level)
{
    switch (level) {
    case 3: __builtin_amdgcn_s_setprio(3); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    default: __builtin_amdgcn_s_setprio(0); break;
    }
}

// Column mask of a block from the ballots of "entry != 0" of the four
// columns 4g + s (s = 0 .. 3) each lane group g holds: bit 16 g + s is set
// when column 4g + s has a non-zero entry in any of its 16 rows.  Bit 15 of
// each 16-bit group of ((b & 0x7fff...) + 0x7fff...) | b is the OR of the
// group's bits (the low 15 bits cannot carry past bit 15).
__device__ __forceinline__ uint64_t column_mask(uint64_t b0, uint64_t b1, uint64_t b2, uint64_t b3)
{
    constexpr uint64_t kLow = 0x7fff7fff7fff7fffull;
    constexpr uint64_t kTop = 0x8000800080008000ull;
    auto any = [](uint64_t b) { return (((b & kLow) + kLow) | b) & kTop; };
    return (any(b0) >> 15) | (any(b1) >> 14) | (any(b2) >> 13) | (any(b3) >> 12);
}

// Mask bits of the block columns c < lim (lim in 0 .. 16), in the layout of
// column_mask.
__device__ __forceinline__ uint64_t columns_below(uint32_t lim)
{
    uint64_t m = 0;
    for (uint32_t g = 0; g < 4; ++g) {
        const uint32_t c0 = 4 * g;
        const uint32_t n = lim > c0 ? (lim - c0 < 4 ? lim - c0 : 4) : 0;
        m |= (uint64_t)((1u << n) - 1u) << (16 * g);
    }
    return m;
}

// NQ: 64-column quads per workgroup (one 16-byte B load per quad and batch
// slot); W: waves per workgroup; D: blocks per ring pass (in flight per
// wave); F: batches taken from the column queue per pass.
template <typename I, int NQ, int W, int D, int F>
__global__ __launch_bounds__(64 * W, (W <= 4 ? 16 / W : 1)) void spmm_f32_batch_kernel(
    const I* __restrict__ brp, const I* __restrict__ bci, const float* __restrict__ vals,
    const float* __restrict__ B, float* __restrict__ C, int64_t M, int64_t K, int64_t N,
    int64_t Kb, const int32_t* __restrict__ order, const I* __restrict__ row_map)
{
    static_assert(NQ == 1 || NQ == 2, "64 or 128 columns per workgroup");
    static_assert(D >= 2 && D <= 8, "2 .. 8 blocks per ring pass");
    // the block stream of a long grid is read once per call and bypasses the
    // caches' reuse (non-temporal); a short grid's blocks (the 16-wave
    // variant) stay cached for the next call
    constexpr int kAPolicy = W <= 4 ? kNonTemporal : 0;
    static_assert(F >= 4 && F <= 8, "4 .. 8 batches per pass");
    // a pass adds at most 15 D columns to a queue the previous pass end left
    // at most kQueueCols - 15 D long; that bound is at least 4, so a queue
    // above it always holds a full batch to take
    static_assert(15 * D + 4 <= kQueueCols, "a pass's sparse columns fit the queue");
    static_assert(D * (int)sizeof(I) <= 256, "a pass's block columns fit one index window");
    constexpr int kRedBytes = 16 * 64 * NQ * 4;  // one wave's partial tile
    constexpr int kLdsBytes = W * (kQueueBytes > kRedBytes ? kQueueBytes : kRedBytes);
    __shared__ __align__(16) unsigned char smem[kLdsBytes];

    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int li = lane & 15;
    const int g = lane >> 4;

    const int64_t br = order ? (int64_t)order[blockIdx.x] : (int64_t)blockIdx.x;
    // a caller-supplied order holds a permutation of the block-rows; an id
    // outside the grid is skipped rather than read past row_ptr
    if ((uint64_t)br >= (uint64_t)gridDim.x) return;
    const int64_t n0 = (int64_t)blockIdx.y * 64 * NQ;
    const int64_t rs = brp[br];
    const int64_t re = brp[br + 1];
    const uint32_t nblk = (uint32_t)(re - rs);
    // this wave's blocks: wave, wave + W, ... (wave-block q is row block wave + W q)
    const uint32_t mine = nblk > (uint32_t)wave ? (nblk - (uint32_t)wave + W - 1) / W : 0u;

    // reads past the row's blocks return zeros (an all-zero block is skipped)
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(vals + rs * 256, nblk * 1024u);
    const __amdgpu_buffer_rsrc_t c_rsrc = make_rsrc(bci + rs, nblk * (uint32_t)sizeof(I));
    const uint32_t b_bytes = (uint32_t)(K * N * 4);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(B, b_bytes);
    const uint32_t rowbytes = (uint32_t)(4 * N);
    const uint32_t kb32 = (uint32_t)Kb;
    constexpr uint32_t kNone = 0xffffffffu;  // a slot (or quad) that loads nothing

    // this wave's column queue: A' columns [kQueueCols][16] fp32 and the byte
    // offsets of their B rows [kQueueCols]; slot s at index s mod kQueueCols
    float* const qa = reinterpret_cast<float*>(smem + wave * kQueueBytes);
    uint32_t* const qr = reinterpret_cast<uint32_t*>(smem + wave * kQueueBytes + kQueueCols * 64);
    uint32_t head = 0;  // next slot to take (wave-uniform)
    uint32_t tail = 0;  // next slot to fill (wave-uniform)

    // lane (li, g) reads row li, columns 4g .. 4g+3 of a block
    const uint32_t a_voff = (uint32_t)(li * 64 + g * 16) + (uint32_t)wave * 1024u;
    // B loads: lane (li, g) covers columns n0 + 64 q + 4 li .. +3 of its slot's
    // row; quads past N read nothing
    uint32_t b_lane[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int64_t col = n0 + 64 * q + 4 * li;
        b_lane[q] = col < N ? (uint32_t)(4 * col) : kNone;
    }
    // index window of a ring pass: lane l holds dword l of the block columns
    // of wave-blocks p .. p + 63 (int64: two dwords per block)
    constexpr uint32_t kIdxDw = sizeof(I) / 4;
    const uint32_t cw_off = (uint32_t)wave * (uint32_t)sizeof(I) +
                            (uint32_t)(lane / kIdxDw) * (uint32_t)(W * sizeof(I)) +
                            4u * (uint32_t)(lane % kIdxDw);

    float4_t acc[NQ][4];
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[q][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    // the batches in flight: A' entry (lane (r, k): A'[r][slot k]) and B
    // operands (lane (n, k): row of slot k, columns n0 + 64 q + 4 n .. +3)
    float ap[F];
    float4_t bq[F][NQ];
#pragma unroll
    for (int f = 0; f < F; ++f) {
        ap[f] = 0.f;
#pragma unroll
        for (int q = 0; q < NQ; ++q) bq[f][q] = float4_t{0.f, 0.f, 0.f, 0.f};
    }
    uint32_t inflight = 0;  // batches held in ap / bq (wave-uniform)

    auto multiply = [&](const float a, const float4_t (&b)[NQ]) __attribute__((always_inline)) {
#pragma unroll
        for (int q = 0; q < NQ; ++q)
#pragma unroll
            for (int j = 0; j < 4; ++j)
                acc[q][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b[q][j], acc[q][j], 0, 0, 0);
    };
    // multiply the batches in flight (waits for their B rows)
    auto multiply_inflight = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int f = 0; f < F; ++f)
            if ((uint32_t)f < inflight) multiply(ap[f], bq[f]);
        inflight = 0;
    };
    // B operands of the rows at byte offsets off[f] (zeros, with no memory
    // access, for kNone and quads past N): always F * NQ loads, the ones that
    // read nothing at distinct offsets past B, so that none is merged away
    auto load_rows = [&](const uint32_t (&off)[F]) __attribute__((always_inline)) {
#pragma unroll
        for (int f = 0; f < F; ++f)
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                uint32_t o = (off[f] != kNone && b_lane[q] != kNone)
                                 ? off[f] + b_lane[q]
                                 : b_bytes + 16u * (uint32_t)(f * NQ + q);
                // an opaque offset: one load on every path (the compiler would
                // otherwise split the select into branches, each with a load)
                asm volatile("" : "+v"(o));
                bq[f][q] = __builtin_bit_cast(
                    float4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)o, 0, 0));
            }
    };
    // take up to F batches of four queued columns (the last one partial when
    // the queue holds fewer) and issue their B loads; the batches in flight
    // must have been multiplied
    auto take = [&](uint32_t nbat) __attribute__((always_inline)) {
        uint32_t off[F];
#pragma unroll
        for (int f = 0; f < F; ++f) {
            const uint32_t slot = head + 4u * (uint32_t)f + (uint32_t)g;
            const bool used = (uint32_t)f < nbat && slot < tail;
            const uint32_t at = slot & (kQueueCols - 1u);
            const float x = qa[at * 16u + (uint32_t)li];
            const uint32_t r = qr[at];
            ap[f] = used ? x : 0.f;
            off[f] = used ? r : kNone;
        }
        load_rows(off);
        head = head + 4u * nbat < tail ? head + 4u * nbat : tail;
        inflight = nbat;
    };

    auto stage_a = [&](uint32_t q, float4_t& P) __attribute__((always_inline)) {
        P = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                             a_rsrc, (int)(a_voff + q * (uint32_t)(W * 1024)), 0,
                                             kAPolicy));
    };
    auto load_cols = [&](uint32_t q) __attribute__((always_inline)) -> uint32_t {
        return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
            c_rsrc, (int)(cw_off + q * (uint32_t)(W * sizeof(I))), 0, 0);
    };

    // block j of the ring pass whose index window is `win`
    auto process = [&](const float4_t& P, uint32_t win, int j) __attribute__((always_inline)) {
        uint32_t cb;
        if constexpr (sizeof(I) == 4) {
            cb = (uint32_t)__builtin_amdgcn_readlane((int)win, j);
        } else {
            const uint32_t lo = (uint32_t)__builtin_amdgcn_readlane((int)win, 2 * j);
            const uint32_t hi = (uint32_t)__builtin_amdgcn_readlane((int)win, 2 * j + 1);
            cb = hi == 0u ? lo : kNone;
        }
        uint64_t m = column_mask(__builtin_amdgcn_ballot_w64(P[0] != 0.f),
                                 __builtin_amdgcn_ballot_w64(P[1] != 0.f),
                                 __builtin_amdgcn_ballot_w64(P[2] != 0.f),
                                 __builtin_amdgcn_ballot_w64(P[3] != 0.f));
        // a block column outside the grid (malformed input) contributes
        // nothing; so do the B rows >= K of a ragged last block column
        if (cb >= kb32) m = 0;
        if (m != 0 && (int64_t)cb * 16 + 16 > K) m &= columns_below((uint32_t)(K - (int64_t)cb * 16));
        if (m == 0) return;
        const uint32_t row0 = cb * 16u;
        if (m == kAllColumns) {
            // every column set: the block is four batches as it stands, batch
            // s holding columns 4k + s -- lane (r, k)'s own register s -- and
            // is multiplied here, after the batches in flight
            multiply_inflight();
            uint32_t off[F];
            const uint32_t rb = (row0 + 4u * (uint32_t)g) * rowbytes;
#pragma unroll
            for (int f = 0; f < F; ++f) {
                ap[f] = f < 4 ? P[f & 3] : 0.f;
                off[f] = f < 4 ? rb + (uint32_t)f * rowbytes : kNone;
            }
            load_rows(off);
            inflight = 4;
            multiply_inflight();
            return;
        }
        // queue the set columns: lane (r, g) writes row r of each of its set
        // columns 4g + s to the column's slot (columns keep their order)
        const uint32_t nib = (uint32_t)(m >> (16 * g)) & 0xfu;
        const uint32_t before = tail + (uint32_t)__builtin_popcountll(m & ((1ull << (16 * g)) - 1ull));
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            if ((nib >> s) & 1u) {
                const uint32_t at = (before + (uint32_t)__builtin_popcount(nib & ((1u << s) - 1u))) &
                                    (kQueueCols - 1u);
                qa[at * 16u + (uint32_t)li] = P[s];
                if (li == 0) qr[at] = (row0 + 4u * (uint32_t)g + (uint32_t)s) * rowbytes;
            }
        }
        tail += (uint32_t)__builtin_popcountll(m);
    };

    // One shape per ring pass: one index-window load, D block loads (each
    // right after its block is processed, for the next pass) and, at the
    // pass's end, F * NQ B loads (the batches taken from the queue, padded
    // with loads that read nothing), so every wait counts exactly the loads
    // it must.  A pass's B rows arrive while the next pass streams its
    // blocks, and are multiplied at that pass's end.  Only full blocks, and a
    // pass that leaves too long a queue for the next one, multiply on the
    // spot.
    if (mine > 0 && mine <= (uint32_t)D) {
        // A single pass (short rows): the blocks it has, then the B rows of
        // all its batches; no later loads, so no padding is needed.
        float4_t P0, P1, P2, P3, P4, P5, P6, P7;
        const uint32_t win = load_cols(0);
        stage_a(0, P0);
        if (mine > 1) stage_a(1, P1);
        if constexpr (D > 2) if (mine > 2) stage_a(2, P2);
        if constexpr (D > 3) if (mine > 3) stage_a(3, P3);
        if constexpr (D > 4) if (mine > 4) stage_a(4, P4);
        if constexpr (D > 5) if (mine > 5) stage_a(5, P5);
        if constexpr (D > 6) if (mine > 6) stage_a(6, P6);
        if constexpr (D > 7) if (mine > 7) stage_a(7, P7);
        process(P0, win, 0);
        if (mine > 1) process(P1, win, 1);
        if constexpr (D > 2) if (mine > 2) process(P2, win, 2);
        if constexpr (D > 3) if (mine > 3) process(P3, win, 3);
        if constexpr (D > 4) if (mine > 4) process(P4, win, 4);
        if constexpr (D > 5) if (mine > 5) process(P5, win, 5);
        if constexpr (D > 6) if (mine > 6) process(P6, win, 6);
        if constexpr (D > 7) if (mine > 7) process(P7, win, 7);
        multiply_inflight();
        while (tail != head) {
            const uint32_t rest = (tail - head + 3u) >> 2;
            take(rest < (uint32_t)F ? rest : (uint32_t)F);
            multiply_inflight();
        }
    } else if (mine > 0) {
        // the first pass's loads in the order a pass leaves them: window,
        // blocks 0 .. D-1, then F * NQ B loads that read nothing (the
        // scheduling barriers keep the blocks in order), so that the waits
        // of the first pass and of later ones agree
        float4_t P0, P1, P2, P3, P4, P5, P6, P7;
        uint32_t win = load_cols(0);
        __builtin_amdgcn_sched_barrier(0);
        stage_a(0, P0);
        __builtin_amdgcn_sched_barrier(0);
        stage_a(1, P1);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (D > 2) stage_a(2, P2);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (D > 3) stage_a(3, P3);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (D > 4) stage_a(4, P4);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (D > 5) stage_a(5, P5);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (D > 6) stage_a(6, P6);
        __builtin_amdgcn_sched_barrier(0);
        if constexpr (D > 7) stage_a(7, P7);
        __builtin_amdgcn_sched_barrier(0);
        {
            uint32_t none[F];
#pragma unroll
            for (int f = 0; f < F; ++f) none[f] = kNone;
            load_rows(none);
        }
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t passes = (mine + D - 1) / D;
        int level = -1;
        for (uint32_t pass = 0; pass < passes; ++pass) {
            const uint32_t q = pass * D;
            if constexpr (XSPMM_F32_PRIO != 0) {
                // waves furthest from done issue first, so the workgroups
                // sharing a CU end together
                const uint32_t rem = passes - pass;
                const int lv = rem > 16u ? 3 : rem > 8u ? 2 : rem > 2u ? 1 : 0;
                if (lv != level) {
                    level = lv;
                    set_prio(lv);
                }
            }
            const uint32_t nwin = load_cols(q + D);
            process(P0, win, 0);
            stage_a(q + D, P0);
            process(P1, win, 1);
            stage_a(q + D + 1, P1);
            if constexpr (D > 2) {
                process(P2, win, 2);
                stage_a(q + D + 2, P2);
            }
            if constexpr (D > 3) {
                process(P3, win, 3);
                stage_a(q + D + 3, P3);
            }
            if constexpr (D > 4) {
                process(P4, win, 4);
                stage_a(q + D + 4, P4);
            }
            if constexpr (D > 5) {
                process(P5, win, 5);
                stage_a(q + D + 5, P5);
            }
            if constexpr (D > 6) {
                process(P6, win, 6);
                stage_a(q + D + 6, P6);
            }
            if constexpr (D > 7) {
                process(P7, win, 7);
                stage_a(q + D + 7, P7);
            }
            // pass end: multiply the previous pass's batches, take this
            // pass's full batches (after the last pass, the partial one too)
            multiply_inflight();
            const uint32_t full = (tail - head + (pass + 1 == passes ? 3u : 0u)) >> 2;
            take(full < (uint32_t)F ? full : (uint32_t)F);
            // leave room for the next pass's columns
            while (tail - head > (uint32_t)(kQueueCols - 15 * D)) {
                multiply_inflight();
                const uint32_t more = (tail - head) >> 2;
                take(more < (uint32_t)F ? more : (uint32_t)F);
            }
            win = nwin;
        }
        multiply_inflight();
        while (tail != head) {
            const uint32_t rest = (tail - head + 3u) >> 2;
            take(rest < (uint32_t)F ? rest : (uint32_t)F);
            multiply_inflight();
        }
    }

    // sum the waves' partial tiles in wave order and store C
    __syncthreads();
    float* const red = reinterpret_cast<float*>(smem);  // W x [16][64 NQ]
    constexpr int kCols = 64 * NQ;
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<float4_t*>(red + wave * 16 * kCols + (4 * g + i) * kCols + 64 * q + 4 * li) =
                float4_t{acc[q][0][i], acc[q][1][i], acc[q][2][i], acc[q][3][i]};
    __syncthreads();
    for (int t = threadIdx.x; t < 16 * kCols / 4; t += 64 * W) {
        const int row = t / (kCols / 4);
        const int c4 = 4 * (t % (kCols / 4));
        const int64_t grow = br * 16 + row;
        const int64_t col = n0 + c4;
        if (grow >= M || col >= N) continue;
        float4_t v = *reinterpret_cast<const float4_t*>(red + row * kCols + c4);
#pragma unroll
        for (int w = 1; w < W; ++w) v += *reinterpret_cast<const float4_t*>(red + w * 16 * kCols + row * kCols + c4);
        const int64_t crow = row_map ? (int64_t)row_map[grow] : grow;
        *reinterpret_cast<float4_t*>(C + crow * N + col) = v;
    }
}

// Four waves per workgroup (four workgroups per CU, 128 VGPRs per wave):
// 8 blocks per pass, and 4 batches at 128 columns, 6 at 64 (at 128 columns,
// templates in fp32: 6 blocks per pass 177.7-178.6 us, 8 173.3-174.0 us, 4
// 183.2-184.2 us).
// Grids of fewer than 512 workgroups: 16 waves per workgroup (one per CU),
// 4 blocks per pass, so that short grids still spread each block-row's
// blocks over many waves.
template <typename I, int NQ>
void launch_batch(dim3 grid, hipStream_t s, const I* brp, const I* bci, const float* v, const float* b,
                  float* C, int64_t M, int64_t K, int64_t N, int64_t Kb, const int32_t* order,
                  const I* row_map)
{
    const bool short_grid = (int64_t)grid.x * grid.y < 512;
    if (short_grid)
        hipLaunchKernelGGL((spmm_f32_batch_kernel<I, NQ, 16, 4, 4>), grid, dim3(64 * 16), 0, s, brp,
                           bci, v, b, C, M, K, N, Kb, order, row_map);
    else if constexpr (NQ == 2)
        hipLaunchKernelGGL((spmm_f32_batch_kernel<I, 2, 4, 8, 4>), grid, dim3(64 * 4), 0, s, brp, bci,
                           v, b, C, M, K, N, Kb, order, row_map);
    else
        hipLaunchKernelGGL((spmm_f32_batch_kernel<I, 1, 4, 8, 6>), grid, dim3(64 * 4), 0, s, brp, bci,
                           v, b, C, M, K, N, Kb, order, row_map);
}

// ---------------------------------------------------------------------------
// Packed fp32 column batches (the Tier-2 pipeline's fp32 form, written by
// csr_pack_emit in convert.hip): strip br's batches [offsets[br],
// offsets[br + 1]) hold its set columns four at a time (batch t: slots
// 4t .. 4t+3, one per MFMA K position), in groups of four batches.  Group G
// is one 16-byte load per lane of A' (lane (i, k): A'[i][k] of batches 4G ..
// 4G+3) and one of row indices (lane (n, k): B row of slot k of the four
// batches).  Wave w of the workgroup of block-row br multiplies the strip's
// groups w, w + 4, ... in order: per batch and 64-column quad, the B rows of
// its four slots as one 16-byte load per lane, straight into MFMA B operands
// (as spmm_f32_batch_kernel does), then one v_mfma_f32_16x16x4f32 per float4
// component.  Row indices arrive two groups ahead and B rows and A' one group
// ahead; every iteration issues the same loads (the ones past the wave's
// groups read nothing or are not multiplied), so each wait counts exactly
// the loads it must.  The waves' partial tiles are summed through LDS in wave
// order; product row r goes to C row row_map[r] when row_map is given.
// grid = (block-rows, ceil(N / (64 NQ))); N % 4 == 0, B and C 16-byte
// aligned, K * N * 4 <= 2^31.
template <typename I, int NQ>
__global__ __launch_bounds__(256, 4) void spmm_f32_packed_kernel(
    const int64_t* __restrict__ offsets, const float* __restrict__ pa, const uint32_t* __restrict__ prow,
    const float* __restrict__ B, float* __restrict__ C, int64_t M, int64_t K, int64_t N,
    const int32_t* __restrict__ order, const I* __restrict__ row_map)
{
    static_assert(NQ == 1 || NQ == 2, "64 or 128 columns per workgroup");
    constexpr int W = 4;
    constexpr int kCols = 64 * NQ;
    __shared__ __align__(16) float red[W * 16 * kCols];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    const int li = lane & 15;
    const int g = lane >> 4;

    const int64_t br = order ? (int64_t)order[blockIdx.x] : (int64_t)blockIdx.x;
    // a caller-supplied order holds a permutation of the block-rows; an id
    // outside the grid is skipped rather than read past the offsets
    if ((uint64_t)br >= (uint64_t)gridDim.x) return;
    const int64_t n0 = (int64_t)blockIdx.y * kCols;
    const int64_t G0 = offsets[br] >> 2;
    const int64_t ng = (offsets[br + 1] >> 2) - G0;
    // this wave's groups: G0 + wave + W i, i < n
    const int64_t n = ng > wave ? (ng - wave + W - 1) / W : 0;

    // reads past the strip's groups return zeros
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(pa + G0 * 256, (uint32_t)(ng * 1024));
    const __amdgpu_buffer_rsrc_t r_rsrc = make_rsrc(prow + G0 * 16, (uint32_t)(ng * 64));
    const uint32_t b_bytes = (uint32_t)(K * N * 4);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(B, b_bytes);
    const uint32_t rowbytes = (uint32_t)(4 * N);
    const uint32_t k32 = (uint32_t)K;
    constexpr uint32_t kNone = 0xffffffffu;
    uint32_t b_lane[NQ];
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
        const int64_t col = n0 + 64 * q + 4 * li;
        b_lane[q] = col < N ? (uint32_t)(4 * col) : kNone;
    }
    // byte offsets of group i of this wave in the strip's A' and index arrays
    const uint32_t a_off0 = (uint32_t)wave * 1024u + 16u * (uint32_t)lane;
    const uint32_t r_off0 = (uint32_t)wave * 64u + 16u * (uint32_t)g;

    float4_t acc[NQ][4];
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[q][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    auto load_rows = [&](int64_t i) __attribute__((always_inline)) -> u32x4_t {
        return __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                               r_rsrc, (int)(r_off0 + (uint32_t)i * (64u * W)), 0, 0));
    };
    // group i's A' and B rows (rows r: slot k of its four batches)
    auto load_group = [&](int64_t i, const u32x4_t& r, float4_t& a, float4_t (&bq)[4][NQ])
        __attribute__((always_inline)) {
        a = __builtin_bit_cast(float4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                             a_rsrc, (int)(a_off0 + (uint32_t)i * (1024u * W)), 0,
                                             kNonTemporal));
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int q = 0; q < NQ; ++q) {
                const uint32_t row = r[c];
                const uint32_t off =
                    (row < k32 && b_lane[q] != kNone) ? __umul24(row, rowbytes) + b_lane[q] : b_bytes;
                bq[c][q] = __builtin_bit_cast(float4_t,
                                              __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)off, 0, 0));
            }
    };
    auto multiply = [&](const float4_t& a, const float4_t (&bq)[4][NQ]) __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < 4; ++c)
#pragma unroll
            for (int q = 0; q < NQ; ++q)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[q][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c], bq[c][q][j], acc[q][j], 0, 0, 0);
    };

    if (n > 0) {
        float4_t a0, a1;
        float4_t b0[4][NQ], b1[4][NQ];
        u32x4_t r0 = load_rows(0);
        u32x4_t r1 = load_rows(1);
        load_group(0, r0, a0, b0);
        for (int64_t i = 0; i < n; i += 2) {
            // group i in a0 / b0, rows of group i + 1 in r1
            r0 = load_rows(i + 2);
            load_group(i + 1, r1, a1, b1);
            multiply(a0, b0);
            // group i + 1 in a1 / b1, rows of group i + 2 in r0
            r1 = load_rows(i + 3);
            load_group(i + 2, r0, a0, b0);
            if (i + 1 < n) multiply(a1, b1);
        }
    }

    // sum the waves' partial tiles in wave order and store C
#pragma unroll
    for (int q = 0; q < NQ; ++q)
#pragma unroll
        for (int i = 0; i < 4; ++i)
            *reinterpret_cast<float4_t*>(red + wave * 16 * kCols + (4 * g + i) * kCols + 64 * q + 4 * li) =
                float4_t{acc[q][0][i], acc[q][1][i], acc[q][2][i], acc[q][3][i]};
    __syncthreads();
    for (int t = threadIdx.x; t < 16 * kCols / 4; t += 64 * W) {
        const int row = t / (kCols / 4);
        const int c4 = 4 * (t % (kCols / 4));
        const int64_t grow = br * 16 + row;
        const int64_t col = n0 + c4;
        if (grow >= M || col >= N) continue;
        float4_t v = *reinterpret_cast<const float4_t*>(red + row * kCols + c4);
#pragma unroll
        for (int w = 1; w < W; ++w) v += *reinterpret_cast<const float4_t*>(red + w * 16 * kCols + row * kCols + c4);
        const int64_t crow = row_map ? (int64_t)row_map[grow] : grow;
        *reinterpret_cast<float4_t*>(C + crow * N + col) = v;
    }
}

}  // namespace

bool spmm_f32_batch_covers(int64_t K, int64_t Kb, int64_t N, const void* B, const void* C)
{
    const char* e = std::getenv("XSPMM_F32_KERNEL");
    if (e && std::string(e) == "tile") return false;
    return N % 4 == 0 && N > 0 && K * N * 4 <= (int64_t(1) << 31) && Kb < (int64_t(1) << 21) &&
           (reinterpret_cast<uintptr_t>(B) & 15) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0 &&
           (N + 127) / 128 <= 65535;
}

template <typename I>
void bcsr_spmm_f32_batch(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                         const float* bvals, const float* B, float* C, int64_t N,
                         const int32_t* order, const I* row_map, hipStream_t s)
{
    if (N <= 64)
        launch_batch<I, 1>(dim3((unsigned)Mb, 1), s, brp, bci, bvals, B, C, M, K, N, Kb, order,
                           row_map);
    else
        launch_batch<I, 2>(dim3((unsigned)Mb, (unsigned)((N + 127) / 128)), s, brp, bci, bvals, B, C,
                           M, K, N, Kb, order, row_map);
    XSPMM_LAUNCH_CHECK();
}

template void bcsr_spmm_f32_batch<int32_t>(int64_t, int64_t, int64_t, int64_t, const int32_t*,
                                           const int32_t*, const float*, const float*, float*,
                                           int64_t, const int32_t*, const int32_t*, hipStream_t);
template void bcsr_spmm_f32_batch<int64_t>(int64_t, int64_t, int64_t, int64_t, const int64_t*,
                                           const int64_t*, const float*, const float*, float*,
                                           int64_t, const int32_t*, const int64_t*, hipStream_t);

template <typename I>
bool spmm_f32_packed(int64_t M, int64_t K, int64_t Mb, const int64_t* offsets, const void* a,
                     const uint32_t* rows, const float* B, float* C, int64_t N, const int32_t* order,
                     const I* row_map, hipStream_t s)
{
    if (M == 0 || N == 0 || Mb == 0) return true;
    if (N % 4 != 0 || K * N * 4 > (int64_t(1) << 31) || (reinterpret_cast<uintptr_t>(B) & 15) != 0 ||
        (reinterpret_cast<uintptr_t>(C) & 15) != 0 || (reinterpret_cast<uintptr_t>(a) & 15) != 0 ||
        (N + 127) / 128 > 65535 || Mb > 0x7fffffffLL)
        return false;
    const float* pa = static_cast<const float*>(a);
    if (N <= 64)
        hipLaunchKernelGGL((spmm_f32_packed_kernel<I, 1>), dim3((unsigned)Mb, 1), dim3(256), 0, s, offsets, pa,
                           rows, B, C, M, K, N, order, row_map);
    else
        hipLaunchKernelGGL((spmm_f32_packed_kernel<I, 2>), dim3((unsigned)Mb, (unsigned)((N + 127) / 128)),
                           dim3(256), 0, s, offsets, pa, rows, B, C, M, K, N, order, row_map);
    XSPMM_LAUNCH_CHECK();
    return true;
}

template bool spmm_f32_packed<int32_t>(int64_t, int64_t, int64_t, const int64_t*, const void*,
                                       const uint32_t*, const float*, float*, int64_t, const int32_t*,
                                       const int32_t*, hipStream_t);
template bool spmm_f32_packed<int64_t>(int64_t, int64_t, int64_t, const int64_t*, const void*,
                                       const uint32_t*, const float*, float*, int64_t, const int32_t*,
                                       const int64_t*, hipStream_t);

}  // namespace detail
}  // namespace xspmm
