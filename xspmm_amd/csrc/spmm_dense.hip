// spmm_dense.hip -- Tier-1 BCSR SpMM for a fully populated block grid (fp16).
//
// When nnzb == Mb * Kb every block-row holds all Kb blocks, and since block
// columns are strictly ascending within a row (the layout csr_to_bcsr
// produces, reference src/core/conversion.cpp:61), block (br, c) sits at
// index br * Kb + c.  The BCSR values array is then a block-tiled dense
// matrix and the product is GEMM-shaped: it is bound by the matrix cores, not
// by HBM.  Semantics are those of the tile kernel (reference
// src/common/spmm_math.hpp:20-146): blocks accumulate in column order, fp32
// accumulators, C overwritten; rows >= M and columns >= N are not stored and
// B rows >= K contribute nothing.
//
// Tiling.  A workgroup (8 waves, a 2 x 4 wave grid) owns 16 block-rows
// (256 rows of C) and 256 columns; each wave owns 8 block-rows x 64 columns,
// i.e. 8 x 4 MFMA tiles of 16 x 16 (128 fp32 accumulators per lane).  The
// 256 x 256 tile keeps the cache traffic per MFMA low: every K step moves
// 16 KB of A and 16 KB of B for 4.2 MFLOP.  Where that leaves the last round
// of workgroups part-empty, 14-block-row tiles (7 per wave) may fill the CUs
// better; the launcher picks the height.  K advances in slices of 32 (two
// block columns), two slices per pipeline step:
//   * each slice's 16 block-rows' two blocks (16 KB, contiguous per
//     block-row) and its 32 x 256 B panel (16 KB) go straight from memory
//     into an LDS stage with direct-to-LDS buffer loads (no staging
//     registers); the next step's loads are issued between the current
//     step's MFMAs;
//   * a wave reads each of its block-rows' A operand with one ds_read_b128
//     (the two blocks' rows in v_mfma_f32_16x16x32_f16 operand order, as
//     loaded) and each of its four B operands with two ds_read_b64_tr_b16
//     from the row-major panel, then issues 32 MFMAs;
//   * C leaves through LDS, one block-row per wave row at a time, as 16-byte
//     stores.
// grid: one workgroup per (row group, column group), ordered so that the
// column groups of a row group run on the same XCD and meet its A tile in that
// XCD's L2.
#include <atomic>

#include "internal.hpp"

namespace xspmm {
namespace detail {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

#ifndef XSPMM_DENSE_MINW
#define XSPMM_DENSE_MINW 2
#endif
#ifndef XSPMM_DENSE_STAGES
#define XSPMM_DENSE_STAGES 2
#endif
#ifndef XSPMM_DENSE_EPI
#define XSPMM_DENSE_EPI 2
#endif
#ifndef XSPMM_DENSE_KSUB
#define XSPMM_DENSE_KSUB 2
#endif
#ifndef XSPMM_DENSE_SPREAD
#define XSPMM_DENSE_SPREAD 1
#endif
#ifndef XSPMM_DENSE_TILE_ROWS
#define XSPMM_DENSE_TILE_ROWS 0  // 14 or 16 fixes the tile height; 0 lets the launcher choose
#endif
constexpr int kDN = 256;                     // columns per workgroup
constexpr int kDW = 8;                       // waves per workgroup
constexpr int kDThreads = 64 * kDW;
// waves form a kWR x kWC grid; each owns RW block-rows x kDTiles column tiles
constexpr int kWR = 2;
constexpr int kWC = kDW / kWR;
constexpr int kDTiles = 16 / kWC;            // 16-column tiles per wave
constexpr int kStageRows = 16;               // block-rows of an A stage (tile height <= 16)
constexpr int kABytes = kStageRows * 1024;   // A stage: 16 block-rows x 2 blocks
constexpr int kBRow = kDN * 2;               // B panel row: 512 bytes
constexpr int kBBytes = 32 * kBRow;          // B stage: 32 rows
constexpr int kStage = kABytes + kBBytes;    // 32 KB per 32-deep K slice
constexpr int kAU = kStageRows / kDW;        // A block-rows loaded per wave
constexpr int kBU = 16 / kDW;                // B panel row pairs loaded per wave
constexpr int kKSub = XSPMM_DENSE_KSUB;      // 32-deep K slices per pipeline stage
constexpr int kLoadsPerStep = kKSub * (kAU + kBU);  // direct-to-LDS loads per wave per stage
static_assert(kStageRows % kDW == 0 && 16 % kWC == 0, "wave grid");
constexpr int kRawWord3 = 0x00020000;        // raw dword buffer access (gfx9)
constexpr int kXcds = 8;                     // accelerator dies of an MI355X

typedef int i32x4_t __attribute__((ext_vector_type(4)));

// Raw buffer resource (4 SGPRs) over [base, base + bytes): loads at offsets
// past `bytes` return zeros without touching memory.
__device__ __forceinline__ i32x4_t raw_rsrc(const void* base, uint32_t bytes)
{
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    i32x4_t r;
    r.x = (int)(uint32_t)a;
    r.y = (int)(uint32_t)((a >> 32) & 0xffffu);  // stride 0
    r.z = (int)bytes;
    r.w = kRawWord3;
    return r;
}

__device__ __forceinline__ uint32_t lds_address(const void* p)
{
    return (uint32_t)(uintptr_t)(const __attribute__((address_space(3))) void*)p;
}

// One direct-to-LDS load: lane l's 16 bytes at byte `off` of the buffer land
// at LDS address lds + 16 l (buffer_load_dwordx4 ... lds, address base in M0).
// Issued as inline assembly so that the compiler adds no wait of its own: the
// callers wait with explicit s_waitcnt vmcnt.
__device__ __forceinline__ void load_to_lds(uint32_t lds, uint32_t off, i32x4_t rsrc)
{
    asm volatile("s_mov_b32 m0, %0\n\tbuffer_load_dwordx4 %1, %2, 0 offen lds"
                 :
                 : "s"(lds), "v"(off), "s"(rsrc)
                 : "memory", "m0");
}

// 16-byte chunk c of B panel row e is stored at chunk c ^ swz(e): the 16 rows
// one transpose read touches spread over all banks.
__device__ __forceinline__ uint32_t panel_swz(uint32_t e)
{
    return 2u * ((e & 3u) | (((e >> 3) & 1u) << 2));
}

typedef _Float16 half4_t __attribute__((ext_vector_type(4)));

// Whether the workgroup's block-rows [br0, br0 + rows) hold their blocks in
// the canonical full-grid layout: row br spans [br * Kb, (br + 1) * Kb) and
// block br * Kb + c has column c.  Every thread of the workgroup gets the
// answer.  Loads go out eight at a time, so a tile of 16 rows x 256 columns
// costs one memory round trip.
template <typename I>
__device__ bool tile_is_canonical(const I* __restrict__ brp, const I* __restrict__ bci,
                                  int64_t br0, int rows, int64_t Kb)
{
    const int t = threadIdx.x;
    bool ok = true;
    if (t <= rows) ok = (int64_t)brp[br0 + t] == (br0 + t) * Kb;
    // rows * Kb < 2^31: the launcher only takes grids with Mb * Kb * 512 < 2^31
    const uint32_t total = (uint32_t)rows * (uint32_t)Kb;
    const uint32_t kb = (uint32_t)Kb;
    const I* base = bci + br0 * Kb;
    for (uint32_t i0 = (uint32_t)t; i0 < total; i0 += 8u * kDThreads) {
        I v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t i = i0 + (uint32_t)u * kDThreads;
            v[u] = i < total ? base[i] : (I)(i % kb);
        }
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t i = i0 + (uint32_t)u * kDThreads;
            ok &= (int64_t)v[u] == (int64_t)(i % kb);
        }
    }
    return __syncthreads_and(ok ? 1 : 0) != 0;
}

// Product of a tile whose blocks are not in the canonical layout (a
// caller-built matrix with nnzb == Mb * Kb but another block order): every
// block of the row in stored order, as the reference tile kernel does
// (src/common/spmm_math.hpp:68-114), with v_mfma_f32_16x16x16_f16 and B read
// straight from memory.  Columns outside [0, Kb) contribute nothing, as in
// the column-batch kernel.  Wave w takes block-rows br0 + w, br0 + w + 8, ...
// and all 16 column tiles of the workgroup.  Slow, but only a malformed or
// unusual input takes it.
template <typename I>
__device__ void dense_tile_generic(const I* __restrict__ brp, const I* __restrict__ bci,
                                   const uint16_t* __restrict__ vals, const uint16_t* __restrict__ B,
                                   float* __restrict__ C, int64_t M, int64_t K, int64_t N,
                                   int64_t Mb, int64_t Kb, int64_t br0, int rows, int64_t n0,
                                   const I* __restrict__ row_map)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int li = lane & 15;
    const int g = lane >> 4;
    const _Float16* Bh = reinterpret_cast<const _Float16*>(B);
    for (int r = wave; r < rows; r += kDW) {
        const int64_t br = br0 + r;
        if (br >= Mb) break;
        float4_t acc[16];
#pragma unroll
        for (int j = 0; j < 16; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};
        const int64_t be = (int64_t)brp[br + 1];
        for (int64_t b = (int64_t)brp[br]; b < be; ++b) {
            const int64_t col = (int64_t)bci[b];
            if (col < 0 || col >= Kb) continue;
            // A[li][4g .. 4g + 3] of the block
            const half4_t a = *reinterpret_cast<const half4_t*>(vals + b * 256 + li * 16 + 4 * g);
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                const int64_t n = n0 + 16 * j + li;
                half4_t bo;
#pragma unroll
                for (int s = 0; s < 4; ++s) {
                    const int64_t k = 16 * col + 4 * g + s;
                    bo[s] = (k < K && n < N) ? Bh[k * N + n] : (_Float16)0.f;
                }
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x16f16(a, bo, acc[j], 0, 0, 0);
            }
        }
#pragma unroll
        for (int j = 0; j < 16; ++j) {
            const int64_t n = n0 + 16 * j + li;
            if (n >= N) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t row = 16 * br + 4 * g + q;
                if (row >= M) continue;
                const int64_t crow = row_map ? (int64_t)row_map[row] : row;
                C[crow * N + n] = acc[j][q];
            }
        }
    }
}

// RW: block-rows per wave (8: 256-row tiles; 7: 224-row tiles, whose A stage
// rows 14 and 15 load as zeros).  I: index type of brp / bci and of the
// optional output row map (C row row_map[r] receives product row r -- the
// clustered pipeline's un-permutation fused into the store; null stores rows
// in place).
template <int RW, typename I>
__global__ __launch_bounds__(kDThreads, XSPMM_DENSE_MINW) void spmm_f16_dense_kernel(const I* __restrict__ brp,
                                                                 const I* __restrict__ bci,
                                                                 const uint16_t* __restrict__ vals,
                                                                 const uint16_t* __restrict__ B,
                                                                 float* __restrict__ C,
                                                                 int64_t M, int64_t K,
                                                                 int64_t N, int64_t Mb,
                                                                 int64_t Kb,
                                                                 const I* __restrict__ row_map)
{
    constexpr int NS = XSPMM_DENSE_STAGES;
    constexpr int kDR = kWR * RW;  // block-rows per workgroup
    static_assert(RW >= 1 && kDR <= kStageRows, "tile height");
    static_assert(NS == 2 || NS == 3, "2 or 3 LDS stages");
    static_assert(NS * kKSub * kStage <= 160 * 1024, "LDS of one CU");
    __shared__ __align__(16) unsigned char smem[NS * kKSub * kStage];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = __builtin_amdgcn_readfirstlane(t >> 6);
    const int wr = wave / kWC;  // this wave's block-rows: RW wr .. RW wr + RW - 1
    const int wc = wave % kWC;  // and column tiles kDTiles wc .. + kDTiles - 1
    const int li = lane & 15;
    const int g = lane >> 4;

    // XCD-aware tile order.  Workgroup w runs on XCD w % 8 (round-robin
    // dispatch); the column groups of one row group get ids that share that
    // residue and are consecutive in dispatch order, so they meet the row
    // group's A tile in the same L2.
    int64_t rg, cg;
    {
        const int64_t w = blockIdx.x;
        const int64_t slot = w / kXcds, xcd = w % kXcds;
        const int64_t ncg = (N + kDN - 1) / kDN;
        rg = (slot / ncg) * kXcds + xcd;
        cg = slot % ncg;
    }
    if (rg * kDR >= Mb) return;  // padding workgroups of the last row-group band
    const int64_t n0 = cg * kDN;
    const int64_t br0 = rg * kDR;
    {
        const int rows = (int)(Mb - br0 < kDR ? Mb - br0 : kDR);
        if (!tile_is_canonical<I>(brp, bci, br0, rows, Kb)) {
            dense_tile_generic<I>(brp, bci, vals, B, C, M, K, N, Mb, Kb, br0, rows, n0, row_map);
            return;
        }
    }

    const uint32_t a_bytes = (uint32_t)(Mb * Kb * 512);
    const i32x4_t a_rsrc = raw_rsrc(vals, a_bytes);
    const uint32_t b_bytes = (uint32_t)(K * N * 2);
    const i32x4_t b_rsrc = raw_rsrc(B, b_bytes);
    const uint32_t lds0 = lds_address(smem);

    // --- direct-to-LDS loads of one K step (6 per wave) ----------------------
    // A: wave w moves block-rows 2w and 2w + 1: 1 KB each, the two consecutive
    // blocks of the step, lane l -> bytes 16l .. 16l + 15 (lanes >= 32 hold the
    // second block, which does not exist in the last step of an odd Kb).
    // B: wave w moves panel rows 8w + 2u and + 1 (u = 0..3): lane l lands at
    // chunk position l & 31 of row 8w + 2u + (l >> 5) and therefore loads
    // global chunk (l & 31) ^ swz(row).
    uint32_t a_off[kAU];
    bool a_row_ok[kAU];
#pragma unroll
    for (int u = 0; u < kAU; ++u) {
        const int64_t br = br0 + kAU * wave + u;
        a_row_ok[u] = kAU * wave + u < kDR && br < Mb;
        a_off[u] = (uint32_t)((a_row_ok[u] ? br : 0) * Kb * 512) + 16u * (uint32_t)lane;
    }
    const bool a_second = lane >= 32;
    uint32_t b_row[kBU];
    uint32_t b_col_off[kBU];
#pragma unroll
    for (int u = 0; u < kBU; ++u) {
        const uint32_t row = (uint32_t)(2 * kBU * wave + 2 * u + (lane >> 5));
        const uint32_t ch = (uint32_t)(lane & 31) ^ panel_swz(row);
        const int64_t col = n0 + 8 * (int64_t)ch;
        b_row[u] = row;
        b_col_off[u] = col < N ? (uint32_t)(2 * col) : 0xffffffffu;
    }
    // a stage holds kKSub slices of 32 K rows (two block columns) each, slice
    // q of stage s being K slice ks = kKSub s + q
    const int64_t steps = (Kb + 2 * kKSub - 1) / (2 * kKSub);
    // load i (0 .. kLoadsPerStep - 1) of step s: slice i / (kAU + kBU), then
    // the wave's kAU A block-rows and kBU B row pairs of that slice
    auto issue_load = [&](int64_t s, int i) {
        const int q = i / (kAU + kBU), u = i % (kAU + kBU);
        const int64_t ks = kKSub * s + q;
        const uint32_t base = lds0 + (uint32_t)(((s % NS) * kKSub + q) * kStage);
        if (u < kAU) {
            const bool ok = a_row_ok[u] && 2 * ks + (a_second ? 1 : 0) < Kb;
            const uint32_t off = ok ? a_off[u] + (uint32_t)(ks * 1024) : a_bytes;
            load_to_lds(base + (uint32_t)((kAU * wave + u) * 1024), off, a_rsrc);
        } else {
            const int v = u - kAU;
            const int64_t k = 32 * ks + b_row[v];
            const uint32_t off = (k < K && b_col_off[v] != 0xffffffffu)
                                     ? (uint32_t)(k * N * 2) + b_col_off[v]
                                     : b_bytes;
            load_to_lds(base + (uint32_t)(kABytes + (2 * kBU * wave + 2 * v) * kBRow), off, b_rsrc);
        }
    };

    // --- operand reads --------------------------------------------------------
    // transpose reads: rows 8g + (li >> 2) and + 4, chunk 2 * tile + ((li & 3) >> 1)
    const uint32_t tr_e = (uint32_t)(8 * g + (li >> 2));
    const uint32_t tr_base = (uint32_t)kABytes + tr_e * kBRow + 8u * (uint32_t)(li & 1);
    const uint32_t tr_swz = panel_swz(tr_e);
    const uint32_t tr_cc = (uint32_t)((li & 3) >> 1);
    // A operand of a pair: block lane >> 5, row li, halves 8 * ((lane >> 4) & 1) .. +8
    const uint32_t a_lane = (uint32_t)((lane >> 5) * 512 + li * 32 + ((lane >> 4) & 1) * 16);

    float4_t acc[RW][kDTiles];
#pragma unroll
    for (int r = 0; r < RW; ++r)
#pragma unroll
        for (int j = 0; j < kDTiles; ++j) acc[r][j] = float4_t{0.f, 0.f, 0.f, 0.f};

    // One stage's MFMAs.  The loads of step `next` (none if next < 0) are
    // spread over its kKSub * RW row groups rather than issued back to back:
    // eight waves issuing all their loads at once queue behind one another at
    // the CU's texture unit and hold up their MFMAs.
    constexpr int kGroups = kKSub * RW;
    auto compute_step = [&](int stage, int64_t next) {
#pragma unroll
        for (int q = 0; q < kKSub; ++q) {
            const unsigned char* S = smem + (stage * kKSub + q) * kStage;
            half8_t bop[kDTiles];
#pragma unroll
            for (int j = 0; j < kDTiles; ++j) {
                const uint32_t c = (uint32_t)(2 * (kDTiles * wc + j)) + tr_cc;
                const uint32_t a = tr_base + ((c ^ tr_swz) << 4);
                unsigned char* P = const_cast<unsigned char*>(S) + a;
                const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)P);
                const short4_t hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(P + 4 * kBRow));
                bop[j] = __builtin_bit_cast(half8_t,
                                            __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
            }
#pragma unroll
            for (int r = 0; r < RW; ++r) {
                const half8_t aop = __builtin_bit_cast(
                    half8_t, *reinterpret_cast<const u32x4_t*>(S + (RW * wr + r) * 1024 + a_lane));
#pragma unroll
                for (int j = 0; j < kDTiles; ++j)
                    acc[r][j] =
                        __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop[j], acc[r][j], 0, 0, 0);
                if (XSPMM_DENSE_SPREAD && next >= 0) {
#pragma unroll
                    for (int i = 0; i < kLoadsPerStep; ++i)
                        if (i * kGroups / kLoadsPerStep == q * RW + r) issue_load(next, i);
                }
            }
        }
    };

    // LDS ring of NS stages of kKSub slices each (two stages of two slices by
    // default; measured: three stages of one slice, or one slice per stage
    // with the loads spread, are slower).  Every wave issues exactly
    // kLoadsPerStep loads per step and no other vector-memory loads, so "at
    // most kLoadsPerStep outstanding" (three stages) or "none outstanding"
    // (two) means this wave's loads of step s have landed; the barrier then
    // makes every wave's visible and guarantees that the stage step s + NS - 1
    // is loaded into, last read at step s - 1, is free.
    auto issue_step = [&](int64_t s) {
#pragma unroll
        for (int i = 0; i < kLoadsPerStep; ++i) issue_load(s, i);
    };
    if (steps > 0) issue_step(0);
    if (NS == 3 && steps > 1) issue_step(1);
    for (int64_t s = 0; s < steps; ++s) {
        if (NS == 3 && s + 1 < steps)
            asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kLoadsPerStep) : "memory");
        else
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        __syncthreads();
        const int64_t next = s + NS - 1 < steps ? s + NS - 1 : -1;
        if (!XSPMM_DENSE_SPREAD && next >= 0) issue_step(next);
        compute_step((int)(s % NS), next);
    }

    // --- store: lane holds C[16 br + 4g + q][16 tile + li] ------------------
    if constexpr (XSPMM_DENSE_EPI == 2) {
        // Through LDS, RW rounds: in round r every wave writes its r-th
        // block-row (16 x kDTiles*16 fp32, MFMA order) and the workgroup reads
        // the kWR * 16 rows back row-major, so every lane stores 16 contiguous
        // bytes (1 KB rows per workgroup).
        __syncthreads();  // the last step's operand reads are done
        float* T = reinterpret_cast<float*>(smem);  // [kWR * 16][256 + 4] fp32
        constexpr int TS = kDN + 4;
        constexpr int TR = kWR * 16;               // rows staged per round
        constexpr int TPR = kDThreads / TR;        // threads per row
        const int row_l = t / TPR;
        const int col_l = (t % TPR) * 4;           // +4 * TPR per pass
#pragma unroll
        for (int r = 0; r < RW; ++r) {
#pragma unroll
            for (int j = 0; j < kDTiles; ++j)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    T[(16 * wr + 4 * g + q) * TS + 16 * kDTiles * wc + 16 * j + li] = acc[r][j][q];
            __syncthreads();
            const int64_t row = 16 * (br0 + RW * (row_l / 16) + r) + (row_l % 16);
            const int64_t crow = (row_map && row < M) ? (int64_t)row_map[row] : row;
#pragma unroll
            for (int p = 0; p < kDN / (4 * TPR); ++p) {
                const int c = col_l + 4 * TPR * p;
                const float4_t v = *reinterpret_cast<const float4_t*>(T + row_l * TS + c);
                const int64_t col = n0 + c;
                if (row < M && col < N) {
                    // 16-byte stores only where C's rows stay 16-byte aligned
                    if (col + 4 <= N && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0)
                        __builtin_nontemporal_store(v, reinterpret_cast<float4_t*>(C + crow * N + col));
                    else
                        for (int e = 0; e < 4 && col + e < N; ++e) C[crow * N + col + e] = v[e];
                }
            }
            __syncthreads();
        }
    } else {
#pragma unroll
        for (int r = 0; r < RW; ++r) {
            const int64_t row0 = 16 * (br0 + RW * wr + r) + 4 * g;
#pragma unroll
            for (int j = 0; j < kDTiles; ++j) {
                const int64_t col = n0 + 16 * kDTiles * wc + 16 * j + li;
                if (col >= N) continue;
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    if (row0 + q < M) {
                        const int64_t crow = row_map ? (int64_t)row_map[row0 + q] : row0 + q;
                        if constexpr (XSPMM_DENSE_EPI == 1)
                            __builtin_nontemporal_store(acc[r][j][q], C + crow * N + col);
                        else
                            C[crow * N + col] = acc[r][j][q];
                    }
            }
        }
    }
}

}  // namespace

namespace {
// workgroups of the dense grid for tiles of dr block-rows: row groups padded
// to a multiple of the XCD count (padding groups exit) times column groups
int64_t dense_groups(int64_t Mb, int64_t N, int64_t dr)
{
    const int64_t ncg = (N + kDN - 1) / kDN;
    const int64_t nrg = (Mb + dr - 1) / dr;
    return ((nrg + kXcds - 1) / kXcds) * kXcds * ncg;
}

// compute units of the current device (one workgroup of this kernel fits a
// CU), queried once per device
int64_t device_cus()
{
    constexpr int kMaxDev = 64;
    static std::atomic<int> cus[kMaxDev];
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return 256;
    int n = cus[dev].load(std::memory_order_relaxed);
    if (n <= 0) {
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        cus[dev].store(n, std::memory_order_relaxed);
    }
    return n;
}

// Tile height (block-rows per workgroup): 16 or 14.  A workgroup's time is
// about proportional to its height and every CU holds one workgroup, so the
// grid takes rounds(h) = ceil(tiles(h) / CUs) workgroup times of height h;
// the height with the smaller rounds(h) * h wins (16 on ties: its loads per
// MFMA are lower).  E.g. 896 block-rows x 8 column groups on 256 CUs: 448
// tiles of 16 (two rounds, a quarter of the second idle) against 512 of 14
// (two full rounds).
int dense_tile_rows(int64_t Mb, int64_t N)
{
    const int64_t ncg = (N + kDN - 1) / kDN;
    const int64_t cus = device_cus();
    auto cost = [&](int64_t h) { return ((((Mb + h - 1) / h) * ncg + cus - 1) / cus) * h; };
    if (XSPMM_DENSE_TILE_ROWS == 14 || XSPMM_DENSE_TILE_ROWS == 16) return XSPMM_DENSE_TILE_ROWS;
    return cost(14) < cost(16) ? 14 : 16;
}
}  // namespace

bool spmm_dense_f16_covers(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, int64_t N)
{
    (void)M;
    if (nnzb != Mb * Kb || Mb <= 0 || Kb <= 0 || N <= 0) return false;
    if (N % 8 != 0) return false;
    if (Mb * Kb * 512 >= (int64_t(1) << 31) || K * N * 2 >= (int64_t(1) << 31)) return false;
    return dense_groups(Mb, N, 14) <= 0x7fffffffLL;
}

template <typename I>
bool bcsr_spmm_dense_f16(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb,
                         const I* brp, const I* bci, const uint16_t* bvals, const uint16_t* B,
                         float* C, int64_t N, hipStream_t s, const I* row_map)
{
    if (!spmm_dense_f16_covers(M, K, Mb, Kb, nnzb, N)) return false;
    const int h = dense_tile_rows(Mb, N);
    const int64_t groups = dense_groups(Mb, N, h);
    if (h == 14)
        hipLaunchKernelGGL((spmm_f16_dense_kernel<7, I>), dim3((unsigned)groups), dim3(kDThreads), 0,
                           s, brp, bci, bvals, B, C, M, K, N, Mb, Kb, row_map);
    else
        hipLaunchKernelGGL((spmm_f16_dense_kernel<8, I>), dim3((unsigned)groups), dim3(kDThreads), 0,
                           s, brp, bci, bvals, B, C, M, K, N, Mb, Kb, row_map);
    XSPMM_LAUNCH_CHECK();
    return true;
}

template bool bcsr_spmm_dense_f16<int32_t>(int64_t, int64_t, int64_t, int64_t, int64_t,
                                           const int32_t*, const int32_t*, const uint16_t*,
                                           const uint16_t*, float*, int64_t, hipStream_t,
                                           const int32_t*);
template bool bcsr_spmm_dense_f16<int64_t>(int64_t, int64_t, int64_t, int64_t, int64_t,
                                           const int64_t*, const int64_t*, const uint16_t*,
                                           const uint16_t*, float*, int64_t, hipStream_t,
                                           const int64_t*);

}  // namespace detail
}  // namespace xspmm
