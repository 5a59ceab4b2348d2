// spmm.hip -- Tier-1 BCSR SpMM on CDNA4 matrix cores (gfx950).
//
// Semantics follow the reference tile kernel (src/common/spmm_math.hpp:20-146):
// for block-row br, C[16*br : +16, :] = sum over the row's blocks (in col_ind
// order) of A_blk * B[16*col : +16, :]; C is overwritten and block-rows without
// blocks become zero.  Rows >= M are not stored; B rows >= K and columns >= N
// contribute nothing.
//
// fp16 kernels (v_mfma_f32_16x16x32_f16; MFMA operands want K contiguous in
// every lane while B is row-major, so B reaches the matrix cores either through
// the gfx950 LDS transpose read or through a repacked copy):
//   spmm_f16_batch_kernel   default (N % 8 == 0): the non-zero block columns of
//                           a row's block pairs are compacted into K = 32
//                           batches and multiplied with their gathered B rows;
//                           count / pack modes store the batches for
//                           spmm_f16_packed_kernel (prepared products);
//   spmm_f16_dense_kernel   (spmm_dense.hip) fully populated block grids;
//   spmm_f16_gather_kernel  per-pair masked B-row gather (XSPMM_SPMM_KERNEL=gather);
//   pack_b_panels + spmm_f16_kernel  any N: B repacked into 16-row panels laid
//                           out [block_col][n][k16], two blocks per K = 32 operand.
//
// fp32 kernels.  v_mfma_f32_16x16x4f32 takes one k per lane, so B is read
// row-major directly:
//   spmm_f32_batch_kernel   (spmm_f32.hip) default where the grid has at
//                           least 512 workgroups of 128 columns: the non-zero
//                           block columns of a block-row packed four to a
//                           K = 4 batch;
//   spmm_f32_short_kernel   short grids: lane l loads A[l&15][4g .. 4g+3]
//                           (g = l>>4) once per block and issues four MFMAs,
//                           step s pairing A[i][4g+s] with B[16*col + 4g + s][n]
//                           (B through a buffer resource);
//   spmm_f32_kernel         the same with 64-bit B addressing, for short
//                           grids whose B offsets exceed 30 bits.
//
// Work split: one workgroup per block-row (grid.x, or the dispatch order of
// order_rows_kernel / xcd_rows_kernel), N split over grid.y.
#include <cstdlib>
#include <mutex>
#include <string>

#include "internal.hpp"
#include "scan.hpp"

namespace xspmm {
namespace detail {

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWave = 64;

__device__ __forceinline__ half8_t load_h8(const uint16_t* p)
{
    u32x4_t v = *reinterpret_cast<const u32x4_t*>(p);
    return __builtin_bit_cast(half8_t, v);
}

// ---------------------------------------------------------------------------
// B (K x N fp16, row-major) -> panels Bt[kb][n][16], n < Np = 16*ceil(N/16).
// Thread (kb, n, h) writes the 8 halves k = 16*kb + 8*h .. +8 of column n.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void pack_b_panels(const uint16_t* __restrict__ B,
                                                     uint16_t* __restrict__ Bt, int64_t K,
                                                     int64_t N, int64_t Kb, int64_t Np)
{
    const int64_t per_kb = Np * 2;
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= per_kb) return;
    const int64_t n = t >> 1;
    const int h = (int)(t & 1);
    for (int64_t kb = blockIdx.y; kb < Kb; kb += gridDim.y) {
        uint32_t w[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const int64_t k0 = kb * 16 + h * 8 + e;
            uint32_t lo = (k0 < K && n < N) ? B[k0 * N + n] : 0u;
            uint32_t hi = (k0 + 1 < K && n < N) ? B[(k0 + 1) * N + n] : 0u;
            w[e >> 1] = lo | (hi << 16);
        }
        u32x4_t v = {w[0], w[1], w[2], w[3]};
        *reinterpret_cast<u32x4_t*>(Bt + ((kb * Np + n) * 2 + h) * 8) = v;
    }
}

// ---------------------------------------------------------------------------
// fp16 x fp16 -> fp32 tile kernel.
// ---------------------------------------------------------------------------
template <typename I, int NTW>
__global__ __launch_bounds__(256) void spmm_f16_kernel(const I* __restrict__ brp,
                                                       const I* __restrict__ bci,
                                                       const uint16_t* __restrict__ vals,
                                                       const uint16_t* __restrict__ Bt,
                                                       float* __restrict__ C, int64_t M,
                                                       int64_t N, int64_t Np, int64_t Kb,
                                                       int ntiles)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int waves = blockDim.x / kWave;
    const int tile0 = (blockIdx.y * waves + wave) * NTW;
    if (tile0 >= ntiles) return;  // no barriers below: idle waves may leave

    const int64_t br = blockIdx.x;
    const int64_t rs = brp[br];
    const int64_t re = brp[br + 1];
    const int sel = lane >> 5;          // which block of the pair
    const int kh = (lane >> 4) & 1;     // which 8-wide k half
    const int li = lane & 15;           // A row / B column within the tile

    float4_t acc[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

    auto load = [&](int64_t p, half8_t& a, half8_t (&b)[NTW]) {
        const int64_t blk = p + sel;
        a = half8_t{};
#pragma unroll
        for (int j = 0; j < NTW; ++j) b[j] = half8_t{};
        const int64_t col = blk < re ? (int64_t)bci[blk] : -1;
        if (col >= 0 && col < Kb) {  // a block column outside the grid contributes nothing
            a = load_h8(vals + blk * 256 + li * 16 + kh * 8);
            const uint16_t* bp = Bt + (col * Np + (int64_t)tile0 * 16 + li) * 16 + kh * 8;
#pragma unroll
            for (int j = 0; j < NTW; ++j)
                if (tile0 + j < ntiles) b[j] = load_h8(bp + (int64_t)j * 256);
        }
    };

    half8_t a0, b0[NTW];
    if (rs < re) load(rs, a0, b0);
    for (int64_t p = rs; p < re; p += 2) {
        half8_t a1, b1[NTW];
        if (p + 2 < re) load(p + 2, a1, b1);
#pragma unroll
        for (int j = 0; j < NTW; ++j)
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a0, b0[j], acc[j], 0, 0, 0);
        a0 = a1;
#pragma unroll
        for (int j = 0; j < NTW; ++j) b0[j] = b1[j];
    }

    const int g = lane >> 4;
#pragma unroll
    for (int j = 0; j < NTW; ++j) {
        const int64_t col = (int64_t)(tile0 + j) * 16 + li;
        if (tile0 + j >= ntiles || col >= N) continue;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int64_t row = br * 16 + g * 4 + r;
            if (row < M) C[row * N + col] = acc[j][r];
        }
    }
}

// ---------------------------------------------------------------------------
// fp16 "gather" tile kernel: the default for fp16.
//
// A block usually touches far fewer than its 16 columns (0.7 % fill at the
// headline configuration), and only the B rows of touched columns can change
// C.  Per pair of blocks the wave therefore
//   1. loads the A pair in MFMA operand layout (16 bytes per lane);
//   2. forms the 32-bit slot mask of columns with a non-zero entry (each lane
//      flags its non-zero halves, a 16-lane OR gives the mask of its k group);
//   3. lists the masked slots in lane order (lane p ranks its bit and forwards
//      p to lane rank) and computes every listed row's byte offset in B in
//      its own lane;
//   4. issues exactly F row loads (F masked rows; unused ones re-read row 0,
//      further ones take a slower path), one dword per lane = two columns of
//      its 128-column chunk -- a fixed count keeps the in-order load counter
//      waits static, so rows stay in flight across pairs;
//   5. transposes the rows through a per-wave LDS tile T[n][slot] into the
//      MFMA B operand (one ds_read_b128 per 16x32 fragment) and clears the
//      written slots again after the reads, so unmasked slots always hold
//      zeros (stale data could be non-finite; A is zero there anyway);
//   6. issues one v_mfma_f32_16x16x32_f16 per 16-column tile.
// Every non-empty block still feeds an MFMA; what is skipped is the B traffic
// of all-zero columns.  A runs three pairs ahead of the multiply and B rows
// two.  On CDNA a wave64 VALU instruction holds the SIMD for four cycles, so
// the per-pair bookkeeping is kept to a few dozen vector instructions.
// The four waves of a workgroup split the block-row's pairs evenly (balancing
// long rows) and their partial 16 x 128 tiles are summed in LDS.
// grid = (block-rows, ceil(N / 128)); N even and B < 4 GiB on this path.
// ---------------------------------------------------------------------------
// Per-wave LDS tile: two sub-tiles (even / odd columns n = 2*lam, 2*lam+1)
// of 64 rows x 16 dwords (32 slots).  The 16-byte chunk c of row lam sits at
// chunk c ^ ((lam >> 2) & 3), and the odd sub-tile starts 8 banks after a
// 64-bank boundary: the 16 lanes of a fragment read then hit 16 disjoint
// 4-bank groups, and a row write (64 lanes, one slot) is 4-way.  8.2 KB per
// wave, so four workgroups fit in the 160 KB of a CU.
constexpr int kTileQ = 16;
constexpr int kOddBase = 64 * kTileQ + 8;
// dwords per wave, padded so every wave's tile starts on a 64-byte boundary
constexpr int kTileWords = ((kOddBase + 64 * kTileQ + 15) / 16) * 16;
// B row loads issued per pair (a pair's further masked rows take a slower
// path).  At the headline configuration 98 % of pairs need at most 6 rows.
#ifndef XSPMM_GATHER_ROWS
#define XSPMM_GATHER_ROWS 6
#endif
constexpr int kGatherRows = XSPMM_GATHER_ROWS;

typedef uint16_t ushort2_t __attribute__((ext_vector_type(2)));

struct GatherA {
    half8_t a;      // A operand of the pair (in flight)
    uint32_t colv;  // block column of this lane's block (in flight)
};

template <int F>
struct GatherRows {
    half8_t a;
    uint32_t mask;     // 32-bit slot mask (wave-uniform)
    uint32_t cnt;      // masked slots (wave-uniform)
    uint32_t slotv;    // lane r < cnt: (B row << 5) | slot of the pair's r-th masked row
    uint32_t offv;     // lane r < cnt: byte offset of that row in B (else: past B)
    uint32_t rows[F];  // B row r < F: columns n0+2*lane, n0+2*lane+1
};

// Cache-policy operand of the buffer-load builtins: non-temporal (nt).
constexpr int kNonTemporal = 2;

// Buffer resource word 3 for raw (untyped, unswizzled) dword access on gfx9.
constexpr int kRawBufferWord3 = 0x00020000;

__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             kRawBufferWord3);
}

// Low dword of a block column; an int64 index with a non-zero high dword
// reads as 0xffffffff (never a valid block column).
template <typename I>
__device__ __forceinline__ uint32_t load_block_col(__amdgpu_buffer_rsrc_t r, uint32_t voff,
                                                   uint32_t soff)
{
    if constexpr (sizeof(I) == 4) {
        return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(r, (int)voff, (int)soff, 0);
    } else {
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t v = __builtin_amdgcn_raw_buffer_load_b64(r, (int)voff, (int)soff, 0);
        return v.y == 0u ? v.x : 0xffffffffu;
    }
}

template <typename I, int NT, int F>
__global__ __launch_bounds__(256) void spmm_f16_gather_kernel(const I* __restrict__ brp,
                                                              const I* __restrict__ bci,
                                                              const uint16_t* __restrict__ vals,
                                                              const uint16_t* __restrict__ B,
                                                              float* __restrict__ C, int64_t M,
                                                              int64_t K, int64_t N, int64_t Kb)
{
    __shared__ __align__(16) uint32_t tiles[4 * kTileWords];
    const int lane = threadIdx.x & (kWave - 1);
    // wave-uniform (the compiler cannot infer it from threadIdx.x), so all
    // block bookkeeping below stays in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    uint32_t* T = tiles + wave * kTileWords;

    const int64_t br = blockIdx.x;
    const int64_t n0 = (int64_t)blockIdx.y * 128;
    const int64_t rs = brp[br];
    const int64_t re = brp[br + 1];
    const int64_t npairs = (re - rs + 1) >> 1;
    const int64_t q0 = npairs * wave / 4;
    const int64_t q1 = npairs * (wave + 1) / 4;

    const int li = lane & 15;
    const int g = lane >> 4;
    const int sel = lane >> 5;
    const int kh = g & 1;

    // --- loop-invariant quantities ------------------------------------------
    // This wave's blocks [wb0, wb1) are read through buffer resources: a read
    // past them (the missing second block of an odd row, the pairs after q1
    // that the software pipeline runs into) returns zeros, which give an empty
    // slot mask.  Pair q sits at byte (q - q0) * 1024 of the A resource.  All
    // offsets go into the per-lane offset operand, which the range check
    // covers.
    const int64_t wb0 = rs + 2 * q0;
    const int64_t wb1 = (rs + 2 * q1 < re) ? rs + 2 * q1 : re;
    const uint32_t nblk = (uint32_t)(wb1 > wb0 ? wb1 - wb0 : 0);
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(vals + wb0 * 256, nblk * 512u);
    const __amdgpu_buffer_rsrc_t c_rsrc = make_rsrc(bci + wb0, nblk * (uint32_t)sizeof(I));
    // B: K * N * 2 <= 2^31 on this path, so an offset of b_bytes plus a lane
    // offset neither wraps nor lands inside B: rows at that offset read as zero
    // without touching memory.
    const uint32_t b_bytes = (uint32_t)(K * N * 2);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(B, b_bytes);
    // A operand: block (lane >> 5) of the pair, row li, halves 8*kh .. +8
    const uint32_t a_voff = (uint32_t)(sel * 512 + li * 32 + kh * 16);
    const uint32_t c_voff = (uint32_t)(sel * sizeof(I));
    // B rows: this lane reads columns n0 + 2*lane and +1 as one dword.  Past N
    // the offset is clamped into the row: such elements land in tile columns
    // >= N, which are never stored.
    const uint32_t lane_off =
        (uint32_t)(2 * ((n0 + 2 * lane + 1 < N) ? n0 + 2 * lane : N - 2));
    const uint32_t rowbytes = (uint32_t)(2 * N);  // < 2^23 on this path
    // slot listing: lane p < 32 owns mask bit p, i.e. column p & 15 of block
    // (p >> 4) of the pair, and sends ((16 * block column + (p & 15)) << 5) | p
    const uint32_t p_bit = (uint32_t)lane & 31u;
    const uint32_t below_p = (1u << p_bit) - 1u;
    const uint32_t p_code = ((p_bit & 15u) << 5) | p_bit;
    const bool p_hi = (p_bit & 16u) != 0u;
    // LDS tile: slot s of this lane's even row is at byte lane_base ^ (2 * s)
    // of the workgroup's tiles, i.e. chunk (s >> 3) ^ swizzle, half s & 7 of
    // row lane (the wave's tile starts on a 64-byte boundary).
    const uint32_t lane_base = 4u * (uint32_t)(wave * kTileWords) + 64u * (uint32_t)lane +
                               16u * (uint32_t)((lane >> 2) & 3);
    constexpr uint32_t kOddDelta = 4 * kOddBase;
    char* const Lc = reinterpret_cast<char*>(tiles);
    char* const Tc = reinterpret_cast<char*>(T);
    // fragment j of this lane: row lam = 8j + li/2 of the even/odd sub-tile,
    // chunk g (swizzled)
    uint32_t frag_off[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) {
        const int lam = 8 * j + (li >> 1);
        frag_off[j] = 4u * (uint32_t)(((li & 1) ? kOddBase : 0) + lam * kTileQ +
                                      4 * ((g ^ (lam >> 2)) & 3));
    }
    // 0x00010001, hidden from the optimiser: min(x, one) on the two halves
    // then stays one packed integer instruction instead of two compares
    uint32_t one;
    asm("s_mov_b32 %0, 0x10001" : "=s"(one));
    const uint32_t kb32 = (uint32_t)Kb;  // < 2^20 on this path: B rows < 2^24

    // the tile starts (and, after every pair, returns to) all zeros
    for (int w = lane; w < kTileWords / 4; w += kWave)
        reinterpret_cast<u32x4_t*>(T)[w] = u32x4_t{0u, 0u, 0u, 0u};

    float4_t acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

    // Stage A: issue the loads of pair q's A operand and block columns.
    auto stage_a = [&](int64_t q, GatherA& P) {
        const uint32_t pq = (uint32_t)(q - q0);
        P.a = __builtin_bit_cast(
            half8_t, __builtin_amdgcn_raw_buffer_load_b128(a_rsrc, (int)(a_voff + pq * 1024u), 0, 0));
        P.colv = load_block_col<I>(c_rsrc, c_voff + pq * 2u * (uint32_t)sizeof(I), 0u);
    };
    // Stage R: mask, listed slots, row offsets, then the F row loads.
    auto stage_rows = [&](const GatherA& P, GatherRows<F>& R) {
        const uint32_t c0 = (uint32_t)__builtin_amdgcn_readlane((int)P.colv, 0);
        const uint32_t c1 = (uint32_t)__builtin_amdgcn_readlane((int)P.colv, 32);
        R.a = P.a;
        const u32x4_t w = __builtin_bit_cast(u32x4_t, R.a);
        // per 16-bit half: 1 if |x| != 0
        uint32_t nz[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const ushort2_t h = __builtin_bit_cast(ushort2_t, w[d] & 0x7fff7fffu);
            nz[d] = __builtin_bit_cast(
                uint32_t, __builtin_elementwise_min(h, __builtin_bit_cast(ushort2_t, one)));
        }
        // element e = 2d (+1 for the high half) -> bit e
        uint32_t v = nz[0] | (nz[1] << 2) | (nz[2] << 4) | (nz[3] << 6);
        v = (v | (v >> 15)) & 0xffu;
        // OR over the 16 lanes of the k group: DPP row rotations by 1, 2, 4, 8
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x121, 0xf, 0xf, false);
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x122, 0xf, 0xf, false);
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, false);
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false);
        // a block column past Kb (malformed input) lists no rows: its block
        // meets only zero slots
        const uint32_t valid = (c0 < kb32 ? 0x0000ffffu : 0u) | (c1 < kb32 ? 0xffff0000u : 0u);
        const uint32_t m = ((uint32_t)__builtin_amdgcn_readlane((int)v, 0) |
                            ((uint32_t)__builtin_amdgcn_readlane((int)v, 16) << 8) |
                            ((uint32_t)__builtin_amdgcn_readlane((int)v, 32) << 16) |
                            ((uint32_t)__builtin_amdgcn_readlane((int)v, 48) << 24)) &
                           valid;
        R.mask = m;
        R.cnt = (uint32_t)__builtin_popcount(m);
        const bool send = lane < 32 && ((m >> p_bit) & 1u);
        const uint32_t rank = (uint32_t)__builtin_popcount(m & below_p);
        const uint32_t code = ((p_hi ? c1 : c0) << 9) + p_code;
        // lanes with nothing to send all target lane 63, which is never read
        const uint32_t sv =
            (uint32_t)__builtin_amdgcn_ds_permute((int)((send ? rank : 63u) * 4u), (int)code);
        R.slotv = sv;
        // rows of a malformed block that run past K read zeros
        R.offv = ((uint32_t)lane < R.cnt) ? __umul24(sv >> 5, rowbytes) : b_bytes;
#pragma unroll
        for (int r = 0; r < F; ++r)
            R.rows[r] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                b_rsrc, (int)(lane_off + (uint32_t)__builtin_amdgcn_readlane((int)R.offv, r)), 0, 0);
    };
    auto put = [&](uint32_t addr, uint32_t r) {
        *reinterpret_cast<uint16_t*>(Lc + addr) = (uint16_t)(r & 0xffffu);
        *reinterpret_cast<uint16_t*>(Lc + addr + kOddDelta) = (uint16_t)(r >> 16);
    };
    auto slot_addr = [&](const GatherRows<F>& R, int r) -> uint32_t {
        return lane_base ^ (2u * ((uint32_t)__builtin_amdgcn_readlane((int)R.slotv, r) & 31u));
    };
    // Stage M: rows into the tile, fragments out, multiply, clear the slots.
    auto stage_mma = [&](const GatherRows<F>& R) {
        if (R.mask == 0u) return;
        uint32_t addr[F];
#pragma unroll
        for (int r = 0; r < F; ++r) {
            addr[r] = slot_addr(R, r);
            if ((uint32_t)r < R.cnt) put(addr[r], R.rows[r]);
        }
        for (uint32_t r = F; r < R.cnt; ++r)  // rare: more than F rows
            put(slot_addr(R, (int)r),
                (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                    b_rsrc,
                    (int)(lane_off + (uint32_t)__builtin_amdgcn_readlane((int)R.offv, (int)r)), 0,
                    0));
#pragma unroll
        for (int j = 0; j < NT; ++j) {
            const u32x4_t raw = *reinterpret_cast<const u32x4_t*>(Tc + frag_off[j]);
            acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(R.a, __builtin_bit_cast(half8_t, raw),
                                                           acc[j], 0, 0, 0);
        }
        // LDS executes a wave's operations in order: these clears land after
        // the fragment reads above.
#pragma unroll
        for (int r = 0; r < F; ++r)
            if ((uint32_t)r < R.cnt) put(addr[r], 0u);
        for (uint32_t r = F; r < R.cnt; ++r) put(slot_addr(R, (int)r), 0u);
    };

    if (q0 < q1) {
        // A (and block columns) run three pairs ahead of the multiply, B rows
        // two pairs ahead.  Pairs past q1 are empty and cost no row traffic.
        GatherA A0, A1, A2;
        GatherRows<F> X, Y, Z;
        stage_a(q0, A0);
        stage_a(q0 + 1, A1);
        stage_a(q0 + 2, A2);
        stage_rows(A0, X);
        stage_rows(A1, Y);
        for (int64_t q = q0; q < q1; q += 3) {
            stage_a(q + 3, A0);
            stage_mma(X);
            stage_rows(A2, Z);
            stage_a(q + 4, A1);
            stage_mma(Y);
            stage_rows(A0, X);
            stage_a(q + 5, A2);
            stage_mma(Z);
            stage_rows(A1, Y);
        }
    }

    // Sum the four waves' partial tiles through LDS and store C.
    __syncthreads();
    float* red = reinterpret_cast<float*>(tiles);  // 4 x [16][128] fp32 = 32 KB
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave * 2048 + (4 * g + r) * 128 + 16 * j + li] = acc[j][r];
    __syncthreads();
    const int t = threadIdx.x;
    const int row = t >> 4;
    const int c0 = (t & 15) * 8;
    const int64_t grow = br * 16 + row;
    if (grow < M && c0 < NT * 16) {
        float out[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            const int o = row * 128 + c0 + e;
            out[e] = red[o] + red[2048 + o] + red[4096 + o] + red[6144 + o];
        }
        float* dst = C + grow * N + n0 + c0;
        if (n0 + c0 + 8 <= N && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0) {
            *reinterpret_cast<float4*>(dst) = make_float4(out[0], out[1], out[2], out[3]);
            *reinterpret_cast<float4*>(dst + 4) = make_float4(out[4], out[5], out[6], out[7]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (n0 + c0 + e < N) dst[e] = out[e];
        }
    }
}

// ---------------------------------------------------------------------------
// fp16 "column batch" tile kernel (the Tier-1 default where N % 8 == 0).
//
// All blocks of a block-row add into the same 16 rows of C, so the K extent
// of a multiply does not have to follow block boundaries: the non-zero
// columns of any blocks of the row can be stacked into one K = 32 operand.
// The four waves of a workgroup take the row's block pairs in turn (wave w:
// pairs w, w + 4, ...) and each wave
//   1. streams its pairs in MFMA operand layout (16 bytes per lane, lane
//      (r, g): row r, pair columns 8g .. 8g+7; non-temporal loads, batch_depth
//      pairs in flight) and, one vector load per ring pass, the pairs' block
//      columns;
//   2. forms the pair's 32-bit mask of columns holding a non-zero (per-lane
//      masks OR-ed over the wave by DPP);
//   3. appends the masked columns to a batch of 32 K slots.  The columns are
//      moved into their slots on the matrix cores: with the pair as the B
//      operand and a one-hot selection S^T (16 slots x 32 pair columns) as
//      the A operand,
//          D_h += S_h^T * pair^T
//      accumulates the transposed A' of slots 16h .. 16h+15 (lane (r, g) of
//      D_h holds A'[r][16h + 4g .. +3]).  Each D entry receives one product
//      x * 1.0 and zeros, so the compaction is exact (a -0.0 entry becomes
//      +0.0, which changes no sum of products).  S^T lives in LDS, all zero
//      between pairs: column lane (i < 8, g) of a set pair column writes 1.0
//      at [slot][column] before the read and 0 after it, and the column's B
//      row index into the slot list;
//   4. when a pair does not fit, closes the batch: converts D to the fp16 A'
//      operand, multiplies the previous batch, and issues the 16-byte loads
//      of this batch's B rows (unused slots get an out-of-range offset, which
//      reads zeros without touching memory).  At 128-column tiles the loads
//      go straight into the wave's XOR-swizzled LDS tile (buffer_load ...
//      lds: lane l of load t fetches the chunk the swizzle puts at position
//      l % 16 of tile row 4 t + l / 16); narrower tiles load into registers;
//   5. one batch later (the row loads have long arrived; narrower tiles
//      first write their rows into the tile) reads the tile back with the
//      gfx950 transpose read ds_read_b64_tr_b16 as MFMA B operands and issues
//      one v_mfma_f32_16x16x32_f16 per 16-column tile.
//   Each wave sets its issue priority from the ring passes it has left, so
//   that the workgroups sharing a CU end together (see kBatchPrio).
// A' carries, in MFMA K position k of lane group g (k = 8g .. 8g+7), slot
// kslot(k) = 16 ((k >> 2) & 1) + 4 (k >> 3) + (k & 3); tile row k holds that
// slot's B row.  Columns that are zero in all 16 rows of a block are skipped:
// they add exact zeros.  The waves' partial tiles are summed in LDS.
// grid = (block-rows, ceil(N / 128)); N % 8 == 0 and K * N * 2 <= 2^31.
//
// Per-wave LDS: B tile 32 rows x 256 B (16-byte chunk c of row e stored at
// chunk c ^ swz(e), which spreads the 16 rows one transpose read touches over
// all banks), S^T 16 rows x 80 B (32 halves + pad: conflict-free 16-byte
// reads), slot list 32 x 4 B.
// ---------------------------------------------------------------------------
constexpr int kBtRow = 256;
constexpr int kBtBytes = 32 * kBtRow;
constexpr int kApStride = 80;
constexpr int kApOff = kBtBytes;                     // S^T
constexpr int kSlotOff = kApOff + 16 * kApStride;    // slot list
constexpr int kBatchWaveLds = kSlotOff + 32 * 4;
// each wave's region starts 16-byte aligned (128-bit LDS accesses)
static_assert(kBatchWaveLds % 16 == 0 && kApOff % 16 == 0 && kSlotOff % 16 == 0,
              "batch kernel LDS layout must keep 16-byte alignment");
#ifndef XSPMM_BATCH_WAVES
#define XSPMM_BATCH_WAVES 4
#endif
// Waves per workgroup of the column-batch kernels (count, pack, multiply and
// the packed kernel): they take a block-row's pairs in turn and sum their
// partial tiles in wave order.  The batch kernel is compiled for four
// resident workgroups per CU, i.e. kBW waves per SIMD and 512 / kBW VGPRs.
constexpr int kBW = XSPMM_BATCH_WAVES;
static_assert(kBW >= 2 && kBW <= 4, "2 .. 4 waves per batch workgroup");
#ifndef XSPMM_BATCH_DEPTH
#define XSPMM_BATCH_DEPTH 5
#endif
#ifndef XSPMM_BATCH_DEPTH_NARROW
#define XSPMM_BATCH_DEPTH_NARROW 8
#endif
#ifndef XSPMM_BATCH_MIN_WAVES
#define XSPMM_BATCH_MIN_WAVES 1
#endif
// B rows of a batch go straight from memory into the wave's LDS tile
// (buffer_load ... lds) at 128-column tiles, instead of through 32 VGPRs
// and ds_write_b128 (0 selects the register path)
#ifndef XSPMM_BATCH_DMA
#define XSPMM_BATCH_DMA 1
#endif
constexpr bool kBatchDma = XSPMM_BATCH_DMA != 0;
typedef __attribute__((address_space(3))) void lds_void_t;
#ifndef XSPMM_BATCH_DEPTH_WIDE
#define XSPMM_BATCH_DEPTH_WIDE 10
#endif
// A pairs in flight per wave.  At 128 columns (NT = 8) five fill the 128-VGPR
// budget of four waves per SIMD; narrower tiles need fewer accumulator and B
// registers and keep more pairs in flight.
template <int NT, int NC = 1>
constexpr int batch_depth()
{
    return NC > 1 ? XSPMM_BATCH_DEPTH_WIDE : (NT >= 8 ? XSPMM_BATCH_DEPTH : XSPMM_BATCH_DEPTH_NARROW);
}
// Wave priority by remaining work.  A SIMD issues from its oldest ready wave
// first, so of the four workgroups sharing a CU the one dispatched first runs
// fastest and the last one slowest: on equal block-rows (the templates
// workload) they ended 59.6, 64.8, 71.1 and 77.0 us in dispatch order while
// the CU idled the early finishers' slots.  Each wave sets its priority
// (s_setprio) from the work it has left -- ring passes in the batch kernel,
// batches in the packed kernel: more than T3 gives 3, more than T2 gives 2,
// more than T1 gives 1, else 0 -- so the waves furthest from done issue
// first and the CU's workgroups end close together.  Scheduling only: no
// operand or summation order changes.
#ifndef XSPMM_BATCH_PRIO
#define XSPMM_BATCH_PRIO 1
#endif
#ifndef XSPMM_BATCH_PRIO_T3
#define XSPMM_BATCH_PRIO_T3 12
#endif
#ifndef XSPMM_BATCH_PRIO_T2
#define XSPMM_BATCH_PRIO_T2 6
#endif
#ifndef XSPMM_BATCH_PRIO_T1
#define XSPMM_BATCH_PRIO_T1 2
#endif
#ifndef XSPMM_PACKED_PRIO
#define XSPMM_PACKED_PRIO 1
#endif
#ifndef XSPMM_PACKED_PRIO_T3
#define XSPMM_PACKED_PRIO_T3 8
#endif
#ifndef XSPMM_PACKED_PRIO_T2
#define XSPMM_PACKED_PRIO_T2 4
#endif
#ifndef XSPMM_PACKED_PRIO_T1
#define XSPMM_PACKED_PRIO_T1 2
#endif
constexpr bool kBatchPrio = XSPMM_BATCH_PRIO != 0;
constexpr bool kPackedPrio = XSPMM_PACKED_PRIO != 0;
// the level for `rem` units of work left under thresholds t3 > t2 > t1
__device__ __forceinline__ int prio_level(int64_t rem, int t3, int t2, int t1)
{
    return rem > t3 ? 3 : rem > t2 ? 2 : rem > t1 ? 1 : 0;
}
__device__ __forceinline__ void set_wave_prio(int level)
{
    switch (level) {
    case 3: __builtin_amdgcn_s_setprio(3); break;
    case 2: __builtin_amdgcn_s_setprio(2); break;
    case 1: __builtin_amdgcn_s_setprio(1); break;
    default: __builtin_amdgcn_s_setprio(0); break;
    }
}
static_assert(XSPMM_BATCH_DEPTH >= 4 && XSPMM_BATCH_DEPTH <= 10 && XSPMM_BATCH_DEPTH_NARROW >= 4 &&
                  XSPMM_BATCH_DEPTH_NARROW <= 10 && XSPMM_BATCH_DEPTH_WIDE >= 4 &&
                  XSPMM_BATCH_DEPTH_WIDE <= 10,
              "batch depth must be 4 .. 10 (the ring holds ten pairs)");

// swizzle of row e: even values 0..14, each used by two of the 16 rows a
// transpose read touches
__device__ __forceinline__ uint32_t bt_swz(uint32_t e)
{
    return 2u * ((e & 3u) | (((e >> 3) & 1u) << 2));
}

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t lds_short4_t;

// What the batch kernel does with each batch it forms: multiply it (the
// Tier-1 SpMM), only count it, or store it for spmm_f16_packed_kernel -- the
// wave's A' operand (64 lanes x 16 bytes) and its 32 B-row indices
// (0xffffffff for unused slots), in the order the wave forms them.
enum class BatchMode { kMultiply, kCount, kPack };

struct BatchPack {
    int32_t* counts;          // kCount: batches of (block-row, wave), 4 per row
    const int64_t* offsets;   // kPack: first batch of (block-row, wave)
    u32x4_t* a;               // kPack: A' operands
    uint32_t* rows;           // kPack: B-row indices
};

// Sum the kBW waves' partial 16 x (16 NT) tiles through LDS (in wave order)
// and store C rows: product row r of the block-row goes to C row row_map[r]
// when row_map is given (the un-permutation fused), else to row r.
template <typename I, int NT>
__device__ __forceinline__ void batch_tile_store(const float4_t (&acc)[NT], unsigned char* smem,
                                                 int wave, int g, int li, int64_t br, int64_t n0,
                                                 int64_t M, int64_t N, float* __restrict__ C,
                                                 const I* __restrict__ row_map)
{
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);  // kBW x [16][128] fp32 = kBW x 8 KB
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave * 2048 + (4 * g + r) * 128 + 16 * j + li] = acc[j][r];
    __syncthreads();
    // 256 items of 8 columns (16 rows x 128 columns)
    for (int t = threadIdx.x; t < 256; t += 64 * kBW) {
        const int row = t >> 4;
        const int c0 = (t & 15) * 8;
        const int64_t grow = br * 16 + row;
        if (grow < M && c0 < NT * 16) {
            float out[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int o = row * 128 + c0 + e;
                float v = red[o];
#pragma unroll
                for (int w = 1; w < kBW; ++w) v += red[w * 2048 + o];
                out[e] = v;
            }
            const int64_t crow = row_map ? (int64_t)row_map[grow] : grow;
            float* dst = C + crow * N + n0 + c0;
            if (n0 + c0 + 8 <= N && (N & 3) == 0 && (reinterpret_cast<uintptr_t>(C) & 15) == 0) {
                *reinterpret_cast<float4*>(dst) = make_float4(out[0], out[1], out[2], out[3]);
                *reinterpret_cast<float4*>(dst + 4) = make_float4(out[4], out[5], out[6], out[7]);
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e)
                    if (n0 + c0 + e < N) dst[e] = out[e];
            }
        }
    }
}

typedef __attribute__((address_space(3))) unsigned char lds_u8_t;
// byte address in LDS of a pointer into a __shared__ array, and back
__device__ __forceinline__ uint32_t lds_addr(const void* p)
{
    return (uint32_t)(uintptr_t)(const lds_u8_t*)p;
}
template <typename T>
__device__ __forceinline__ __attribute__((address_space(3))) T* lds_ptr(uint32_t a)
{
    return (__attribute__((address_space(3))) T*)(uintptr_t)a;
}

// batch slot carried in MFMA K position k of an A' operand (lane group
// k >> 3 holds D_0 slots 4g .. 4g+3, then D_1 slots 16 + 4g .. +3)
__device__ __forceinline__ constexpr uint32_t kslot(uint32_t k)
{
    return 16u * ((k >> 2) & 1u) + 4u * (k >> 3) + (k & 3u);
}

// NC: 128-column chunks one workgroup multiplies each batch with (1, or 2
// for N > 128: each pair is streamed and compacted once for 256 columns).
// The chunks' products accumulate exactly as two NC = 1 workgroups would,
// so C does not depend on NC.  With NC = 2 every wave holds the second
// chunk's accumulators, B rows and LDS tile, and two workgroups fit a CU.
// (HIP's second __launch_bounds__ argument is the minimum number of waves per
// SIMD: kBW for four resident workgroups per CU, kBW / 2 for two.)
//
// XM (two 128-column chunks, Mb % 4 == 0, grid (2 Mb, 1)): workgroup l runs
// chunk (l / 4) % 2 of block-row 4 (l / 8) + l % 4, so (workgroups going to
// the 8 XCDs round-robin) XCDs 0-3 take the first chunk and XCDs 4-7 the
// second, and each XCD's L2 holds half of B's columns instead of all of them.
template <typename I, int NT, BatchMode MODE = BatchMode::kMultiply, int NC = 1, bool XM = false>
__global__ __launch_bounds__(64 * kBW, NC == 1 ? kBW : kBW / 2) void spmm_f16_batch_kernel(
    const I* __restrict__ brp, const I* __restrict__ bci, const uint16_t* __restrict__ vals,
    const uint16_t* __restrict__ B, float* __restrict__ C, int64_t M, int64_t K, int64_t N,
    int64_t Kb, const int32_t* __restrict__ order, const I* __restrict__ row_map, BatchPack pk)
{
    static_assert(NT == 1 || NT == 2 || NT == 4 || NT == 8, "NT must be a power of two <= 8");
    static_assert(NC == 1 || (NC == 2 && NT == 8 && MODE == BatchMode::kMultiply),
                  "two chunks per workgroup: 128-column chunks, multiply mode");
    // B rows straight into the LDS tile at 128-column tiles, where one load
    // covers four whole tile rows (narrower tiles use half of each 256-byte
    // row and keep the register path)
    constexpr bool kDma = kBatchDma && NT == 8 && MODE == BatchMode::kMultiply;
    constexpr int D = batch_depth<NT, NC>();
    // per-wave LDS: the first chunk's B tile, S^T, the slot list, then the
    // other chunks' B tiles
    constexpr int kWaveLds = kBatchWaveLds + (NC - 1) * kBtBytes;
    static_assert(4 * D <= kWave, "one index window per ring pass");
    constexpr int CPR = 2 * NT;    // 16-byte chunks per B row
    constexpr int RPL = 64 / CPR;  // B rows per load instruction
    constexpr uint32_t kSel = kApOff;  // S^T: 16 rows x kApStride bytes
    // discard word for slot-list writes of lanes without a column: pad bytes
    // 72..75 of S^T row 0 (reads cover bytes 0..63 of each row)
    constexpr uint32_t kSlotPad = kSel + 72;
    __shared__ __align__(16) unsigned char smem[kBW * kWaveLds];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    unsigned char* const W = smem + wave * kWaveLds;
    // B tile of chunk c
    auto tile = [&](int c) __attribute__((always_inline)) -> unsigned char* {
        return c == 0 ? W : W + kBatchWaveLds + (c - 1) * kBtBytes;
    };

    static_assert(!XM || (NC == 1 && NT == 8 && MODE == BatchMode::kMultiply), "XCD chunk map: two 128-column chunks");
    const uint32_t bx = XM ? (((blockIdx.x >> 3) << 2) | (blockIdx.x & 3u)) : blockIdx.x;
    const uint32_t by = XM ? ((blockIdx.x >> 2) & 1u) : blockIdx.y;
    const uint32_t rows = XM ? (gridDim.x >> 1) : gridDim.x;
    const int64_t br = order ? (int64_t)order[bx] : (int64_t)bx;
    // a caller-supplied order holds a permutation of the block-rows; an id
    // outside the grid is skipped rather than read past row_ptr
    if ((uint64_t)br >= (uint64_t)rows) return;
    const int64_t n0 = (int64_t)by * 128 * NC;
    const int64_t rs = brp[br];
    const int64_t re = brp[br + 1];
    const int64_t npairs = (re - rs + 1) >> 1;

    const int li = lane & 15;
    const int g = lane >> 4;
    const int sel = lane >> 5;
    const int kh = g & 1;

    // A of this row and its block columns: reads past either return zeros
    const uint32_t nblk = (uint32_t)(re - rs);
    const __amdgpu_buffer_rsrc_t a_rsrc = make_rsrc(vals + rs * 256, nblk * 512u);
    const __amdgpu_buffer_rsrc_t c_rsrc = make_rsrc(bci + rs, nblk * (uint32_t)sizeof(I));
    const uint32_t b_bytes = (uint32_t)(K * N * 2);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(B, b_bytes);
    const uint32_t a_voff = (uint32_t)(sel * 512 + li * 32 + kh * 16);
    const uint32_t kb32 = (uint32_t)Kb;
    const uint32_t k32 = (uint32_t)K;
    const uint32_t rowbytes = (uint32_t)(2 * N);
    // index window of one ring pass (pairs q, q + kBW, ..., q + kBW (depth - 1)
    // of this wave): lane l holds dword l of their block columns in order,
    // so pair j's columns sit in lanes 2j, 2j + 1 (int64: 4j .. 4j + 3)
    const uint32_t cw_off = sizeof(I) == 4
                                ? 8u * kBW * (uint32_t)(lane >> 1) + 4u * (uint32_t)(lane & 1)
                                : 16u * kBW * (uint32_t)(lane >> 2) +
                                      8u * (uint32_t)((lane >> 1) & 1) + 4u * (uint32_t)(lane & 1);

    // --- per-lane constants --------------------------------------------------
    // Pair mask layout: lane (r, g)'s non-zero halves 2d go to bit 4g + d and
    // halves 2d + 1 to bit 16 + 4g + d, so the four groups never overlap.
    // Column lane (i < 8, g) stands for bit 16 (i >> 2) + 4g + (i & 3), i.e.
    // half e = 2 (i & 3) + (i >> 2) of group g (pair column 8g + e); the other
    // lanes never match a bit.
    const int ce = 2 * (li & 3) + ((li >> 2) & 1);
    const uint32_t bitk = li < 8 ? 1u << (16 * ((li >> 2) & 1) + 4 * g + (li & 3)) : 0u;
    // its S^T entry: row (slot & 15), half 8g + e; lanes without a column
    // write to pad bytes 64.. of S^T row li, which no read covers
    // (LDS byte addresses, kept in VGPRs so that each access costs one
    // address instruction)
    uint32_t st_k = lds_addr(W + kSel + 2 * (8 * g + ce));
    uint32_t st_pad = lds_addr(W + kSel + li * kApStride + 64 + 2 * g);
    uint32_t slot_w = lds_addr(W + kSlotOff);
    uint32_t slot_pad = lds_addr(W + kSlotPad);
    // ds_bpermute address of this lane's block column in the index window
    // (pair j adds 8 j, int64: 16 j)
    const uint32_t csel_addr = 4u * (uint32_t)sel * (uint32_t)(sizeof(I) / 4);
    // its B row: 16 * (block column of block sel) + 8 kh + e
    const uint32_t row_k = (uint32_t)(8 * kh + ce);
    // selection lanes: S^T row li, halves 8g .. 8g+7
    uint32_t st_rd = lds_addr(W + kSel + li * kApStride + 16 * g);
    asm volatile("" : "+v"(st_k), "+v"(st_pad), "+v"(slot_w), "+v"(slot_pad), "+v"(st_rd));
    const uint32_t gshift = (uint32_t)(4 * g);
    // B row loads: load t moves tile row t * RPL + lane / CPR, chunk lane % CPR
    const uint32_t ld_c = (uint32_t)(lane % CPR);
    const uint32_t ld_r = (uint32_t)(lane / CPR);
    const uint32_t ld_off = (uint32_t)(2 * n0) + 16u * ld_c;
    const uint32_t tr_e0 = (uint32_t)(8 * g + (li >> 2));
    const uint32_t tr_base = tr_e0 * kBtRow + 16u * ((li & 3) >> 1) + 8u * (li & 1);
    const uint32_t tr_a0 = tr_base ^ (bt_swz(tr_e0) << 4);
    // slot of tile row t * RPL + ld_r is kslot(t * RPL) + ks_r (RPL is 4 or a
    // multiple of 8)
    const int ks_r = (int)kslot(ld_r);
    uint32_t one;
    asm("s_mov_b32 %0, 0x10001" : "=s"(one));

    // S^T starts all zero and every pair leaves it so
    for (int i = lane; i < 16 * kApStride / 4; i += kWave)
        reinterpret_cast<uint32_t*>(W + kSel)[i] = 0u;

    float4_t acc[NC][NT];
#pragma unroll
    for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[c][j] = float4_t{0.f, 0.f, 0.f, 0.f};
    float4_t d0 = float4_t{0.f, 0.f, 0.f, 0.f};  // A' slots 0..15 (transposed)
    float4_t d1 = float4_t{0.f, 0.f, 0.f, 0.f};  // A' slots 16..31

    u32x4_t bv[NC][NT];
    half8_t aop{};
    bool started = false;
    uint32_t pending = 0;

    auto finish = [&]() __attribute__((always_inline)) {
#pragma unroll
        for (int c = 0; c < NC; ++c) {
            unsigned char* const T = tile(c);
            if constexpr (!kDma) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const uint32_t e = (uint32_t)(t * RPL) + ld_r;
                    *reinterpret_cast<u32x4_t*>(T + e * kBtRow + ((ld_c ^ bt_swz(e)) << 4)) = bv[c][t];
                }
            }
            // read address of tile j: tr_a0 ^ 32 j (the swizzle XORs bits
            // 5..7, which tr_base leaves clear); recomputed here rather than
            // kept live
            uint32_t a0 = tr_a0;
            asm volatile("" : "+v"(a0));
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const uint32_t a = a0 ^ (uint32_t)(32 * j);
                const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(T + a));
                const short4_t hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(T + a + 4 * kBtRow));
                const half8_t bop = __builtin_bit_cast(
                    half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[c][j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, acc[c][j], 0, 0, 0);
            }
        }
    };
    int64_t nbatch = 0;
    int64_t pbase = 0;
    if constexpr (MODE == BatchMode::kPack) pbase = pk.offsets[br * kBW + wave];
    // Close the open batch of `cnt` slots: A' from the D registers (exact
    // fp16 values), then multiply the previous batch and issue this one's
    // B row loads in K order.
    auto start = [&](uint32_t cnt) __attribute__((always_inline)) {
        if constexpr (MODE == BatchMode::kCount) {
            ++nbatch;
            return;
        }
        const half8_t a = half8_t{(_Float16)d0[0], (_Float16)d0[1], (_Float16)d0[2], (_Float16)d0[3],
                                  (_Float16)d1[0], (_Float16)d1[1], (_Float16)d1[2], (_Float16)d1[3]};
        d0 = float4_t{0.f, 0.f, 0.f, 0.f};
        d1 = float4_t{0.f, 0.f, 0.f, 0.f};
        if constexpr (MODE == BatchMode::kPack) {
            const int64_t bi = pbase + nbatch;
            pk.a[bi * 64 + lane] = __builtin_bit_cast(u32x4_t, a);
            if (lane < 32) {
                const uint32_t s = kslot((uint32_t)lane);
                const uint32_t r = *reinterpret_cast<const uint32_t*>(W + kSlotOff + 4u * s);
                pk.rows[bi * 32 + lane] = s < cnt ? r : 0xffffffffu;
            }
            ++nbatch;
            return;
        }
        if (started) finish();
        aop = a;
        uint32_t row[NT];
#pragma unroll
        for (int t = 0; t < NT; ++t)
            row[t] = *reinterpret_cast<const uint32_t*>(
                W + kSlotOff + 4u * ((uint32_t)ks_r + kslot((uint32_t)(t * RPL))));
        // the tile's transposed reads (finish) complete before loads rewrite it
        if constexpr (kDma) asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
#pragma unroll
        for (int c = 0; c < NC; ++c)
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const bool use = (ks_r < (int)cnt - (int)kslot((uint32_t)(t * RPL))) & (row[t] < k32);
                if constexpr (kDma) {
                    // load t fills tile bytes [1024 t, 1024 t + 1024) lane by
                    // lane: lane l writes position l % 16 of tile row
                    // 4 t + l / 16, which holds chunk position ^ swizzle
                    const uint32_t e = (uint32_t)(t * RPL) + ld_r;
                    const uint32_t at = __umul24(row[t], rowbytes) + (uint32_t)(2 * n0) +
                                        16u * (ld_c ^ bt_swz(e)) + 256u * (uint32_t)c;
                    const uint32_t off = use ? at : b_bytes + ld_off;
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(b_rsrc, (lds_void_t*)(tile(c) + t * 1024),
                                                             16, (int)off, 0, 0, 0);
                } else {
                    // chunk c starts 128 columns (256 bytes) after chunk c - 1
                    const uint32_t at = __umul24(row[t], rowbytes) + ld_off + 256u * (uint32_t)c;
                    const uint32_t off = use ? at : b_bytes + ld_off;
                    bv[c][t] = __builtin_bit_cast(
                        u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)off, 0, 0));
                }
            }
        started = true;
    };

    auto stage_a = [&](int64_t q, half8_t& P) __attribute__((always_inline)) {
        P = __builtin_bit_cast(half8_t, __builtin_amdgcn_raw_buffer_load_b128(
                                            a_rsrc, (int)(a_voff + (uint32_t)q * 1024u), 0, kNonTemporal));
    };
    auto load_cols = [&](int64_t q) __attribute__((always_inline)) -> uint32_t {
        return (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
            c_rsrc, (int)(cw_off + (uint32_t)q * (uint32_t)(2 * sizeof(I))), 0, 0);
    };

    // One compaction MFMA into D_h: column lanes in `mine` (slots 16h ..
    // 16h+15) set their S^T entry before the read and clear it after; the
    // other lanes write to the pad bytes of their S^T row, which no read sees.
    const uint16_t h_one = 0x3c00u;  // fp16 1.0
    auto round = [&](float4_t& d, bool mine, uint32_t st, const half8_t& pa) __attribute__((always_inline)) {
        const uint32_t at = mine ? st : st_pad;
        *lds_ptr<uint16_t>(at) = h_one;
        const half8_t x = __builtin_bit_cast(half8_t, *lds_ptr<const u32x4_t>(st_rd));
        d = __builtin_amdgcn_mfma_f32_16x16x32_f16(x, pa, d, 0, 0, 0);
        *lds_ptr<uint16_t>(at) = (uint16_t)0u;
    };

    // pair j of the ring pass whose index window is `win`
    auto process = [&](const half8_t& pa, uint32_t win, int j) __attribute__((always_inline)) {
        uint32_t c0, c1;
        // this lane's block column (lane l: block l >> 5 of the pair)
        uint32_t csel;
        if constexpr (sizeof(I) == 4) {
            c0 = (uint32_t)__builtin_amdgcn_readlane((int)win, 2 * j);
            c1 = (uint32_t)__builtin_amdgcn_readlane((int)win, 2 * j + 1);
            csel = (uint32_t)__builtin_amdgcn_ds_bpermute((int)(csel_addr + 8u * (uint32_t)j), (int)win);
        } else {
            const uint32_t l0 = (uint32_t)__builtin_amdgcn_readlane((int)win, 4 * j);
            const uint32_t h0 = (uint32_t)__builtin_amdgcn_readlane((int)win, 4 * j + 1);
            const uint32_t l1 = (uint32_t)__builtin_amdgcn_readlane((int)win, 4 * j + 2);
            const uint32_t h1 = (uint32_t)__builtin_amdgcn_readlane((int)win, 4 * j + 3);
            c0 = h0 == 0u ? l0 : 0xffffffffu;
            c1 = h1 == 0u ? l1 : 0xffffffffu;
            // the low dword is enough: a set bit implies a valid column
            csel = (uint32_t)__builtin_amdgcn_ds_bpermute((int)(csel_addr + 16u * (uint32_t)j), (int)win);
        }
        const u32x4_t w = __builtin_bit_cast(u32x4_t, pa);
        uint32_t nz[4];
#pragma unroll
        for (int d = 0; d < 4; ++d) {
            const uint32_t x = w[d];
            nz[d] = __builtin_bit_cast(
                uint32_t, __builtin_elementwise_min(__builtin_bit_cast(ushort2_t, x),
                                                    __builtin_bit_cast(ushort2_t, one)));
        }
        uint32_t v = (nz[0] | (nz[1] << 1) | (nz[2] << 2) | (nz[3] << 3)) << gshift;
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x121, 0xf, 0xf, false);
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x122, 0xf, 0xf, false);
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x124, 0xf, 0xf, false);
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x128, 0xf, 0xf, false);
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xa, 0xf, false);
        v |= (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xc, 0xf, false);
        // block 0 owns groups 0 and 1 (bits 0..7, 16..23), block 1 the rest; a
        // block column outside the grid (malformed input) contributes nothing
        const uint32_t valid = (c0 < kb32 ? 0x00ff00ffu : 0u) | (c1 < kb32 ? 0xff00ff00u : 0u);
        const uint32_t pm = (uint32_t)__builtin_amdgcn_readlane((int)v, 63) & valid;
        if (pm == 0u) return;
        const uint32_t cnt = (uint32_t)__builtin_popcount(pm);
        if (pending + cnt > 32u) {
            start(pending);
            pending = 0;
        }
        if constexpr (MODE != BatchMode::kCount) {
            const bool set = (pm & bitk) != 0u;
            const uint32_t rank = (uint32_t)__builtin_popcount(pm & (bitk - 1u)) + pending;
            *lds_ptr<uint32_t>(set ? slot_w + 4u * rank : slot_pad) = 16u * csel + row_k;
            const uint32_t st = st_k + (rank & 15u) * (uint32_t)kApStride;
            const bool lo = rank < 16u;
            if (pending < 16u) round(d0, set & lo, st, pa);
            if (pending + cnt > 16u) round(d1, set & !lo, st, pa);
        }
        pending += cnt;
    };

    if (wave < npairs) {
        half8_t P0, P1, P2, P3, P4, P5, P6, P7, P8, P9;
        constexpr int S = kBW;
        constexpr int A = S * D;
        const int64_t q0 = wave;
        // the window before the A loads, as in every later pass, so the
        // loads complete in the same order on the first pass
        uint32_t win = load_cols(q0);
        stage_a(q0, P0);
        stage_a(q0 + S, P1);
        stage_a(q0 + 2 * S, P2);
        stage_a(q0 + 3 * S, P3);
        if constexpr (D > 4) stage_a(q0 + 4 * S, P4);
        if constexpr (D > 5) stage_a(q0 + 5 * S, P5);
        if constexpr (D > 6) stage_a(q0 + 6 * S, P6);
        if constexpr (D > 7) stage_a(q0 + 7 * S, P7);
        if constexpr (D > 8) stage_a(q0 + 8 * S, P8);
        if constexpr (D > 9) stage_a(q0 + 9 * S, P9);
        // this wave's ring passes
        const int64_t passes = ((npairs - q0 + S - 1) / S + D - 1) / D;
        int64_t pass = 0;
        int level = -1;
        for (int64_t q = q0; q < npairs; q += A) {
            if constexpr (kBatchPrio) {
                const int lv = prio_level(passes - pass, XSPMM_BATCH_PRIO_T3, XSPMM_BATCH_PRIO_T2,
                                          XSPMM_BATCH_PRIO_T1);
                if (lv != level) {
                    level = lv;
                    set_wave_prio(lv);
                }
                ++pass;
            }
            // next pass's window, issued a pass ahead like the A loads
            const uint32_t nwin = load_cols(q + A);
            process(P0, win, 0);
            stage_a(q + A, P0);
            process(P1, win, 1);
            stage_a(q + A + S, P1);
            process(P2, win, 2);
            stage_a(q + A + 2 * S, P2);
            process(P3, win, 3);
            stage_a(q + A + 3 * S, P3);
            if constexpr (D > 4) {
                process(P4, win, 4);
                stage_a(q + A + 4 * S, P4);
            }
            if constexpr (D > 5) {
                process(P5, win, 5);
                stage_a(q + A + 5 * S, P5);
            }
            if constexpr (D > 6) {
                process(P6, win, 6);
                stage_a(q + A + 6 * S, P6);
            }
            if constexpr (D > 7) {
                process(P7, win, 7);
                stage_a(q + A + 7 * S, P7);
            }
            if constexpr (D > 8) {
                process(P8, win, 8);
                stage_a(q + A + 8 * S, P8);
            }
            if constexpr (D > 9) {
                process(P9, win, 9);
                stage_a(q + A + 9 * S, P9);
            }
            win = nwin;
        }
        if (pending > 0u) start(pending);
        if constexpr (MODE == BatchMode::kMultiply) {
            if (started) finish();
        }
    }
    if constexpr (MODE == BatchMode::kCount) {
        if (lane == 0) pk.counts[br * kBW + wave] = (int32_t)nbatch;
        return;
    } else if constexpr (MODE == BatchMode::kPack) {
        return;
    } else {
#pragma unroll
        for (int c = 0; c < NC; ++c)
            if (n0 + 128 * c < N)
                batch_tile_store<I, NT>(acc[c], smem, wave, g, li, br, n0 + 128 * c, M, N, C,
                                        row_map);
    }
}

// ---------------------------------------------------------------------------
// Multiply packed column batches (written by the batch kernel in pack mode).
// Wave w of the workgroup of block-row br multiplies the batches
// [offsets[4 br + w], offsets[4 br + w + 1]) in order: the stored A' operand,
// the B rows of the stored slot indices (unused slots read zeros), and the
// batch kernel's own multiply step and store -- the same MFMA operands in the
// same order, so C equals the batch kernel's C.  While a batch multiplies,
// the next batch's B rows are in flight and the indices of the one after
// are loading.  LDS holds only the B tile of each wave (8 KB).  grid = (block-rows, ceil(N / 128)); N % 8 == 0, K * N * 2 <= 2^31.
// ---------------------------------------------------------------------------
template <typename I, int NT>
__global__ __launch_bounds__(64 * kBW, XSPMM_BATCH_MIN_WAVES) void spmm_f16_packed_kernel(
    const int64_t* __restrict__ offsets, const u32x4_t* __restrict__ pa,
    const uint32_t* __restrict__ prow, const uint16_t* __restrict__ B, float* __restrict__ C,
    int64_t M, int64_t K, int64_t N, const int32_t* __restrict__ order, const I* __restrict__ row_map)
{
    static_assert(NT == 1 || NT == 2 || NT == 4 || NT == 8, "NT must be a power of two <= 8");
    constexpr int CPR = 2 * NT;    // 16-byte chunks per B row
    constexpr int RPL = 64 / CPR;  // B rows per load instruction
    __shared__ __align__(16) unsigned char smem[kBW * kBtBytes];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
    unsigned char* const W = smem + wave * kBtBytes;
    const int64_t br = order ? (int64_t)order[blockIdx.x] : (int64_t)blockIdx.x;
    // a caller-supplied order holds a permutation of the block-rows; an id
    // outside the grid is skipped rather than read past row_ptr
    if ((uint64_t)br >= (uint64_t)gridDim.x) return;
    const int64_t n0 = (int64_t)blockIdx.y * 128;
    const int li = lane & 15;
    const int g = lane >> 4;

    const uint32_t b_bytes = (uint32_t)(K * N * 2);
    const __amdgpu_buffer_rsrc_t b_rsrc = make_rsrc(B, b_bytes);
    const uint32_t k32 = (uint32_t)K;
    const uint32_t rowbytes = (uint32_t)(2 * N);
    const uint32_t ld_c = (uint32_t)(lane % CPR);
    const uint32_t ld_r = (uint32_t)(lane / CPR);
    const uint32_t ld_off = (uint32_t)(2 * n0) + 16u * ld_c;
    const uint32_t tr_e0 = (uint32_t)(8 * g + (li >> 2));
    const uint32_t tr_base = tr_e0 * kBtRow + 16u * ((li & 3) >> 1) + 8u * (li & 1);
    const uint32_t tr_swz16 = bt_swz(tr_e0) << 4;

    float4_t acc[NT];
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

    const int64_t b0 = offsets[br * kBW + wave];
    const int nb = (int)(offsets[br * kBW + wave + 1] - b0);
    if (nb > 0) {
        const u32x4_t* pa_w = pa + b0 * 64 + lane;
        const uint32_t* pr_w = prow + b0 * 32 + ld_r;
        u32x4_t bv[NT];
        uint32_t row[NT];
        u32x4_t a_cur = pa_w[0];
#pragma unroll
        for (int t = 0; t < NT; ++t) {
            const uint32_t r = pr_w[t * RPL];
            const uint32_t off = r < k32 ? __umul24(r, rowbytes) + ld_off : b_bytes + ld_off;
            bv[t] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)off, 0, 0));
        }
        {
            const int nx = nb > 1 ? 1 : 0;
#pragma unroll
            for (int t = 0; t < NT; ++t) row[t] = pr_w[nx * 32 + t * RPL];
        }
        int level = -1;
        for (int bi = 0; bi < nb; ++bi) {
            if constexpr (kPackedPrio) {
                const int lv = prio_level(nb - bi, XSPMM_PACKED_PRIO_T3, XSPMM_PACKED_PRIO_T2,
                                          XSPMM_PACKED_PRIO_T1);
                if (lv != level) {
                    level = lv;
                    set_wave_prio(lv);
                }
            }
            const bool more = bi + 1 < nb;
#pragma unroll
            for (int t = 0; t < NT; ++t) {
                const uint32_t e = (uint32_t)(t * RPL) + ld_r;
                *reinterpret_cast<u32x4_t*>(W + e * kBtRow + ((ld_c ^ bt_swz(e)) << 4)) = bv[t];
            }
            const half8_t aop = __builtin_bit_cast(half8_t, a_cur);
            if (more) {
#pragma unroll
                for (int t = 0; t < NT; ++t) {
                    const uint32_t off = row[t] < k32 ? __umul24(row[t], rowbytes) + ld_off : b_bytes + ld_off;
                    bv[t] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(b_rsrc, (int)off, 0, 0));
                }
            }
            const int n2 = bi + 2 < nb ? bi + 2 : (more ? bi + 1 : bi);
#pragma unroll
            for (int t = 0; t < NT; ++t) row[t] = pr_w[n2 * 32 + t * RPL];
#pragma unroll
            for (int j = 0; j < NT; ++j) {
                const uint32_t a = tr_base + ((uint32_t)(32 * j) ^ tr_swz16);
                const short4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(W + a));
                const short4_t hi =
                    __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_t*)(W + a + 4 * kBtRow));
                const half8_t bop = __builtin_bit_cast(
                    half8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(aop, bop, acc[j], 0, 0, 0);
            }
            a_cur = pa_w[(more ? bi + 1 : bi) * 64];
        }
    }
    batch_tile_store<I, NT>(acc, smem, wave, g, li, br, n0, M, N, C, row_map);
}

// ---------------------------------------------------------------------------
// Dispatch orders of the column-batch kernels (block-row ids by workgroup id).
// Only scheduling changes: each row's result is computed exactly as before.
//   * more than kOrderMinRows block-rows (skewed rows trail a long grid): one
//     1024-thread workgroup buckets the block-rows by the bit length of their
//     block count and writes the row ids longest bucket first; workgroups are
//     dispatched in id order, so long rows start first;
//   * kXcdOrderMinRows .. kOrderMinRows block-rows, for an order computed
//     once per matrix (spmm_dispatch_order_cols): when the block-rows are
//     short (at most kXcdOrderMaxAvg blocks on average) and neighbouring
//     block-rows are alike (their middle block columns differ by at most
//     max(2, length / 8) for at least half of 256 sampled pairs), each XCD
//     takes a contiguous range of block-rows: workgroups go to the 8 XCDs
//     round-robin by id, so workgroup i takes row start[i % 8] + i / 8,
//     where XCD x's range starts at start[x].  The B rows the neighbours
//     share then stay in one XCD's L2 instead of being fetched by all eight
//     (banded matrices at 0.5-5 %: 6-25 % faster).  Otherwise the order is
//     the identity: long rows (a 90 % band ran 18 % slower with the XCD
//     ranges) and unrelated neighbours (random dense blocks) gain nothing.
// ---------------------------------------------------------------------------
constexpr int kOrderThreads = 1024;
#ifndef XSPMM_ORDER_MIN_ROWS
#define XSPMM_ORDER_MIN_ROWS 2048
#endif
constexpr int64_t kOrderMinRows = XSPMM_ORDER_MIN_ROWS;
constexpr int64_t kXcdOrderMinRows = 256;
constexpr int64_t kXcdOrderMaxAvg = 128;
constexpr int kXcds = 8;
constexpr int kOrderBuckets = 33;

template <typename I>
__global__ __launch_bounds__(kOrderThreads) void order_rows_kernel(const I* __restrict__ brp,
                                                                   int64_t Mb,
                                                                   int32_t* __restrict__ order)
{
    __shared__ uint32_t count[kOrderBuckets];
    __shared__ uint32_t next[kOrderBuckets];
    const int t = threadIdx.x;
    if (t < kOrderBuckets) count[t] = 0u;
    __syncthreads();
    auto bucket = [&](int64_t r) -> int {
        const int64_t len = (int64_t)brp[r + 1] - (int64_t)brp[r];
        const uint64_t u = len > 0 ? (uint64_t)len : 0u;
        const int bits = u ? 64 - __builtin_clzll(u) : 0;  // 0..33
        return bits > 32 ? 32 : bits;
    };
    for (int64_t r = t; r < Mb; r += kOrderThreads) atomicAdd(&count[bucket(r)], 1u);
    __syncthreads();
    if (t == 0) {
        uint32_t run = 0;
        for (int b = kOrderBuckets - 1; b >= 0; --b) {  // longest bucket first
            next[b] = run;
            run += count[b];
        }
    }
    __syncthreads();
    for (int64_t r = t; r < Mb; r += kOrderThreads) {
        const uint32_t pos = atomicAdd(&next[bucket(r)], 1u);
        order[pos] = (int32_t)r;
    }
}

// one 256-thread workgroup: the decision above, then order[i] for i < Mb,
// and order[Mb] = 1 for the XCD ranges, 0 for the identity
template <typename I>
__global__ __launch_bounds__(256) void order_local_kernel(const I* __restrict__ brp, const I* __restrict__ bci,
                                                          int64_t Mb, int32_t* __restrict__ order)
{
    __shared__ int s_alike;
    const int t = threadIdx.x;
    if (t == 0) s_alike = 0;
    __syncthreads();
    const int64_t nnzb = (int64_t)brp[Mb] - (int64_t)brp[0];
    if (Mb > 1 && nnzb <= kXcdOrderMaxAvg * Mb) {
        const int64_t r = (int64_t)t * (Mb - 1) / 256;  // pair (r, r + 1)
        const int64_t a0 = brp[r], a1 = brp[r + 1], a2 = brp[r + 2];
        const int64_t l0 = a1 - a0, l1 = a2 - a1;
        if (l0 > 0 && l1 > 0) {
            const int64_t m0 = (int64_t)bci[a0 + l0 / 2], m1 = (int64_t)bci[a1 + l1 / 2];
            const int64_t d = m1 > m0 ? m1 - m0 : m0 - m1;
            const int64_t lim = l0 / 8 > 2 ? l0 / 8 : 2;
            if (d <= lim) atomicAdd(&s_alike, 1);
        }
    }
    __syncthreads();
    const bool xcd = s_alike >= 128;
    for (int64_t i = t; i < Mb; i += 256) {
        int64_t br = i;
        if (xcd) {
            const int64_t x = i % kXcds;
            int64_t start = 0;
            for (int64_t y = 0; y < x; ++y) start += (Mb - y + kXcds - 1) / kXcds;
            br = start + i / kXcds;
        }
        order[i] = (int32_t)br;
    }
    if (t == 0) order[Mb] = xcd ? 1 : 0;
}

// ---------------------------------------------------------------------------
// fp32 x fp32 -> fp32 tile kernel.
//
// A workgroup of kF32Waves waves owns one block-row and NTW 16-column tiles
// (up to 64 columns; the launcher narrows NTW when the grid would have fewer
// than 512 workgroups).  The waves split the row's blocks (wave w: blocks
// w, w + kF32Waves, ...), f32_unroll(NTW) blocks per step with all their
// loads issued before the MFMAs (v_mfma_f32_16x16x4_f32, four per block and
// tile; a step past the row's end loads the row's last block again and does
// not multiply it, so a wave's last blocks need no step of their own), and
// their partial tiles are summed through LDS in wave order.  Splitting the
// row keeps short rows' dependent load chains short: a small matrix has few
// block-rows, and one wave per row would leave the chip idle.
// ---------------------------------------------------------------------------
constexpr int kF32Waves = 8;
// blocks per wave whose loads are in flight together: 8 at one tile (64
// VGPRs of operands), fewer at wider tiles
constexpr int f32_unroll(int ntw) { return ntw == 1 ? 8 : (ntw == 2 ? 4 : 2); }

template <typename I, int NTW>
__global__ __launch_bounds__(64 * kF32Waves) void spmm_f32_kernel(const I* __restrict__ brp,
                                                                  const I* __restrict__ bci,
                                                                  const float* __restrict__ vals,
                                                                  const float* __restrict__ B,
                                                                  float* __restrict__ C, int64_t M,
                                                                  int64_t K, int64_t N, int ntiles)
{
    __shared__ float red[kF32Waves][16][NTW * 16];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int tile0 = blockIdx.y * NTW;
    const int64_t br = blockIdx.x;
    const int64_t rs = brp[br];
    const int64_t re = brp[br + 1];
    const int li = lane & 15;
    const int g = lane >> 4;

    float4_t acc[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

    auto b_panel = [&](int64_t col, float (&bv)[NTW][4]) {
        const int64_t kbase = (col >= 0 ? col : K) * 16 + g * 4;  // invalid columns read nothing
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            const int64_t n = (int64_t)(tile0 + j) * 16 + li;
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int64_t k = kbase + s;
                bv[j][s] = (k >= 0 && k < K && n < N) ? B[k * N + n] : 0.f;
            }
        }
    };
    auto multiply = [&](const float4_t& a, const float (&bv)[NTW][4]) {
#pragma unroll
        for (int j = 0; j < NTW; ++j)
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], bv[j][s], acc[j], 0, 0, 0);
    };

    // the wave's blocks rs + wave + 8 i in ascending order, U at a time:
    // all their loads first, then their MFMAs (blocks past the row's end
    // load the last block and are not multiplied: the order of the MFMAs
    // is the blocks' order)
    constexpr int U = f32_unroll(NTW);
    for (int64_t blk = rs + wave; blk < re; blk += (int64_t)U * kF32Waves) {
        float4_t a[U];
        float bv[U][NTW][4];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t b0 = blk + u * kF32Waves;
            const int64_t b = b0 < re ? b0 : re - 1;
            a[u] = *reinterpret_cast<const float4_t*>(vals + b * 256 + li * 16 + g * 4);
            b_panel((int64_t)bci[b], bv[u]);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (blk + u * kF32Waves < re) multiply(a[u], bv[u]);
    }

#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][4 * g + r][16 * j + li] = acc[j][r];
    __syncthreads();
    for (int o = threadIdx.x; o < 16 * NTW * 16; o += 64 * kF32Waves) {
        const int row = o / (NTW * 16), c = o % (NTW * 16);
        float sum = red[0][row][c];
#pragma unroll
        for (int w = 1; w < kF32Waves; ++w) sum += red[w][row][c];
        const int64_t grow = br * 16 + row;
        const int64_t col = (int64_t)tile0 * 16 + c;
        if (grow < M && col < N && tile0 + c / 16 < ntiles) C[grow * N + col] = sum;
    }
}

// ---------------------------------------------------------------------------
// fp32 short-grid kernel where B's byte offsets fit 30 bits (16 * Kb * N * 4
// <= 2^30): the tile kernel's product with B read through a buffer resource.
// A lane's B offset within a block's 16 rows is fixed for the kernel, so each
// B load is one add and one buffer load; an offset past the end of B (rows
// >= K, columns >= N, invalid block columns) reads zero, so no load needs a
// branch of its own and every step issues the same loads.  Sixteen waves
// split a block-row's blocks (wave w: blocks w, w + 16, ...), four blocks'
// loads in flight per wave; the partial tiles are summed through LDS in wave
// order.  Every block column multiplies, as in the tile kernel: a non-finite
// B row makes NaN wherever it meets a block.
// ---------------------------------------------------------------------------
constexpr int kF32ShortWaves = 16;
constexpr int kF32ShortUnroll = 4;
// an offset part past every in-range offset: in-range parts are below 2^30,
// so a sum with one or two of these parts stays below 2^32 and past the end
constexpr uint32_t kF32ShortPast = 1u << 30;
constexpr int64_t kF32ShortMaxBytes = int64_t(1) << 30;

template <typename I, int NTW>
__global__ __launch_bounds__(64 * kF32ShortWaves) void spmm_f32_short_kernel(
    const I* __restrict__ brp, const I* __restrict__ bci, const float* __restrict__ vals,
    const float* __restrict__ B, float* __restrict__ C, int64_t M, int64_t K, int64_t N, int64_t Kb,
    int ntiles)
{
    constexpr int W = kF32ShortWaves;
    constexpr int U = kF32ShortUnroll;
    __shared__ float red[W][16][NTW * 16];
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int li = lane & 15;
    const int g = lane >> 4;
    const int tile0 = blockIdx.y * NTW;
    const int64_t br = blockIdx.x;
    const int64_t rs = brp[br];
    const int64_t re = brp[br + 1];
    const __amdgpu_buffer_rsrc_t rb = make_rsrc(B, (uint32_t)(K * N * 4));
    // byte offset of lane (li, g)'s B element at step s, tile t, from the
    // block's first B row
    uint32_t loff[NTW][4];
#pragma unroll
    for (int t = 0; t < NTW; ++t)
#pragma unroll
        for (int s = 0; s < 4; ++s) {
            const int64_t n = (int64_t)(tile0 + t) * 16 + li;
            loff[t][s] = n < N ? (uint32_t)(((4 * g + s) * N + n) * 4) : kF32ShortPast;
        }
    const uint32_t rowbytes = (uint32_t)(16 * N * 4);

    float4_t acc[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

    // U blocks per step, loads first; a block past the row's end loads the
    // row's last block again and is not multiplied
    for (int64_t blk = rs + wave; blk < re; blk += (int64_t)U * W) {
        float4_t a[U];
        uint32_t base[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int64_t b0 = blk + u * W;
            const int64_t b = b0 < re ? b0 : re - 1;
            a[u] = *reinterpret_cast<const float4_t*>(vals + b * 256 + li * 16 + g * 4);
            const int64_t col = (int64_t)bci[b];
            base[u] = (col >= 0 && col < Kb) ? (uint32_t)col * rowbytes : kF32ShortPast;
        }
        float bv[U][4][NTW];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int s = 0; s < 4; ++s)
#pragma unroll
                for (int t = 0; t < NTW; ++t)
                    bv[u][s][t] = __builtin_bit_cast(
                        float, (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
                                   rb, (int)(base[u] + loff[t][s]), 0, 0));
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (blk + u * W < re) {
#pragma unroll
                for (int s = 0; s < 4; ++s)
#pragma unroll
                    for (int t = 0; t < NTW; ++t)
                        acc[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u][s], bv[u][s][t], acc[t],
                                                                       0, 0, 0);
            }
    }

#pragma unroll
    for (int j = 0; j < NTW; ++j)
#pragma unroll
        for (int r = 0; r < 4; ++r) red[wave][4 * g + r][16 * j + li] = acc[j][r];
    __syncthreads();
    for (int o = threadIdx.x; o < 16 * NTW * 16; o += 64 * W) {
        const int row = o / (NTW * 16), c = o % (NTW * 16);
        float sum = red[0][row][c];
#pragma unroll
        for (int w = 1; w < W; ++w) sum += red[w][row][c];
        const int64_t grow = br * 16 + row;
        const int64_t col = (int64_t)tile0 * 16 + c;
        if (grow < M && col < N && tile0 + c / 16 < ntiles) C[grow * N + col] = sum;
    }
}

// Whether the fp32 short-grid product takes spmm_f32_short_kernel: B's
// offsets fit its 30-bit range, unless XSPMM_F32_SHORT=off (read on every
// call, so a process can compare the two kernels).
bool f32_short_wanted(int64_t Kb, int64_t N)
{
    const char* e = std::getenv("XSPMM_F32_SHORT");
    if (e && std::string(e) == "off") return false;
    return N > 0 && N <= kF32ShortMaxBytes / 64 && Kb <= kF32ShortMaxBytes / (64 * N);
}

// Launch geometry: waves per workgroup and 16-column tiles per wave.
struct Geometry {
    int ntw;
    int waves;
    int grid_y;
};

Geometry pick_geometry(int ntiles)
{
    Geometry g;
    g.ntw = ntiles >= 16 ? 4 : (ntiles >= 8 ? 2 : 1);
    const int groups = (ntiles + g.ntw - 1) / g.ntw;
    g.waves = groups < 4 ? groups : 4;
    g.grid_y = (groups + g.waves - 1) / g.waves;
    return g;
}

// fp16 kernel family: "batch" (column batches, default where N % 8 == 0),
// "gather" (per-pair masked B-row gather) or "panel" (whole 16-row B panels
// from a repacked copy of B; any N).  XSPMM_SPMM_KERNEL=batch|gather|panel
// forces one where its shape conditions hold.
enum class Fp16Kernel { kAuto, kBatch, kGather, kPanel };

Fp16Kernel fp16_kernel_choice()
{
    static const Fp16Kernel k = [] {
        const char* e = std::getenv("XSPMM_SPMM_KERNEL");
        if (!e) return Fp16Kernel::kAuto;
        const std::string v(e);
        if (v == "panel") return Fp16Kernel::kPanel;
        if (v == "gather") return Fp16Kernel::kGather;
        if (v == "batch") return Fp16Kernel::kBatch;
        return Fp16Kernel::kAuto;
    }();
    return k;
}

// Whether N > 128 takes the two-chunk batch kernel: when its grid still has
// at least 1024 workgroups (two fit a CU, so fewer would leave CUs short of
// waves: configs[1], 512 block-rows at N = 256, runs 7 % slower with two
// chunks, the headline matrix at N = 256 1.43x faster).  XSPMM_BATCH_WIDE=on
// or off forces the choice; C is the same either way.  Read on every call,
// so a process can compare the two.
// Whether a grid of two 128-column chunks puts each chunk on its own half of
// the XCDs (XSPMM_BATCH_XCD=off keeps both chunks of a block-row on one XCD).
bool batch_xcd_chunks()
{
    static const bool on = [] {
        const char* e = std::getenv("XSPMM_BATCH_XCD");
        return !(e && std::string(e) == "off");
    }();
    return on;
}

bool wide_batches(int64_t Mb, int64_t N)
{
    const char* e = std::getenv("XSPMM_BATCH_WIDE");
    if (e && std::string(e) == "on") return true;
    if (e && std::string(e) == "off") return false;
    return Mb * ((N + 255) / 256) >= 1024;
}

// fp32: the column-batch kernel runs one workgroup per block-row and 128
// columns; a grid shorter than this takes the tile kernel, which splits each
// block-row over 8 waves and narrower column tiles.  XSPMM_F32_KERNEL=batch
// forces the batch kernel (where it covers the shape), =tile the tile kernel.
constexpr int64_t kF32BatchMinGroups = 512;

bool f32_kernel_forced_batch()
{
    const char* e = std::getenv("XSPMM_F32_KERNEL");
    return e && std::string(e) == "batch";
}

void check_shape(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, int64_t N)
{
    if (M < 0 || K < 0 || Mb < 0 || Kb < 0 || nnzb < 0 || N < 0)
        throw std::invalid_argument("xSpMM: negative size passed to BCSR SpMM.");
    if (M > Mb * 16 || K > Kb * 16)
        throw std::invalid_argument("xSpMM: element shape exceeds the 16x16 block grid.");
    if (Mb > 0x7fffffffLL)
        throw std::invalid_argument("xSpMM: too many block-rows for one launch.");
}

// The kernels read the block values, and fp16 B rows, with 16-byte vector
// loads (fp16 B also straight into LDS); a pointer off a 16-byte boundary (a
// tensor view starting mid-row, for instance) is rejected before any launch.
void check_alignment(const void* bvals, const void* B, bool b_vector)
{
    if ((reinterpret_cast<uintptr_t>(bvals) & 15) != 0)
        throw std::invalid_argument("xSpMM: the block values must be 16-byte aligned.");
    if (b_vector && (reinterpret_cast<uintptr_t>(B) & 15) != 0)
        throw std::invalid_argument("xSpMM: fp16 B must be 16-byte aligned.");
}

}  // namespace

bool spmm_order_wanted(int64_t Mb) { return Mb > kOrderMinRows && Mb <= 0x7fffffffLL; }

bool spmm_order_cols_wanted(int64_t Mb) { return Mb >= kXcdOrderMinRows && Mb <= 0x7fffffffLL; }

int spmm_batch_waves() { return kBW; }

bool spmm_f16_pack_supported(int64_t K, int64_t Mb, int64_t Kb)
{
    return Mb > 0 && Mb <= 0x7fffffffLL && Kb < (int64_t(1) << 20) && K < (int64_t(1) << 24);
}

template <typename I>
void spmm_f16_pack_count(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                         const uint16_t* bvals, int32_t* counts, hipStream_t s)
{
    BatchPack pk{counts, nullptr, nullptr, nullptr};
    hipLaunchKernelGGL((spmm_f16_batch_kernel<I, 1, BatchMode::kCount>), dim3((unsigned)Mb, 1),
                       dim3(64 * kBW), 0, s, brp, bci, bvals, nullptr, nullptr, M, K, (int64_t)16, Kb,
                       nullptr, nullptr, pk);
    XSPMM_LAUNCH_CHECK();
}

template <typename I>
void spmm_f16_pack_fill(int64_t M, int64_t K, int64_t Mb, int64_t Kb, const I* brp, const I* bci,
                        const uint16_t* bvals, const int64_t* offsets, void* a, uint32_t* rows,
                        hipStream_t s)
{
    BatchPack pk{nullptr, offsets, static_cast<u32x4_t*>(a), rows};
    hipLaunchKernelGGL((spmm_f16_batch_kernel<I, 1, BatchMode::kPack>), dim3((unsigned)Mb, 1),
                       dim3(64 * kBW), 0, s, brp, bci, bvals, nullptr, nullptr, M, K, (int64_t)16, Kb,
                       nullptr, nullptr, pk);
    XSPMM_LAUNCH_CHECK();
}

template <typename I>
bool spmm_f16_packed(int64_t M, int64_t K, int64_t Mb, const int64_t* offsets, const void* a,
                     const uint32_t* rows, const uint16_t* B, float* C, int64_t N,
                     const int32_t* order, const I* row_map, hipStream_t s)
{
    if (M == 0 || N == 0 || Mb == 0) return true;
    check_alignment(a, B, true);
    if (N % 8 != 0 || K * N * 2 > (int64_t(1) << 31) || N >= (int64_t(1) << 22)) return false;
    const int64_t chunks = (N + 127) / 128;
    if (chunks > 65535) return false;
    const dim3 grid((unsigned)Mb, (unsigned)chunks);
    const u32x4_t* pa = static_cast<const u32x4_t*>(a);
    if (N <= 16)
        hipLaunchKernelGGL((spmm_f16_packed_kernel<I, 1>), grid, dim3(64 * kBW), 0, s, offsets, pa, rows,
                           B, C, M, K, N, order, row_map);
    else if (N <= 32)
        hipLaunchKernelGGL((spmm_f16_packed_kernel<I, 2>), grid, dim3(64 * kBW), 0, s, offsets, pa, rows,
                           B, C, M, K, N, order, row_map);
    else if (N <= 64)
        hipLaunchKernelGGL((spmm_f16_packed_kernel<I, 4>), grid, dim3(64 * kBW), 0, s, offsets, pa, rows,
                           B, C, M, K, N, order, row_map);
    else
        hipLaunchKernelGGL((spmm_f16_packed_kernel<I, 8>), grid, dim3(64 * kBW), 0, s, offsets, pa, rows,
                           B, C, M, K, N, order, row_map);
    XSPMM_LAUNCH_CHECK();
    return true;
}

int64_t spmm_f16_pack_offsets(const int32_t* counts, int64_t n, int64_t* offsets, hipStream_t s)
{
    device_exclusive_scan(ArrayValue<int32_t>{counts}, n, offsets, s);
    int64_t total = 0;
    XSPMM_HIP_CHECK(hipMemcpyAsync(&total, offsets + n, sizeof(int64_t), hipMemcpyDeviceToHost, s));
    XSPMM_HIP_CHECK(hipStreamSynchronize(s));
    return total;
}

#define XSPMM_PACK(I)                                                                             \
    template void spmm_f16_pack_count<I>(int64_t, int64_t, int64_t, int64_t, const I*, const I*,   \
                                         const uint16_t*, int32_t*, hipStream_t);                 \
    template void spmm_f16_pack_fill<I>(int64_t, int64_t, int64_t, int64_t, const I*, const I*,    \
                                        const uint16_t*, const int64_t*, void*, uint32_t*,        \
                                        hipStream_t);                                              \
    template bool spmm_f16_packed<I>(int64_t, int64_t, int64_t, const int64_t*, const void*,       \
                                     const uint32_t*, const uint16_t*, float*, int64_t,            \
                                     const int32_t*, const I*, hipStream_t);
XSPMM_PACK(int32_t)
XSPMM_PACK(int64_t)
#undef XSPMM_PACK

template <typename I>
void spmm_dispatch_order(const I* brp, int64_t Mb, int32_t* order, hipStream_t s)
{
    hipLaunchKernelGGL((order_rows_kernel<I>), dim3(1), dim3(kOrderThreads), 0, s, brp, Mb, order);
    XSPMM_LAUNCH_CHECK();
}
template void spmm_dispatch_order<int32_t>(const int32_t*, int64_t, int32_t*, hipStream_t);
template void spmm_dispatch_order<int64_t>(const int64_t*, int64_t, int32_t*, hipStream_t);

template <typename I>
bool spmm_dispatch_order_cols(const I* brp, const I* bci, int64_t Mb, int32_t* order, hipStream_t s)
{
    if (Mb > kOrderMinRows) {
        hipLaunchKernelGGL((order_rows_kernel<I>), dim3(1), dim3(kOrderThreads), 0, s, brp, Mb, order);
        XSPMM_LAUNCH_CHECK();
        return true;
    }
    hipLaunchKernelGGL((order_local_kernel<I>), dim3(1), dim3(256), 0, s, brp, bci, Mb, order);
    XSPMM_LAUNCH_CHECK();
    int32_t used = 0;
    XSPMM_HIP_CHECK(hipMemcpyAsync(&used, order + Mb, sizeof(used), hipMemcpyDeviceToHost, s));
    XSPMM_HIP_CHECK(hipStreamSynchronize(s));
    return used != 0;
}
template bool spmm_dispatch_order_cols<int32_t>(const int32_t*, const int32_t*, int64_t, int32_t*, hipStream_t);
template bool spmm_dispatch_order_cols<int64_t>(const int64_t*, const int64_t*, int64_t, int32_t*, hipStream_t);

namespace {

// The Tier-1 launcher: kernel choice as described at the top of this file;
// temporaries (the dispatch order, repacked B panels) come from `arena`.
template <typename T, typename I>
bool bcsr_spmm_launch(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
                      const I* bci, const T* bvals, const T* B, float* C, int64_t N,
                      const int32_t* order_in, const I* row_map, TempArena& arena, hipStream_t s)
{
    check_shape(M, K, Mb, Kb, nnzb, N);
    if (M == 0 || N == 0 || Mb == 0) return true;
    check_alignment(bvals, B, sizeof(T) == 2);
    const int64_t ntiles64 = (N + 15) / 16;
    if (ntiles64 > (1 << 24)) throw std::invalid_argument("xSpMM: N too large.");
    const int ntiles = (int)ntiles64;
    const Geometry geo = pick_geometry(ntiles);
    const dim3 grid((unsigned)Mb, (unsigned)geo.grid_y);
    const dim3 block(geo.waves * kWave);

    if constexpr (sizeof(T) == 2) {
        const uint16_t* v = reinterpret_cast<const uint16_t*>(bvals);
        const uint16_t* b = reinterpret_cast<const uint16_t*>(B);
        // batch and gather paths: byte offsets into B, and a wave's A range,
        // fit 32 bits; B row indices fit 24 bits
        const Fp16Kernel choice = fp16_kernel_choice();
        // every block present: GEMM-tiled kernel (matrix-core bound)
        if (choice == Fp16Kernel::kAuto && spmm_dense_f16_covers(M, K, Mb, Kb, nnzb, N))
            return bcsr_spmm_dense_f16<I>(M, K, Mb, Kb, nnzb, brp, bci, v, b, C, N, s, row_map);
        const bool offsets32 = K * N * 2 <= (int64_t(1) << 31) && N < (int64_t(1) << 22) &&
                               Kb < (int64_t(1) << 20);
        const int64_t chunks = (N + 127) / 128;
        if (chunks > 65535) throw std::invalid_argument("xSpMM: N too large.");
        const dim3 ggrid((unsigned)Mb, (unsigned)chunks);
        if ((choice == Fp16Kernel::kAuto || choice == Fp16Kernel::kBatch) && N % 8 == 0 &&
            offsets32) {
            // more block-rows than resident workgroups (4 per CU on 256 CUs,
            // times two): dispatch the longest rows first
            const int32_t* order = order_in;
            if (!order && spmm_order_wanted(Mb)) {
                int32_t* buf = arena.take_as<int32_t>((size_t)Mb);
                spmm_dispatch_order<I>(brp, Mb, buf, s);
                order = buf;
            }
            if (N <= 16)
                hipLaunchKernelGGL((spmm_f16_batch_kernel<I, 1>), ggrid, dim3(64 * kBW), 0, s, brp, bci,
                                   v, b, C, M, K, N, Kb, order, row_map, BatchPack{});
            else if (N <= 32)
                hipLaunchKernelGGL((spmm_f16_batch_kernel<I, 2>), ggrid, dim3(64 * kBW), 0, s, brp, bci,
                                   v, b, C, M, K, N, Kb, order, row_map, BatchPack{});
            else if (N <= 64)
                hipLaunchKernelGGL((spmm_f16_batch_kernel<I, 4>), ggrid, dim3(64 * kBW), 0, s, brp, bci,
                                   v, b, C, M, K, N, Kb, order, row_map, BatchPack{});
            else if (chunks == 2 && Mb % 4 == 0 && !wide_batches(Mb, N) && batch_xcd_chunks())
                hipLaunchKernelGGL((spmm_f16_batch_kernel<I, 8, BatchMode::kMultiply, 1, true>),
                                   dim3((unsigned)(2 * Mb), 1), dim3(64 * kBW), 0, s, brp, bci, v, b, C, M,
                                   K, N, Kb, order, row_map, BatchPack{});
            else if (N <= 128 || !wide_batches(Mb, N))
                hipLaunchKernelGGL((spmm_f16_batch_kernel<I, 8>), ggrid, dim3(64 * kBW), 0, s, brp, bci,
                                   v, b, C, M, K, N, Kb, order, row_map, BatchPack{});
            else  // 256 columns per workgroup: each pair compacted once for two chunks
                hipLaunchKernelGGL((spmm_f16_batch_kernel<I, 8, BatchMode::kMultiply, 2>),
                                   dim3((unsigned)Mb, (unsigned)((N + 255) / 256)), dim3(64 * kBW), 0,
                                   s, brp, bci, v, b, C, M, K, N, Kb, order, row_map, BatchPack{});
            XSPMM_LAUNCH_CHECK();
            return true;
        }
        if (row_map) return false;  // the other fp16 kernels store rows in place
        if (choice == Fp16Kernel::kGather && N % 2 == 0 && offsets32) {
            if (N <= 64)
                hipLaunchKernelGGL((spmm_f16_gather_kernel<I, 4, kGatherRows>), ggrid, dim3(256), 0, s, brp, bci,
                                   v, b, C, M, K, N, Kb);
            else
                hipLaunchKernelGGL((spmm_f16_gather_kernel<I, 8, kGatherRows>), ggrid, dim3(256), 0, s, brp, bci,
                                   v, b, C, M, K, N, Kb);
            XSPMM_LAUNCH_CHECK();
            return true;
        }
        const int64_t Np = ntiles64 * 16;
        uint16_t* bt = arena.take_as<uint16_t>((size_t)(Kb > 0 ? Kb : 1) * (size_t)Np * 16);
        if (Kb > 0) {
            const int64_t per_kb = Np * 2;
            const dim3 pg((unsigned)((per_kb + 255) / 256), (unsigned)(Kb < 65535 ? Kb : 65535));
            hipLaunchKernelGGL(pack_b_panels, pg, dim3(256), 0, s, b, bt, K, N, Kb, Np);
            XSPMM_LAUNCH_CHECK();
        }
        switch (geo.ntw) {
        case 4:
            hipLaunchKernelGGL((spmm_f16_kernel<I, 4>), grid, block, 0, s, brp, bci, v, bt, C, M,
                               N, Np, Kb, ntiles);
            break;
        case 2:
            hipLaunchKernelGGL((spmm_f16_kernel<I, 2>), grid, block, 0, s, brp, bci, v, bt, C, M,
                               N, Np, Kb, ntiles);
            break;
        default:
            hipLaunchKernelGGL((spmm_f16_kernel<I, 1>), grid, block, 0, s, brp, bci, v, bt, C, M,
                               N, Np, Kb, ntiles);
            break;
        }
        XSPMM_LAUNCH_CHECK();
    } else {
        const float* v = reinterpret_cast<const float*>(bvals);
        const float* b = reinterpret_cast<const float*>(B);
        // column batches (spmm_f32.hip) unless the grid is too short to keep
        // the chip busy with one workgroup per block-row
        if (spmm_f32_batch_covers(K, Kb, N, B, C) &&
            (f32_kernel_forced_batch() || Mb * ((N + 127) / 128) >= kF32BatchMinGroups)) {
            const int32_t* order = order_in;
            if (!order && spmm_order_wanted(Mb)) {
                int32_t* buf = arena.take_as<int32_t>((size_t)Mb);
                spmm_dispatch_order<I>(brp, Mb, buf, s);
                order = buf;
            }
            bcsr_spmm_f32_batch<I>(M, K, Mb, Kb, brp, bci, v, b, C, N, order, row_map, s);
            return true;
        }
        if (row_map) return false;  // the fp32 tile kernel stores rows in place
        // 16-column tiles per wave: 4 (fewer B loads per block) unless that
        // leaves fewer than 512 workgroups, when narrower tiles spread the
        // block-rows over more CUs
        int ntw = ntiles >= 4 ? 4 : (ntiles >= 2 ? 2 : 1);
        while (ntw > 1 && Mb * ((ntiles + ntw - 1) / ntw) < 512) ntw /= 2;
        const int64_t gy = (ntiles + ntw - 1) / ntw;
        if (gy > 65535) throw std::invalid_argument("xSpMM: N too large.");
        const dim3 fgrid((unsigned)Mb, (unsigned)gy);
        if (f32_short_wanted(Kb, N)) {
            const dim3 sblock(64 * kF32ShortWaves);
            switch (ntw) {
            case 4:
                hipLaunchKernelGGL((spmm_f32_short_kernel<I, 4>), fgrid, sblock, 0, s, brp, bci, v,
                                   b, C, M, K, N, Kb, ntiles);
                break;
            case 2:
                hipLaunchKernelGGL((spmm_f32_short_kernel<I, 2>), fgrid, sblock, 0, s, brp, bci, v,
                                   b, C, M, K, N, Kb, ntiles);
                break;
            default:
                hipLaunchKernelGGL((spmm_f32_short_kernel<I, 1>), fgrid, sblock, 0, s, brp, bci, v,
                                   b, C, M, K, N, Kb, ntiles);
                break;
            }
            XSPMM_LAUNCH_CHECK();
            return true;
        }
        const dim3 fblock(64 * kF32Waves);
        switch (ntw) {
        case 4:
            hipLaunchKernelGGL((spmm_f32_kernel<I, 4>), fgrid, fblock, 0, s, brp, bci, v, b, C, M,
                               K, N, ntiles);
            break;
        case 2:
            hipLaunchKernelGGL((spmm_f32_kernel<I, 2>), fgrid, fblock, 0, s, brp, bci, v, b, C, M,
                               K, N, ntiles);
            break;
        default:
            hipLaunchKernelGGL((spmm_f32_kernel<I, 1>), fgrid, fblock, 0, s, brp, bci, v, b, C, M,
                               K, N, ntiles);
            break;
        }
        XSPMM_LAUNCH_CHECK();
    }
    return true;
}

constexpr int kMaxDevices = 64;

}  // namespace

// Scratch of the allocation-free entry point (bcsr_spmm_noalloc): the only
// device memory it uses beyond its inputs and outputs.  Each GPU holds its
// own copy for the life of the process; every call on a GPU shares it, so
// calls that overlap on one GPU race.  Host code never passes `scratch`
// itself to a kernel (on the host it names a shadow variable, not device
// memory): it uses the device address that hipGetSymbolAddress returns,
// looked up once per device.
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

void* noalloc_scratch(int dev)
{
    static std::mutex mu;
    static void* ptr[kMaxDevices] = {};
    if (dev < 0 || dev >= kMaxDevices)
        throw std::invalid_argument("xSpMM: device index outside the allocation-free entry point's table.");
    std::lock_guard<std::mutex> lock(mu);
    if (!ptr[dev]) {
        void* p = nullptr;
        XSPMM_HIP_CHECK(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
        if (!p) throw std::runtime_error("xSpMM: no device address for the SpMM scratch array.");
        ptr[dev] = p;
    }
    return ptr[dev];
}

}  // namespace

template <typename T, typename I>
void bcsr_spmm(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
               const I* bci, const T* bvals, const T* B, float* C, int64_t N, hipStream_t s)
{
    TempArena arena(s);
    (void)bcsr_spmm_launch<T, I>(M, K, Mb, Kb, nnzb, brp, bci, bvals, B, C, N, nullptr, nullptr,
                                 arena, s);
}

template <typename T, typename I>
bool bcsr_spmm_ex(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
                  const I* bci, const T* bvals, const T* B, float* C, int64_t N,
                  const int32_t* order_in, const I* row_map, hipStream_t s)
{
    TempArena arena(s);
    return bcsr_spmm_launch<T, I>(M, K, Mb, Kb, nnzb, brp, bci, bvals, B, C, N, order_in, row_map,
                                  arena, s);
}

template <typename T, typename I>
void bcsr_spmm_band(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp, const I* bci,
                    const T* bvals, const T* B, float* C, int64_t N, hipStream_t s)
{
    check_shape(M, K, Mb, Kb, nnzb, N);
    if (M == 0 || N == 0 || Mb == 0) return;
    check_alignment(bvals, B, sizeof(T) == 2);
    if constexpr (sizeof(T) == 2) {
        if (bcsr_spmm_band_f16<I>(M, K, Mb, Kb, brp, bci, bvals, B, C, N, nullptr, s)) return;
    } else {
        if (bcsr_spmm_band_f32<I>(M, K, Mb, Kb, brp, bci, bvals, B, C, N, nullptr, nnzb, s)) return;
    }
    (void)bcsr_spmm_ex<T, I>(M, K, Mb, Kb, nnzb, brp, bci, bvals, B, C, N, nullptr, nullptr, s);
}
#define XSPMM_SPMM_BAND(T, I)                                                                          \
    template void bcsr_spmm_band<T, I>(int64_t, int64_t, int64_t, int64_t, int64_t, const I*, const I*, \
                                       const T*, const T*, float*, int64_t, hipStream_t);
XSPMM_SPMM_BAND(uint16_t, int32_t)
XSPMM_SPMM_BAND(uint16_t, int64_t)
XSPMM_SPMM_BAND(float, int32_t)
XSPMM_SPMM_BAND(float, int64_t)
#undef XSPMM_SPMM_BAND

template <typename T, typename I>
void bcsr_spmm_noalloc(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
                       const I* bci, const T* bvals, const T* B, float* C, int64_t N,
                       hipStream_t s)
{
    check_shape(M, K, Mb, Kb, nnzb, N);
    if (M > 0 && N > 0 && Mb > 0) check_alignment(bvals, B, sizeof(T) == 2);
    int dev = 0;
    XSPMM_HIP_CHECK(hipGetDevice(&dev));
    TempArena arena(noalloc_scratch(dev), kNoAllocScratchBytes, s);
    (void)bcsr_spmm_launch<T, I>(M, K, Mb, Kb, nnzb, brp, bci, bvals, B, C, N, nullptr, nullptr,
                                 arena, s);
}

#define XSPMM_SPMM_EX(T, I)                                                                      \
    template bool bcsr_spmm_ex<T, I>(int64_t, int64_t, int64_t, int64_t, int64_t, const I*,      \
                                     const I*, const T*, const T*, float*, int64_t,              \
                                     const int32_t*, const I*, hipStream_t);                     \
    template void bcsr_spmm<T, I>(int64_t, int64_t, int64_t, int64_t, int64_t, const I*,         \
                                  const I*, const T*, const T*, float*, int64_t, hipStream_t);   \
    template void bcsr_spmm_noalloc<T, I>(int64_t, int64_t, int64_t, int64_t, int64_t, const I*, \
                                          const I*, const T*, const T*, float*, int64_t,         \
                                          hipStream_t);
XSPMM_SPMM_EX(uint16_t, int32_t)
XSPMM_SPMM_EX(uint16_t, int64_t)
XSPMM_SPMM_EX(float, int32_t)
XSPMM_SPMM_EX(float, int64_t)
#undef XSPMM_SPMM_EX

}  // namespace detail
}  // namespace xspmm
