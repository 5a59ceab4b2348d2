// spmm.hip -- Tier-1 BCSR SpMM on CDNA4 matrix cores (gfx950).
//
// Semantics follow the reference tile kernel (src/common/spmm_math.hpp:20-146):
// for block-row br, C[16*br : +16, :] = sum over the row's blocks (in col_ind
// order) of A_blk * B[16*col : +16, :]; C is overwritten and block-rows without
// blocks become zero.  Rows >= M are not stored; B rows >= K and columns >= N
// contribute nothing.
//
// fp16 path.  MFMA operands want K contiguous in every lane, while B is
// row-major (N contiguous).  B is therefore first repacked into 16-row panels
// laid out [block_col][n][k16] (pack_b_panels), zero-padded beyond K and N.
// Two consecutive blocks of a block-row then form one K=32 operand pair for
// v_mfma_f32_16x16x32_f16:
//   A operand, lane l: block (l>>5), row l&15, k = 8*((l>>4)&1) .. +8  (16 bytes)
//   B operand, lane l: panel of the same block, n = l&15, the same 8 k
// so one 16-byte load per lane fetches each operand.  Output lane l holds
// C[4*(l>>4) + r][l&15], r = 0..3.
//
// fp32 path.  v_mfma_f32_16x16x4f32 takes one k per lane, so B is read
// row-major directly: lane l loads A[l&15][4g .. 4g+3] (g = l>>4) once per block
// and issues four MFMAs, step s pairing A[i][4g+s] with B[16*col + 4g + s][n].
//
// Work split: one workgroup per block-row (grid.x), its waves own disjoint
// groups of NTW 16-column tiles of C (grid.y covers wide N).  All waves of a
// workgroup walk the same A blocks, which stay in the CU's L1.
#include "internal.hpp"

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
// fp32 x fp32 -> fp32 tile kernel.
// ---------------------------------------------------------------------------
template <typename I, int NTW>
__global__ __launch_bounds__(256) void spmm_f32_kernel(const I* __restrict__ brp,
                                                       const I* __restrict__ bci,
                                                       const float* __restrict__ vals,
                                                       const float* __restrict__ B,
                                                       float* __restrict__ C, int64_t M,
                                                       int64_t K, int64_t N, int ntiles)
{
    const int lane = threadIdx.x & (kWave - 1);
    const int wave = threadIdx.x / kWave;
    const int waves = blockDim.x / kWave;
    const int tile0 = (blockIdx.y * waves + wave) * NTW;
    if (tile0 >= ntiles) return;

    const int64_t br = blockIdx.x;
    const int64_t rs = brp[br];
    const int64_t re = brp[br + 1];
    const int li = lane & 15;
    const int g = lane >> 4;

    float4_t acc[NTW];
#pragma unroll
    for (int j = 0; j < NTW; ++j) acc[j] = float4_t{0.f, 0.f, 0.f, 0.f};

    for (int64_t blk = rs; blk < re; ++blk) {
        const float4_t a = *reinterpret_cast<const float4_t*>(vals + blk * 256 + li * 16 + g * 4);
        const int64_t col = (int64_t)bci[blk];
        const int64_t kbase = (col >= 0 ? col : K) * 16 + g * 4;  // invalid columns read nothing
#pragma unroll
        for (int j = 0; j < NTW; ++j) {
            const int64_t n = (int64_t)(tile0 + j) * 16 + li;
            float bv[4];
#pragma unroll
            for (int s = 0; s < 4; ++s) {
                const int64_t k = kbase + s;
                bv[s] = (k >= 0 && k < K && n < N) ? B[k * N + n] : 0.f;
            }
#pragma unroll
            for (int s = 0; s < 4; ++s)
                acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[s], bv[s], acc[j], 0, 0, 0);
        }
    }

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

void check_shape(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, int64_t N)
{
    if (M < 0 || K < 0 || Mb < 0 || Kb < 0 || nnzb < 0 || N < 0)
        throw std::invalid_argument("xSpMM: negative size passed to BCSR SpMM.");
    if (M > Mb * 16 || K > Kb * 16)
        throw std::invalid_argument("xSpMM: element shape exceeds the 16x16 block grid.");
    if (Mb > 0x7fffffffLL)
        throw std::invalid_argument("xSpMM: too many block-rows for one launch.");
}

}  // namespace

template <typename T, typename I>
void bcsr_spmm(int64_t M, int64_t K, int64_t Mb, int64_t Kb, int64_t nnzb, const I* brp,
               const I* bci, const T* bvals, const T* B, float* C, int64_t N, hipStream_t s)
{
    check_shape(M, K, Mb, Kb, nnzb, N);
    if (M == 0 || N == 0 || Mb == 0) return;
    const int64_t ntiles64 = (N + 15) / 16;
    if (ntiles64 > (1 << 24)) throw std::invalid_argument("xSpMM: N too large.");
    const int ntiles = (int)ntiles64;
    const Geometry geo = pick_geometry(ntiles);
    const dim3 grid((unsigned)Mb, (unsigned)geo.grid_y);
    const dim3 block(geo.waves * kWave);

    if constexpr (sizeof(T) == 2) {
        const int64_t Np = ntiles64 * 16;
        Scratch bt((size_t)(Kb > 0 ? Kb : 1) * (size_t)Np * 16 * sizeof(uint16_t), s);
        if (Kb > 0) {
            const int64_t per_kb = Np * 2;
            const dim3 pg((unsigned)((per_kb + 255) / 256), (unsigned)(Kb < 65535 ? Kb : 65535));
            hipLaunchKernelGGL(pack_b_panels, pg, dim3(256), 0, s,
                               reinterpret_cast<const uint16_t*>(B), bt.as<uint16_t>(), K, N, Kb,
                               Np);
            XSPMM_LAUNCH_CHECK();
        }
        const uint16_t* v = reinterpret_cast<const uint16_t*>(bvals);
        switch (geo.ntw) {
        case 4:
            hipLaunchKernelGGL((spmm_f16_kernel<I, 4>), grid, block, 0, s, brp, bci, v,
                               bt.as<uint16_t>(), C, M, N, Np, Kb, ntiles);
            break;
        case 2:
            hipLaunchKernelGGL((spmm_f16_kernel<I, 2>), grid, block, 0, s, brp, bci, v,
                               bt.as<uint16_t>(), C, M, N, Np, Kb, ntiles);
            break;
        default:
            hipLaunchKernelGGL((spmm_f16_kernel<I, 1>), grid, block, 0, s, brp, bci, v,
                               bt.as<uint16_t>(), C, M, N, Np, Kb, ntiles);
            break;
        }
        XSPMM_LAUNCH_CHECK();
    } else {
        const float* v = reinterpret_cast<const float*>(bvals);
        const float* b = reinterpret_cast<const float*>(B);
        switch (geo.ntw) {
        case 4:
            hipLaunchKernelGGL((spmm_f32_kernel<I, 4>), grid, block, 0, s, brp, bci, v, b, C, M,
                               K, N, ntiles);
            break;
        case 2:
            hipLaunchKernelGGL((spmm_f32_kernel<I, 2>), grid, block, 0, s, brp, bci, v, b, C, M,
                               K, N, ntiles);
            break;
        default:
            hipLaunchKernelGGL((spmm_f32_kernel<I, 1>), grid, block, 0, s, brp, bci, v, b, C, M,
                               K, N, ntiles);
            break;
        }
        XSPMM_LAUNCH_CHECK();
    }
}

template void bcsr_spmm<uint16_t, int32_t>(int64_t, int64_t, int64_t, int64_t, int64_t,
                                           const int32_t*, const int32_t*, const uint16_t*,
                                           const uint16_t*, float*, int64_t, hipStream_t);
template void bcsr_spmm<uint16_t, int64_t>(int64_t, int64_t, int64_t, int64_t, int64_t,
                                           const int64_t*, const int64_t*, const uint16_t*,
                                           const uint16_t*, float*, int64_t, hipStream_t);
template void bcsr_spmm<float, int32_t>(int64_t, int64_t, int64_t, int64_t, int64_t,
                                        const int32_t*, const int32_t*, const float*,
                                        const float*, float*, int64_t, hipStream_t);
template void bcsr_spmm<float, int64_t>(int64_t, int64_t, int64_t, int64_t, int64_t,
                                        const int64_t*, const int64_t*, const float*,
                                        const float*, float*, int64_t, hipStream_t);

}  // namespace detail
}  // namespace xspmm
