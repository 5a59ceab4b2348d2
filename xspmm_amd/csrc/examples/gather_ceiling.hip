// gather_ceiling.hip -- how fast can B rows be gathered at all?
//
// The Tier-1 kernels are bound, beside the A stream from HBM, by gathering B
// rows (mostly L2 hits) through the CUs' vector memory path.  This program
// measures that path alone, with the access patterns of two workloads and no
// A, no matrix cores and no C:
//   panels  configs[1] ("blocks"): 13 107 blocks on a 512 x 512 block grid
//           (5 %, uniform), N = 256.  Each block needs its 16 B rows; a wave
//           gathers the blocks w, w + 4, ... of its block-row, for one
//           128-column chunk (the batch kernel's grid: 2 chunks) or for whole
//           rows, with U blocks' loads in flight.
//   rows    the headline matrix's batches: 44 066 batches of 32 B rows
//           (fp16, N = 128: 256 bytes each) drawn uniformly from K = 16 384
//           rows, 10.8 batches per wave on 1024 workgroups of 4 waves.
// Each wave XORs what it loads (so nothing is optimized away) and stores one
// 16-byte value per lane.  Times are per launch, from 50 back-to-back
// launches between two events (best of 4 rounds).
//
// usage: gather_ceiling
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <random>
#include <vector>

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define CK(x)                                                                              \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

namespace {

// Raw buffer over [base, base + bytes): reads past the end return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void* base, uint32_t bytes)
{
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes,
                                             0x00020000);
}

// panels: workgroup (block-row, chunk), 4 waves; wave w gathers the 16 B rows
// (CB bytes from byte CB * chunk of each row, row stride RB) of blocks
// rs + w, rs + w + 4, ..., U blocks' loads in flight
template <int CB, int U>
__global__ __launch_bounds__(256) void gather_panels(const int* __restrict__ brp,
                                                     const int* __restrict__ cols,
                                                     const uint16_t* __restrict__ B, uint32_t bbytes,
                                                     uint32_t RB, u32x4_t* __restrict__ out)
{
    constexpr int LPR = CB / 16;  // lanes per row
    constexpr int RPL = 64 / LPR; // rows per load
    constexpr int NL = 16 / RPL;  // loads per block
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int rs = brp[blockIdx.x];
    const int re = brp[blockIdx.x + 1];
    const __amdgpu_buffer_rsrc_t r = rsrc(B, bbytes);
    const uint32_t lo = (uint32_t)(lane / LPR) * RB + (uint32_t)(lane % LPR) * 16u + blockIdx.y * CB;
    u32x4_t acc = {0u, 0u, 0u, 0u};
    int b = rs + wave;
    for (; b + 4 * (U - 1) < re; b += 4 * U) {
        u32x4_t v[U][NL];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const uint32_t base = (uint32_t)cols[b + 4 * u] * 16u * RB + lo;
#pragma unroll
            for (int l = 0; l < NL; ++l)
                v[u][l] = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(base + l * RPL * RB), 0, 0));
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int l = 0; l < NL; ++l) acc ^= v[u][l];
    }
    for (; b < re; b += 4) {
        const uint32_t base = (uint32_t)cols[b] * 16u * RB + lo;
#pragma unroll
        for (int l = 0; l < NL; ++l)
            acc ^= __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(base + l * RPL * RB), 0, 0));
    }
    out[((size_t)(blockIdx.y * gridDim.x + blockIdx.x) * 4 + wave) * 64 + lane] = acc;
}

// rows: wave (workgroup g, wave w) gathers batches first[g * 4 + w] ..
// first[g * 4 + w + 1] - 1, each 32 B rows of 256 bytes (row indices in idx,
// 32 per batch); lane l moves row 4 t + l / 16, chunk l % 16 of load t;
// U batches' loads in flight
template <int U>
__global__ __launch_bounds__(256) void gather_rows(const int64_t* __restrict__ first,
                                                   const uint32_t* __restrict__ idx,
                                                   const uint16_t* __restrict__ B, uint32_t bbytes,
                                                   u32x4_t* __restrict__ out)
{
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    const int64_t unit = (int64_t)blockIdx.x * 4 + wave;
    const int64_t b0 = first[unit];
    const int64_t b1 = first[unit + 1];
    const __amdgpu_buffer_rsrc_t r = rsrc(B, bbytes);
    const uint32_t chunk = 16u * (uint32_t)(lane & 15);
    u32x4_t acc = {0u, 0u, 0u, 0u};
    int64_t b = b0;
    for (; b + U <= b1; b += U) {
        u32x4_t v[U][8];
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < 8; ++t) {
                const uint32_t row = idx[(b + u) * 32 + 4 * t + (lane >> 4)];
                v[u][t] = __builtin_bit_cast(
                    u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(row * 256u + chunk), 0, 0));
            }
#pragma unroll
        for (int u = 0; u < U; ++u)
#pragma unroll
            for (int t = 0; t < 8; ++t) acc ^= v[u][t];
    }
    for (; b < b1; ++b)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
            const uint32_t row = idx[b * 32 + 4 * t + (lane >> 4)];
            acc ^= __builtin_bit_cast(
                u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(r, (int)(row * 256u + chunk), 0, 0));
        }
    out[unit * 64 + lane] = acc;
}

}  // namespace

int main()
{
    hipEvent_t e0, e1;
    CK(hipEventCreate(&e0));
    CK(hipEventCreate(&e1));
    // best per-launch time of 4 rounds of 50 back-to-back launches
    auto time_it = [&](auto launch, float& best_us) -> int {
        best_us = 1e30f;
        for (int round = 0; round < 5; ++round) {
            CK(hipEventRecord(e0));
            for (int k = 0; k < 50; ++k) launch();
            CK(hipGetLastError());
            CK(hipEventRecord(e1));
            CK(hipEventSynchronize(e1));
            float ms = 0.f;
            CK(hipEventElapsedTime(&ms, e0, e1));
            if (round > 0) best_us = std::min(best_us, ms * 1e3f / 50.f);
        }
        return 0;
    };
    std::mt19937_64 rng(1);

    // --- panels: configs[1] -----------------------------------------------
    {
        const int Mb = 512, Kb = 512, N = 256;
        const long total = (long)Mb * Kb, nnzb = (long)(0.05 * total + 0.5);
        std::vector<long> ids(total);
        for (long i = 0; i < total; ++i) ids[i] = i;
        for (long i = 0; i < nnzb; ++i) {
            std::uniform_int_distribution<long> d(i, total - 1);
            std::swap(ids[i], ids[d(rng)]);
        }
        std::sort(ids.begin(), ids.begin() + nnzb);
        std::vector<int> brp(Mb + 1, 0), cols(nnzb);
        for (long i = 0; i < nnzb; ++i) {
            brp[ids[i] / Kb + 1]++;
            cols[i] = (int)(ids[i] % Kb);
        }
        for (int r = 0; r < Mb; ++r) brp[r + 1] += brp[r];
        const uint32_t RB = N * 2, bbytes = (uint32_t)Kb * 16u * RB;
        int *dbrp, *dcols;
        uint16_t* dB;
        u32x4_t* dout;
        CK(hipMalloc(&dbrp, brp.size() * sizeof(int)));
        CK(hipMalloc(&dcols, cols.size() * sizeof(int)));
        CK(hipMalloc(&dB, bbytes));
        CK(hipMalloc(&dout, (size_t)Mb * 2 * 4 * 64 * sizeof(u32x4_t)));
        CK(hipMemcpy(dbrp, brp.data(), brp.size() * sizeof(int), hipMemcpyHostToDevice));
        CK(hipMemcpy(dcols, cols.data(), cols.size() * sizeof(int), hipMemcpyHostToDevice));
        CK(hipMemset(dB, 1, bbytes));
        struct V {
            const char* name;
            int chunks, cb;
            void (*k)(const int*, const int*, const uint16_t*, uint32_t, uint32_t, u32x4_t*);
        };
        const V vs[] = {{"128-column chunks, 1 block in flight", 2, 256, gather_panels<256, 1>},
                        {"128-column chunks, 2 blocks in flight", 2, 256, gather_panels<256, 2>},
                        {"128-column chunks, 4 blocks in flight", 2, 256, gather_panels<256, 4>},
                        {"whole rows, 1 block in flight", 1, 512, gather_panels<512, 1>},
                        {"whole rows, 2 blocks in flight", 1, 512, gather_panels<512, 2>}};
        for (const V& v : vs) {
            float us;
            if (time_it([&] {
                    hipLaunchKernelGGL(v.k, dim3(Mb, v.chunks), dim3(256), 0, 0, dbrp, dcols, dB,
                                       bbytes, RB, dout);
                }, us))
                return 1;
            const double bytes = (double)nnzb * 16 * v.cb * v.chunks;
            std::printf("panels (configs[1], %ld blocks, N=%d) %-40s %7.2f us  %6.1f MB  %5.2f TB/s\n",
                        nnzb, N, v.name, us, bytes / 1e6, bytes / (us * 1e-6) / 1e12);
        }
        CK(hipFree(dbrp));
        CK(hipFree(dcols));
        CK(hipFree(dB));
        CK(hipFree(dout));
    }

    // --- rows: the headline matrix's batches ---------------------------------
    {
        const int K = 16384, waves = 1024 * 4;
        const int64_t nb = 44066;
        const uint32_t bbytes = (uint32_t)K * 256u;
        std::vector<uint32_t> idx((size_t)nb * 32);
        std::uniform_int_distribution<uint32_t> d(0, K - 1);
        for (auto& x : idx) x = d(rng);
        std::vector<int64_t> first(waves + 1);
        for (int w = 0; w <= waves; ++w) first[w] = nb * w / waves;
        int64_t* dfirst;
        uint32_t* didx;
        uint16_t* dB;
        u32x4_t* dout;
        CK(hipMalloc(&dfirst, first.size() * sizeof(int64_t)));
        CK(hipMalloc(&didx, idx.size() * sizeof(uint32_t)));
        CK(hipMalloc(&dB, bbytes));
        CK(hipMalloc(&dout, (size_t)waves * 64 * sizeof(u32x4_t)));
        CK(hipMemcpy(dfirst, first.data(), first.size() * sizeof(int64_t), hipMemcpyHostToDevice));
        CK(hipMemcpy(didx, idx.data(), idx.size() * sizeof(uint32_t), hipMemcpyHostToDevice));
        CK(hipMemset(dB, 1, bbytes));
        struct V {
            const char* name;
            void (*k)(const int64_t*, const uint32_t*, const uint16_t*, uint32_t, u32x4_t*);
        };
        const V vs[] = {{"1 batch in flight", gather_rows<1>},
                        {"2 batches in flight", gather_rows<2>},
                        {"4 batches in flight", gather_rows<4>}};
        for (const V& v : vs) {
            float us;
            if (time_it([&] {
                    hipLaunchKernelGGL(v.k, dim3(waves / 4), dim3(256), 0, 0, dfirst, didx, dB,
                                       bbytes, dout);
                }, us))
                return 1;
            const double bytes = (double)nb * 32 * 256;
            std::printf("rows (templates batches, %lld x 32 rows, N=128) %-26s %7.2f us  %6.1f MB  %5.2f TB/s\n",
                        (long long)nb, v.name, us, bytes / 1e6, bytes / (us * 1e-6) / 1e12);
        }
        CK(hipFree(dfirst));
        CK(hipFree(didx));
        CK(hipFree(dB));
        CK(hipFree(dout));
    }
    return 0;
}
