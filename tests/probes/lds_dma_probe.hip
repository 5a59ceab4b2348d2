// lds_dma_probe.hip -- the two properties of buffer_load_dwordx4 ... lds that
// spmm_f16_batch_kernel relies on when it loads a batch's B rows straight into
// its LDS tile:
//   layout  one load fills 1 KB of LDS lane by lane: lane l's 16 bytes land
//           at [base + 16 l, base + 16 l + 16), whatever address it read;
//   zeros   a lane whose buffer offset lies past the resource's size writes
//           16 zero bytes there (the kernel points unused batch slots past
//           the end of B; stale tile rows would turn Inf or NaN entries of an
//           earlier batch into NaN through the compaction's zeros).
// One workgroup of one wave.  Every access stays in bounds: the source buffer
// holds 1 KB, the LDS array 2 KB, the output 2 KB, and the out-of-range
// offsets never reach memory (the buffer resource's range check).
//
// usage: lds_dma_probe   (prints "lds dma probe ok" and exits 0 when both hold)
#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <vector>

#define CK(x)                                                                              \
    do {                                                                                   \
        hipError_t e_ = (x);                                                               \
        if (e_ != hipSuccess) {                                                            \
            std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
            return 1;                                                                      \
        }                                                                                  \
    } while (0)

namespace {

typedef __attribute__((address_space(3))) void lds_void_t;

constexpr uint32_t kSrcBytes = 1024;
constexpr uint32_t kMarker = 0xdeadbeefu;

// lane l of load 0 reads source chunk (5 l) mod 64 (a permutation);
// lane l of load 1 reads chunk l for l < 32 and nothing (past the end) else
__global__ __launch_bounds__(64) void probe(const uint32_t* __restrict__ src, uint32_t* __restrict__ out)
{
    __shared__ __align__(16) uint32_t lds[512];
    const uint32_t lane = threadIdx.x;
    for (uint32_t i = lane; i < 512; i += 64) lds[i] = kMarker;
    __syncthreads();
    const __amdgpu_buffer_rsrc_t r =
        __builtin_amdgcn_make_buffer_rsrc((void*)src, (short)0, (int)kSrcBytes, 0x00020000);
    const uint32_t off0 = 16u * ((5u * lane) & 63u);
    const uint32_t off1 = lane < 32u ? 16u * lane : kSrcBytes + 16u * lane;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)&lds[0], 16, (int)off0, 0, 0, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (lds_void_t*)&lds[256], 16, (int)off1, 0, 0, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (uint32_t i = lane; i < 512; i += 64) out[i] = lds[i];
}

}  // namespace

int main()
{
    std::vector<uint32_t> h_src(kSrcBytes / 4);
    for (size_t i = 0; i < h_src.size(); ++i) h_src[i] = 0x01000000u + (uint32_t)i * 2654435761u % 1000003u;
    uint32_t *d_src = nullptr, *d_out = nullptr;
    CK(hipMalloc(&d_src, kSrcBytes));
    CK(hipMalloc(&d_out, 2048));
    CK(hipMemcpy(d_src, h_src.data(), kSrcBytes, hipMemcpyHostToDevice));
    CK(hipMemset(d_out, 0, 2048));
    hipLaunchKernelGGL(probe, dim3(1), dim3(64), 0, 0, d_src, d_out);
    CK(hipGetLastError());
    CK(hipDeviceSynchronize());
    std::vector<uint32_t> h_out(512);
    CK(hipMemcpy(h_out.data(), d_out, 2048, hipMemcpyDeviceToHost));
    CK(hipFree(d_src));
    CK(hipFree(d_out));

    int bad_layout = 0, bad_zero = 0, bad_in = 0;
    for (uint32_t l = 0; l < 64; ++l) {
        const uint32_t chunk = (5u * l) & 63u;
        for (uint32_t d = 0; d < 4; ++d)
            if (h_out[4 * l + d] != h_src[4 * chunk + d]) ++bad_layout;
    }
    for (uint32_t l = 0; l < 64; ++l)
        for (uint32_t d = 0; d < 4; ++d) {
            const uint32_t v = h_out[256 + 4 * l + d];
            if (l < 32 && v != h_src[4 * l + d]) ++bad_in;
            if (l >= 32 && v != 0u) ++bad_zero;
        }
    std::printf("layout mismatches %d, in-range mismatches %d, out-of-range words not zero %d\n",
                bad_layout, bad_in, bad_zero);
    if (bad_layout || bad_in || bad_zero) return 1;
    std::printf("lds dma probe ok\n");
    return 0;
}
