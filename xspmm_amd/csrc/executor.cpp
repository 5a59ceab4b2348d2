// executor.cpp -- CpuExecutor / HipExecutor (reference src/core/executor.cpp).
#include <cstdlib>
#include <cstring>
#include <mutex>
#include <new>
#include <set>

#include "internal.hpp"

namespace xspmm {

// ---------------------------------------------------------------------------
// CPU: 64-byte aligned host memory (reference executor.cpp:44-72).
// ---------------------------------------------------------------------------
namespace {
constexpr size_t kCpuAlignment = 64;
}

void CpuExecutor::allocate(void** ptr, size_t bytes) const
{
    const size_t aligned = (bytes + kCpuAlignment - 1) & ~(kCpuAlignment - 1);
    *ptr = std::aligned_alloc(kCpuAlignment, aligned ? aligned : kCpuAlignment);
    if (*ptr == nullptr) throw std::bad_alloc();
}
void CpuExecutor::free(void* ptr) const { std::free(ptr); }
void CpuExecutor::copy_from_host(void* dst, const void* src, size_t bytes) const
{
    if (bytes) std::memcpy(dst, src, bytes);
}
void CpuExecutor::copy_to_host(void* dst, const void* src, size_t bytes) const
{
    if (bytes) std::memcpy(dst, src, bytes);
}
void CpuExecutor::copy_device_to_device(void* dst, const void* src, size_t bytes) const
{
    if (bytes) std::memcpy(dst, src, bytes);
}
void CpuExecutor::synchronize() const {}

// ---------------------------------------------------------------------------
// CUDA: not part of this build (reference stub behaviour, executor.cpp:110-121).
// ---------------------------------------------------------------------------
CudaExecutor::CudaExecutor(int device_id) : device_id_(device_id)
{
    throw std::runtime_error("xSpMM was not compiled with CUDA support.");
}
CudaExecutor::~CudaExecutor() = default;
void CudaExecutor::allocate(void**, size_t) const {}
void CudaExecutor::free(void*) const {}
void CudaExecutor::copy_from_host(void*, const void*, size_t) const {}
void CudaExecutor::copy_to_host(void*, const void*, size_t) const {}
void CudaExecutor::copy_device_to_device(void*, const void*, size_t) const {}
void CudaExecutor::synchronize() const {}

// ---------------------------------------------------------------------------
// HIP (reference executor.cpp:130-158).  Copies are blocking hipMemcpy on the
// null stream, so they order with every kernel the library enqueues there.
// ---------------------------------------------------------------------------
HipExecutor::HipExecutor(int device_id) : device_id_(device_id)
{
    XSPMM_HIP_CHECK(hipSetDevice(device_id_));
    detail::init_device_pool(device_id_);
}
HipExecutor::~HipExecutor() = default;

void HipExecutor::allocate(void** ptr, size_t bytes) const { XSPMM_HIP_CHECK(hipMalloc(ptr, bytes)); }
void HipExecutor::free(void* ptr) const { XSPMM_HIP_CHECK(hipFree(ptr)); }
void HipExecutor::copy_from_host(void* dst, const void* src, size_t bytes) const
{
    if (bytes) XSPMM_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyHostToDevice));
}
void HipExecutor::copy_to_host(void* dst, const void* src, size_t bytes) const
{
    if (bytes) XSPMM_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToHost));
}
void HipExecutor::copy_device_to_device(void* dst, const void* src, size_t bytes) const
{
    if (bytes) XSPMM_HIP_CHECK(hipMemcpy(dst, src, bytes, hipMemcpyDeviceToDevice));
}
void HipExecutor::synchronize() const { XSPMM_HIP_CHECK(hipDeviceSynchronize()); }

namespace detail {

void init_device_pool(int device)
{
    static std::mutex mu;
    static std::set<int> done;
    std::lock_guard<std::mutex> lock(mu);
    if (done.count(device)) return;
    hipMemPool_t pool = nullptr;
    if (hipDeviceGetDefaultMemPool(&pool, device) == hipSuccess && pool) {
        uint64_t keep = UINT64_MAX;
        (void)hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep);
    }
    (void)hipGetLastError();
    done.insert(device);
}

}  // namespace detail
}  // namespace xspmm
