#pragma once
// Executors own device selection and raw memory transport.
// Interface as in the reference (include/xspmm/core/executor.hpp:10-67).
//
// HipExecutor targets one MI355X (gfx950).  All library work issued through it
// runs on the null stream of its device, so it orders with blocking hipMemcpy
// and with any stream created by hipStreamCreate.  CudaExecutor is kept for
// source compatibility only: constructing it throws, exactly like the
// reference's build without the CUDA backend (src/core/executor.cpp:110-121).

#include <cstddef>
#include <memory>
#include <stdexcept>

namespace xspmm {

class Executor {
public:
    virtual ~Executor() = default;

    virtual void allocate(void** ptr, size_t bytes) const = 0;
    virtual void free(void* ptr) const = 0;

    virtual void copy_from_host(void* device_dst, const void* host_src, size_t bytes) const = 0;
    virtual void copy_to_host(void* host_dst, const void* device_src, size_t bytes) const = 0;
    virtual void copy_device_to_device(void* dst, const void* src, size_t bytes) const = 0;

    virtual void synchronize() const = 0;

    // Typed helper used by the reference README quick start.
    template <typename T>
    T* allocate_temp(size_t count) const {
        void* p = nullptr;
        allocate(&p, count * sizeof(T));
        return static_cast<T*>(p);
    }
};

class CpuExecutor : public Executor {
public:
    CpuExecutor() = default;
    ~CpuExecutor() override = default;

    void allocate(void** ptr, size_t bytes) const override;
    void free(void* ptr) const override;
    void copy_from_host(void* device_dst, const void* host_src, size_t bytes) const override;
    void copy_to_host(void* host_dst, const void* device_src, size_t bytes) const override;
    void copy_device_to_device(void* dst, const void* src, size_t bytes) const override;
    void synchronize() const override;
};

class CudaExecutor : public Executor {
public:
    explicit CudaExecutor(int device_id = 0);
    ~CudaExecutor() override;

    void allocate(void** ptr, size_t bytes) const override;
    void free(void* ptr) const override;
    void copy_from_host(void* device_dst, const void* host_src, size_t bytes) const override;
    void copy_to_host(void* host_dst, const void* device_src, size_t bytes) const override;
    void copy_device_to_device(void* dst, const void* src, size_t bytes) const override;
    void synchronize() const override;

private:
    [[maybe_unused]] int device_id_;
};

class HipExecutor : public Executor {
public:
    explicit HipExecutor(int device_id = 0);
    ~HipExecutor() override;

    void allocate(void** ptr, size_t bytes) const override;
    void free(void* ptr) const override;
    void copy_from_host(void* device_dst, const void* host_src, size_t bytes) const override;
    void copy_to_host(void* host_dst, const void* device_src, size_t bytes) const override;
    void copy_device_to_device(void* dst, const void* src, size_t bytes) const override;
    void synchronize() const override;

    int get_device_id() const { return device_id_; }

private:
    int device_id_;
};

}  // namespace xspmm
