// runtime.hpp — HIP runtime plumbing of the C ABI: error mapping, device
// selection, device buffers.
#pragma once

#include <hip/hip_runtime.h>

#include <string>

#include "status.hpp"

namespace nut {

[[noreturn]] void fail_hip(hipError_t error, const char *what);

inline void hip_check(hipError_t error, const char *what)
{
    if (error != hipSuccess)
        fail_hip(error, what);
}

// Raises NUT_EDEVICE if the last kernel launch failed.
void check_launch(const char *what);

// Makes sure a gfx950 device is current for this thread; throws
// NUT_EDEVICE when there is none.
void ensure_device();

// Device allocations made by this library since it was loaded (every
// hipMalloc it issues: DeviceBuffer::allocate and nut_malloc).
unsigned long long device_allocations();
void count_device_allocation();

// RAII device allocation.
class DeviceBuffer {
public:
    DeviceBuffer() = default;
    explicit DeviceBuffer(size_t bytes) { allocate(bytes); }
    ~DeviceBuffer() { release(); }
    DeviceBuffer(const DeviceBuffer &) = delete;
    DeviceBuffer &operator=(const DeviceBuffer &) = delete;
    DeviceBuffer(DeviceBuffer &&other) noexcept
        : ptr_(other.ptr_), bytes_(other.bytes_)
    {
        other.ptr_ = nullptr;
        other.bytes_ = 0;
    }
    void allocate(size_t bytes);
    void release();
    template <typename T> T *as() const { return static_cast<T *>(ptr_); }
    void *get() const { return ptr_; }
    size_t bytes() const { return bytes_; }

private:
    void *ptr_ = nullptr;
    size_t bytes_ = 0;
};

} // namespace nut
