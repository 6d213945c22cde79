// runtime.cpp — HIP error mapping, device selection and buffers.
#include <atomic>
#include "runtime.hpp"

#include <cstring>
#include <string>

namespace nut {

namespace {

thread_local std::string g_last_error;
thread_local int g_device = 0;
thread_local bool g_device_ready = false;

} // namespace

void set_last_error(const char *message) { g_last_error = message; }
const char *last_error() { return g_last_error.c_str(); }

void fail_hip(hipError_t error, const char *what)
{
    fail(NUT_EDEVICE, std::string(what) + ": " + hipGetErrorString(error));
}

void check_launch(const char *what)
{
    const hipError_t error = hipGetLastError();
    if (error != hipSuccess)
        fail_hip(error, what);
}

int select_device(int device)
{
    int count = 0;
    if (hipGetDeviceCount(&count) != hipSuccess)
        count = 0;
    if (device < 0 || device >= count)
        fail(NUT_EDEVICE, "no such HIP device");
    hipDeviceProp_t props;
    hip_check(hipGetDeviceProperties(&props, device), "hipGetDeviceProperties");
    if (std::strncmp(props.gcnArchName, "gfx950", 6) != 0)
        fail(NUT_EDEVICE, std::string("device is ") + props.gcnArchName +
                              ", this library is built for gfx950");
    hip_check(hipSetDevice(device), "hipSetDevice");
    g_device = device;
    g_device_ready = true;
    return device;
}

void ensure_device()
{
    if (g_device_ready) {
        hip_check(hipSetDevice(g_device), "hipSetDevice");
        return;
    }
    select_device(g_device);
}

namespace {
std::atomic<unsigned long long> g_allocations{0};
}

unsigned long long device_allocations() { return g_allocations.load(); }

void count_device_allocation() { g_allocations.fetch_add(1); }

void DeviceBuffer::allocate(size_t bytes)
{
    release();
    if (bytes == 0)
        bytes = 1;
    hip_check(hipMalloc(&ptr_, bytes), "hipMalloc");
    count_device_allocation();
    bytes_ = bytes;
}

void DeviceBuffer::release()
{
    if (ptr_ != nullptr)
        (void)hipFree(ptr_);
    ptr_ = nullptr;
    bytes_ = 0;
}

} // namespace nut
