#pragma once
// HIP runtime helpers: checked calls, device allocations, and the thread-local error message of the C-ABI.

#include <hip/hip_runtime.h>

#include <stdexcept>
#include <string>

namespace mya
{
struct HipError : std::runtime_error
{
    using std::runtime_error::runtime_error;
};

inline void hip_check(hipError_t e, const char* what)
{
    if (e != hipSuccess)
        throw HipError(std::string(what) + ": " + hipGetErrorString(e));
}

/// Device memory through a per-device cache of freed blocks (runtime.cpp): a freed block is kept for a later allocation
/// of the same size on the same device (repeated searches and env pools reuse their buffers without hipMalloc / hipFree);
/// the cache holds at most a fixed share of device memory and is released when an allocation fails.
void* device_alloc(size_t bytes, const char* what);
void device_free(void* p);
/// Frees every cached block (all devices).
void device_cache_release();

template<class T>
T* dev_alloc(size_t count, const char* what)
{
    if (count == 0)
        count = 1;
    return static_cast<T*>(device_alloc(count * sizeof(T), what));
}

inline void dev_free(void* p)
{
    if (p)
        device_free(p);
}

/// HIP events from a process-wide pool (created once, reused).
hipEvent_t event_acquire();
void event_release(hipEvent_t e);

/// Launch check: the error of the last launch, if any.
inline void launch_check(const char* what) { hip_check(hipGetLastError(), what); }

constexpr unsigned blocks_for(unsigned long long n, unsigned block)
{
    return static_cast<unsigned>((n + block - 1) / block);
}
}  // namespace mya
