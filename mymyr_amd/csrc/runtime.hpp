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

template<class T>
T* dev_alloc(size_t count, const char* what)
{
    if (count == 0)
        count = 1;
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, count * sizeof(T));
    if (e != hipSuccess)
        throw HipError(std::string("device allocation of ") + std::to_string(count * sizeof(T)) + " bytes for " + what +
                       " failed: " + hipGetErrorString(e));
    return static_cast<T*>(p);
}

inline void dev_free(void* p)
{
    if (p)
        (void)hipFree(p);
}

/// Launch check: the error of the last launch, if any.
inline void launch_check(const char* what) { hip_check(hipGetLastError(), what); }

constexpr unsigned blocks_for(unsigned long long n, unsigned block)
{
    return static_cast<unsigned>((n + block - 1) / block);
}
}  // namespace mya
