#pragma once
// HIP runtime helpers: checked calls, device allocations, and the thread-local error message of the C-ABI.

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <mutex>
#include <stdexcept>
#include <string>

namespace mya
{
using u64 = std::uint64_t;
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
/// Returns a block to the cache after waiting for the device (for frees whose last stream is unknown).
void device_free(void* p);
/// Returns a block to the cache in stream order: an event recorded on `stream` marks the work queued so far, and the
/// block is handed out again only once that event has completed (no device-wide wait). The block must not be used by
/// work queued later on other streams.
void device_free_async(void* p, hipStream_t stream);
/// Frees every cached block (all devices).
void device_cache_release();

/// Process-wide device memory figures of the cache (the reference's PoolUsage, include/mymyr/cuda/runtime.hpp:140-146):
/// bytes held from the driver (handed out, idle or awaiting a stream-ordered free), bytes handed out, their high-water
/// marks, and how many blocks the library has handed out (cache hits included) and taken from the driver.
struct MemoryUsage
{
    u64 reserved = 0;
    u64 used = 0;
    u64 reserved_high = 0;
    u64 used_high = 0;
    u64 allocations = 0;
    u64 driver_allocations = 0;
};
MemoryUsage memory_usage();

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

inline void dev_free_async(void* p, hipStream_t stream)
{
    if (p)
        device_free_async(p, stream);
}

/// Exclusive use of the current device's persistent scratch block for the lifetime of the lease, grown to at least
/// `bytes` (the block is kept between calls: synchronous entry points that need per-call device scratch allocate
/// nothing once it is large enough). The lease holds the device's scratch lock, so calls using it are serialized; a
/// holder must have drained its work on the block (synchronized its stream) before the lease ends.
class ScratchLease
{
public:
    ScratchLease(size_t bytes, const char* what);
    ScratchLease(const ScratchLease&) = delete;
    ScratchLease& operator=(const ScratchLease&) = delete;
    /// The whole block (256-byte aligned, at least the requested bytes).
    void* base() const { return m_p; }
    /// The next `count` elements of T from the block (aligned to 256 bytes).
    template<class T>
    T* take(size_t count)
    {
        m_used = (m_used + 255) & ~size_t{255};
        T* p = reinterpret_cast<T*>(m_p + m_used);
        m_used += std::max<size_t>(count, 1) * sizeof(T);
        if (m_used > m_bytes)
            throw std::logic_error("mymyr_amd: scratch lease overrun");
        return p;
    }

private:
    std::unique_lock<std::mutex> m_lock;
    unsigned char* m_p = nullptr;
    size_t m_bytes = 0;
    size_t m_used = 0;
};

/// Bytes a lease needs for the given element counts of T (each aligned to 256 bytes).
template<class T>
constexpr size_t scratch_bytes(size_t count)
{
    return ((count == 0 ? 1 : count) * sizeof(T) + 255) & ~size_t{255};
}

/// HIP events from a process-wide pool (created once, reused).
hipEvent_t event_acquire();
void event_release(hipEvent_t e);

/// Pinned host blocks of at most 4 KiB from a process-wide pool (hipHostMalloc once per block, reused): the drivers'
/// scalar readbacks take one per call without pinning and unpinning host memory each time.
void* pinned_acquire(size_t bytes);
void pinned_release(void* p);

/// A non-blocking stream of the current device for the calling thread (created on first use, kept until the process
/// ends): a synchronous driver runs on it without creating and destroying a stream per call.
hipStream_t thread_stream();

/// Launch check: the error of the last launch, if any.
inline void launch_check(const char* what) { hip_check(hipGetLastError(), what); }

constexpr unsigned blocks_for(unsigned long long n, unsigned block)
{
    return static_cast<unsigned>((n + block - 1) / block);
}
}  // namespace mya
