// The flat expansion with no device allocation (mya_expand_noalloc, include/mymyr_amd.h): the same kernels and
// results as mya_expand, with the expansion's scratch (per-row counts, offsets, scan partials, status words) in a
// fixed array of device memory that the library holds for the life of the process, instead of the device scratch
// block that mya_expand grows on demand. For callers that cannot allocate device memory: tight serving loops and
// harnesses that forbid hipMalloc.
//
// The array is a file-scope __device__ variable: each device the library runs on holds its own copy, at its own
// address. The host-side name `scratch` is a stand-in, not a device address, so the address of the current device's
// copy is resolved once per device with hipGetSymbolAddress and only that pointer is handed to kernels.

#include "../../include/mymyr_amd.h"

#include "capi_internal.hpp"

#include <array>
#include <mutex>
#include <string>

using namespace mya;

namespace
{
constexpr u64 kNoallocRows = MYA_EXPAND_NOALLOC_MAX_ROWS;           // the most rows one call expands
constexpr size_t kNoallocBytes = expand_scratch_bytes(kNoallocRows);  // about 7 MiB
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kNoallocBytes];

std::mutex g_mutex;                        // guards the addresses and serializes the calls of this process
std::array<void*, kMaxDevices> g_ptr{};    // per device: the address of its copy of `scratch` (null: not resolved)

/// The current device's copy of `scratch`, resolved on the first call on that device (with the device current).
void* scratch_ptr(int dev)
{
    if (dev < 0 || dev >= kMaxDevices)
        throw std::invalid_argument("mymyr_amd: expand_noalloc: device ordinal " + std::to_string(dev) + " out of range");
    if (!g_ptr[dev])
    {
        void* p = nullptr;
        hip_check(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), "expand_noalloc: scratch address");
        if (!p)
            throw HipError("mymyr_amd: expand_noalloc: no device address for the static scratch");
        g_ptr[dev] = p;
    }
    return g_ptr[dev];
}
}  // namespace

extern "C" {

int mya_expand_noalloc(mya_task* task, const uint64_t* states, uint64_t rows, uint32_t words, const mya_expand_options* options,
                       mya_expansion* out, void* stream)
{
    return guarded([&] {
        if (!task)
            throw std::invalid_argument("mymyr_amd: expand_noalloc: null argument");
        if (rows > kNoallocRows)
            throw std::invalid_argument("mymyr_amd: expand_noalloc: " + std::to_string(rows) + " rows exceed the static scratch's " +
                                        std::to_string(kNoallocRows) + " (use mya_expand)");
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        std::unique_lock<std::mutex> lazy_lock;
        if (lazy_task(task))
            lazy_lock = std::unique_lock<std::mutex>(task->lazy_mutex);
        const TaskDev* T = nullptr;
        {
            // the task's device image must be there already: uploading it would allocate
            std::lock_guard lock(task->mutex);
            if (!task->dev.image || task->dev.device != dev)
                throw std::invalid_argument("mymyr_amd: expand_noalloc: the task has no device image on device " + std::to_string(dev) +
                                            " (one allocating call with the task, such as mya_expand of 0 rows, uploads it)");
            T = task->dev.thost.get();
        }
        std::lock_guard lock(g_mutex);
        void* block = scratch_ptr(dev);
        expand_rows({T}, nullptr, nullptr, states, rows, words, options, out, static_cast<hipStream_t>(stream), block,
                    lazy_task(task) ? task : nullptr);
    });
}

}  // extern "C"
