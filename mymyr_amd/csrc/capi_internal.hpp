#pragma once
// Internals shared by the C-ABI translation units: the opaque handle types and the exception guard.

#include "brfs.hpp"
#include "state_set.hpp"
#include "task.hpp"

#include <hip/hip_runtime.h>

#include <atomic>
#include <exception>
#include <memory>
#include <mutex>
#include <string>

namespace mya
{
void set_error(const std::string& m);

struct TaskDev;

/// A task's device image, uploaded on first device use, plus the pointer table into it (host and device copies).
struct DeviceTask
{
    u64* image = nullptr;
    u64 words = 0;
    int device = -1;
    std::unique_ptr<TaskDev> thost;  // host copy
};

template<class F>
int guarded(F&& f)
{
    try
    {
        f();
        return 0;
    }
    catch (const std::exception& e)
    {
        set_error(e.what());
    }
    catch (...)
    {
        set_error("mymyr_amd: unknown error");
    }
    return -1;
}
}  // namespace mya

struct mya_task
{
    std::unique_ptr<mya::CompiledTask> compiled;
    mya::DeviceTask dev;
    std::mutex mutex;
    mya::BrfsCache brfs;  // the BrFS's device tables of the task's ground actions
};

namespace mya
{
const DeviceTask& device_task(mya_task* t);
}

/// A state set handle; mya_hashset_free drops the creator's reference and every exported rows tensor holds another.
struct mya_hashset
{
    mya::StateSet set;
    std::atomic<int> refs{1};
};

namespace mya
{
void hashset_unref(mya_hashset* h);
}
