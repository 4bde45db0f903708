#pragma once
// Internals shared by the C-ABI translation units: the opaque handle types and the exception guard.

#include "brfs.hpp"
#include "runtime.hpp"
#include "scan.hpp"
#include "state_set.hpp"
#include "task.hpp"

#include <hip/hip_runtime.h>

#include <atomic>
#include <exception>
#include <memory>
#include <mutex>
#include <string>
#include <vector>

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
    u64* missing = nullptr;          // lazy slots: the successor kernels' bitmap of added atoms without a slot
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
    // lazy slots: held for the whole of a search, expansion or successor listing, which intern atoms into the task
    std::mutex lazy_mutex;
};

struct mya_env;
struct mya_expand_options;
struct mya_expansion;

namespace mya
{
const DeviceTask& device_task(mya_task* t);

/// Lazy slots: interns the atoms the device bitmap holds (ascending canonical id), uploads the changed words of the task's
/// image, refreshes its pointer table (device_task(t).thost) and clears the bitmap; synchronizes `s`. Returns whether
/// any atom was interned. The caller holds t->lazy_mutex.
bool resolve_missing(mya_task* t, hipStream_t s);

/// Whether the task has lazy atom slots.
inline bool lazy_task(const mya_task* t) { return t->compiled->mode == AtomMode::Lazy; }

/// The device scratch of one flat expansion of n rows, carved from one block: per-row counts, no-op counts and kept
/// counts, offsets before and after dropping no-ops, the scans' scratch, and two status words.
struct ExpandScratch
{
    u32* counts;
    u32* noops;
    u32* kept;
    u64* pre;
    u64* fin;
    u64* scan;
    u32* words_status;  // [0] words needed, [1] status
};

constexpr size_t expand_scratch_bytes(u64 n)
{
    return 3 * scratch_bytes<u32>(n) + 2 * scratch_bytes<u64>(n + 1) + scratch_bytes<u64>(scan_scratch_words(n)) + scratch_bytes<u32>(2);
}

/// Carves the scratch of an expansion of n rows from a block of at least expand_scratch_bytes(n) bytes (256-aligned).
ExpandScratch carve_expand_scratch(void* block, u64 n);

/// The flat expansion of rows over instances `inst` (one: batch order; several: grouped by instance with `env`'s
/// scratch and the rows' task ids). `block` (device, at least expand_scratch_bytes(max(rows, 1)) bytes) holds the
/// expansion's scratch; the call synchronizes the stream before it returns, so the block is free again then.
/// `lazy`: the one instance's task when it has lazy slots (its atoms are interned between repeats of the successor
/// pass; the caller holds its lazy_mutex), else null.
void expand_rows(const std::vector<const TaskDev*>& inst, mya_env* env, const int32_t* task_ids, const uint64_t* states, uint64_t rows,
                 uint32_t words, const mya_expand_options* options, mya_expansion* out, hipStream_t stream, void* block,
                 mya_task* lazy = nullptr);
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
