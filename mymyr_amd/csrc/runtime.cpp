// Device memory cache and event pool (runtime.hpp).

#include "runtime.hpp"

#include <algorithm>
#include <map>
#include <mutex>
#include <unordered_map>
#include <vector>

namespace mya
{
namespace
{
constexpr size_t kCacheMax = size_t{96} << 30;  // cached bytes per process (MI355X: 288 GB of HBM per device)

struct Block
{
    int device;
    size_t bytes;
};

/// A block freed on a stream: reusable once the event recorded after the stream's queued work has completed.
struct Pending
{
    hipEvent_t event;
    int device;
    size_t bytes;
    void* p;
};

struct Cache
{
    std::mutex mutex;
    std::unordered_map<void*, Block> live;             // every block handed out
    std::multimap<std::pair<int, size_t>, void*> idle;  // freed blocks by (device, bytes)
    std::vector<Pending> pending;                       // stream-ordered frees whose streams have not passed them yet
    size_t idle_bytes = 0;
    MemoryUsage usage;  // reserved / used bytes (held under `mutex`) and the allocation counts

    void on_reserve(size_t bytes)
    {
        usage.reserved += bytes;
        usage.reserved_high = std::max(usage.reserved_high, usage.reserved);
        ++usage.driver_allocations;
    }
    void on_use(size_t bytes)
    {
        usage.used += bytes;
        usage.used_high = std::max(usage.used_high, usage.used);
        ++usage.allocations;
    }

    void release_idle()
    {
        for (auto& [key, p] : idle)
            (void)hipFree(p);
        idle.clear();
        usage.reserved -= idle_bytes;
        idle_bytes = 0;
    }
    /// Moves every pending block whose event completed (or, with wait, every pending block) to the idle blocks.
    void collect(bool wait);
    void make_idle(int device, size_t bytes, void* p)
    {
        if (idle_bytes + bytes > kCacheMax)
            release_idle();
        if (bytes > kCacheMax)
        {
            (void)hipFree(p);
            usage.reserved -= bytes;
            return;
        }
        idle.emplace(std::make_pair(device, bytes), p);
        idle_bytes += bytes;
    }
};

Cache& cache()
{
    static Cache* c = new Cache();  // never destroyed: blocks are released with the process
    return *c;
}

std::mutex g_event_mutex;
std::vector<hipEvent_t>* g_events = new std::vector<hipEvent_t>();

void Cache::collect(bool wait)
{
    for (size_t i = 0; i < pending.size();)
    {
        const hipError_t q = wait ? hipEventSynchronize(pending[i].event) : hipEventQuery(pending[i].event);
        if (q == hipErrorNotReady)
        {
            (void)hipGetLastError();  // not an error: the stream has not reached the event yet
            ++i;
            continue;
        }
        const Pending b = pending[i];
        pending[i] = pending.back();
        pending.pop_back();
        event_release(b.event);
        make_idle(b.device, b.bytes, b.p);
    }
}
}  // namespace

void* device_alloc(size_t bytes, const char* what)
{
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    Cache& c = cache();
    {
        std::lock_guard lock(c.mutex);
        if (!c.pending.empty())
            c.collect(false);
        auto it = c.idle.find({dev, bytes});
        if (it != c.idle.end())
        {
            void* p = it->second;
            c.idle.erase(it);
            c.idle_bytes -= bytes;
            c.live.emplace(p, Block{dev, bytes});
            c.on_use(bytes);
            return p;
        }
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, bytes);
    if (e != hipSuccess)
    {
        (void)hipGetLastError();
        {
            std::lock_guard lock(c.mutex);
            c.collect(true);
            c.release_idle();
        }
        e = hipMalloc(&p, bytes);
    }
    if (e != hipSuccess)
        throw HipError(std::string("device allocation of ") + std::to_string(bytes) + " bytes for " + what + " failed: " +
                       hipGetErrorString(e));
    std::lock_guard lock(c.mutex);
    c.live.emplace(p, Block{dev, bytes});
    c.on_reserve(bytes);
    c.on_use(bytes);
    return p;
}

void device_free(void* p)
{
    // the block may still be in use by queued work on any stream of the device: wait for it, as hipFree does, before
    // the block can be handed out again (callers that know the stream use device_free_async)
    (void)hipDeviceSynchronize();
    Cache& c = cache();
    std::lock_guard lock(c.mutex);
    auto it = c.live.find(p);
    if (it == c.live.end())
    {
        (void)hipFree(p);
        return;
    }
    const Block b = it->second;
    c.live.erase(it);
    c.usage.used -= b.bytes;
    c.make_idle(b.device, b.bytes, p);
}

void device_free_async(void* p, hipStream_t stream)
{
    Cache& c = cache();
    Block b{};
    {
        std::lock_guard lock(c.mutex);
        auto it = c.live.find(p);
        if (it == c.live.end())
            b.device = -1;
        else
        {
            b = it->second;
            c.live.erase(it);
            c.usage.used -= b.bytes;
        }
    }
    if (b.device < 0)
    {
        (void)hipStreamSynchronize(stream);
        (void)hipFree(p);
        return;
    }
    // the event marks the end of the work queued on the stream so far; the block is reused only after it completed
    hipEvent_t e = event_acquire();
    if (hipEventRecord(e, stream) != hipSuccess)
    {
        (void)hipGetLastError();
        (void)hipStreamSynchronize(stream);
        event_release(e);
        std::lock_guard lock(c.mutex);
        c.make_idle(b.device, b.bytes, p);
        return;
    }
    std::lock_guard lock(c.mutex);
    c.pending.push_back(Pending{e, b.device, b.bytes, p});
}

void device_cache_release()
{
    Cache& c = cache();
    std::lock_guard lock(c.mutex);
    c.collect(true);
    c.release_idle();
}

MemoryUsage memory_usage()
{
    Cache& c = cache();
    std::lock_guard lock(c.mutex);
    return c.usage;
}

namespace
{
struct DeviceScratch
{
    std::mutex mutex;
    void* p = nullptr;
    size_t bytes = 0;
};

DeviceScratch& device_scratch_of(int dev)
{
    static std::mutex m;
    static auto* all = new std::map<int, DeviceScratch*>();  // never destroyed, as the cache
    std::lock_guard lock(m);
    DeviceScratch*& d = (*all)[dev];
    if (!d)
        d = new DeviceScratch();
    return *d;
}
}  // namespace

ScratchLease::ScratchLease(size_t bytes, const char* what)
{
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    DeviceScratch& d = device_scratch_of(dev);
    m_lock = std::unique_lock<std::mutex>(d.mutex);
    if (d.bytes < bytes)
    {
        // grown to the largest request so far, in steps of at least 1 MiB (earlier calls have drained: every user
        // synchronizes its stream before it returns)
        if (d.p)
            device_free(d.p);
        d.p = nullptr;
        d.bytes = 0;
        const size_t want = std::max<size_t>((bytes + (size_t{1} << 20) - 1) & ~((size_t{1} << 20) - 1), size_t{1} << 20);
        d.p = device_alloc(want, what);
        d.bytes = want;
    }
    m_p = static_cast<unsigned char*>(d.p);
    m_bytes = d.bytes;
}

hipEvent_t event_acquire()
{
    {
        std::lock_guard lock(g_event_mutex);
        if (!g_events->empty())
        {
            hipEvent_t e = g_events->back();
            g_events->pop_back();
            return e;
        }
    }
    hipEvent_t e = nullptr;
    hip_check(hipEventCreate(&e), "event");
    return e;
}

void event_release(hipEvent_t e)
{
    std::lock_guard lock(g_event_mutex);
    g_events->push_back(e);
}

namespace
{
constexpr size_t kPinnedBlock = 4096;
std::mutex g_pinned_mutex;
std::vector<void*>* g_pinned = new std::vector<void*>();  // never destroyed: blocks live until the process ends
}  // namespace

void* pinned_acquire(size_t bytes)
{
    if (bytes > kPinnedBlock)
        throw std::invalid_argument("mymyr_amd: pinned scalar blocks hold at most 4 KiB");
    {
        std::lock_guard lock(g_pinned_mutex);
        if (!g_pinned->empty())
        {
            void* p = g_pinned->back();
            g_pinned->pop_back();
            return p;
        }
    }
    void* p = nullptr;
    hip_check(hipHostMalloc(&p, kPinnedBlock, hipHostMallocDefault), "pinned block");
    return p;
}

void pinned_release(void* p)
{
    if (!p)
        return;
    std::lock_guard lock(g_pinned_mutex);
    g_pinned->push_back(p);
}

hipStream_t thread_stream()
{
    thread_local std::unordered_map<int, hipStream_t> streams;
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    hipStream_t& s = streams[dev];
    if (!s)
        hip_check(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "stream");
    return s;
}
}  // namespace mya
