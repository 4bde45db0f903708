// Device memory cache and event pool (runtime.hpp).

#include "runtime.hpp"

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

struct Cache
{
    std::mutex mutex;
    std::unordered_map<void*, Block> live;             // every block handed out
    std::multimap<std::pair<int, size_t>, void*> idle;  // freed blocks by (device, bytes)
    size_t idle_bytes = 0;

    void release_idle()
    {
        for (auto& [key, p] : idle)
            (void)hipFree(p);
        idle.clear();
        idle_bytes = 0;
    }
};

Cache& cache()
{
    static Cache* c = new Cache();  // never destroyed: blocks are released with the process
    return *c;
}

std::mutex g_event_mutex;
std::vector<hipEvent_t>* g_events = new std::vector<hipEvent_t>();
}  // namespace

void* device_alloc(size_t bytes, const char* what)
{
    int dev = 0;
    hip_check(hipGetDevice(&dev), "hipGetDevice");
    Cache& c = cache();
    {
        std::lock_guard lock(c.mutex);
        auto it = c.idle.find({dev, bytes});
        if (it != c.idle.end())
        {
            void* p = it->second;
            c.idle.erase(it);
            c.idle_bytes -= bytes;
            c.live.emplace(p, Block{dev, bytes});
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
            c.release_idle();
        }
        e = hipMalloc(&p, bytes);
    }
    if (e != hipSuccess)
        throw HipError(std::string("device allocation of ") + std::to_string(bytes) + " bytes for " + what + " failed: " +
                       hipGetErrorString(e));
    std::lock_guard lock(c.mutex);
    c.live.emplace(p, Block{dev, bytes});
    return p;
}

void device_free(void* p)
{
    // the block may still be in use by queued work on any stream of the device: wait for it, as hipFree does, before
    // the block can be handed out again
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
    if (c.idle_bytes + b.bytes > kCacheMax)
        c.release_idle();
    if (b.bytes > kCacheMax)
    {
        (void)hipFree(p);
        return;
    }
    c.idle.emplace(std::make_pair(b.device, b.bytes), p);
    c.idle_bytes += b.bytes;
}

void device_cache_release()
{
    Cache& c = cache();
    std::lock_guard lock(c.mutex);
    c.release_idle();
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
}  // namespace mya
