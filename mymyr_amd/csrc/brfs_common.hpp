#pragma once
// Pieces shared by the device BrFS drivers (brfs.hip over ground actions, brfs_wide.hip over the lifted expansion): the
// drivers' device scalars and small kernels (chunk ends, goal-flag sums and searches, the fingerprint), owned device
// buffers, and HIP-event timing of kernel classes. Included by one driver translation unit each; everything here has
// internal linkage.

#include "brfs.hpp"
#include "device_common.hpp"
#include "runtime.hpp"
#include "scan.hpp"
#include "state_set_device.hpp"

#include <algorithm>
#include <chrono>
#include <stdexcept>
#include <vector>

namespace mya
{
namespace
{
// The chunk end: the largest parent p in (p0, hi] whose first successor offset offsets[p * stride] <= bound, at least
// p0 + 1 (one parent's successors always fit). out[0] = p, out[1] = offsets[p * stride].
__global__ void k_chunk_end(const u64* __restrict__ offsets, u32 stride, u64 p0, u64 hi, u64 bound, u64* __restrict__ out)
{
    u64 a = p0 + 1, b = hi + 1;  // the first parent in [p0 + 1, hi + 1) past the bound
    while (a < b)
    {
        const u64 mid = a + (b - a) / 2;
        if (offsets[mid * stride] <= bound)
            a = mid + 1;
        else
            b = mid;
    }
    const u64 p = a - 1 < p0 + 1 ? p0 + 1 : a - 1;
    out[0] = p;
    out[1] = offsets[p * stride];
}

// The driver's scalars that a synchronization reads, gathered in one launch: the set's current size and status, and
// (optional) a counted block's offset total.
__global__ void k_gather_small(u64* __restrict__ small, int size_at, const u64* __restrict__ size_now, int status_at,
                               const u32* __restrict__ status, int total_at, const u64* __restrict__ total)
{
    small[size_at] = *size_now;
    small[status_at] = *status;
    if (total)
        small[total_at] = *total;
}

__global__ void k_sum_u8(const u8* __restrict__ v, u64 n, u64* __restrict__ out)
{
    u64 s = 0;
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += static_cast<u64>(gridDim.x) * blockDim.x)
        s += v[i];
    s = wave_sum64(s);
    if (lane_id() == 0 && s)
        atomicAdd(reinterpret_cast<unsigned long long*>(out), static_cast<unsigned long long>(s));
}

__global__ void k_first_u8(const u8* __restrict__ v, u64 n, u64* __restrict__ out)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += static_cast<u64>(gridDim.x) * blockDim.x)
        if (v[i])
            atomicMin(reinterpret_cast<unsigned long long*>(out), static_cast<unsigned long long>(i));
}

__global__ void k_fingerprint(const u64* __restrict__ arena, u64 n, u32 W, const u64* __restrict__ slot_cid, u64* __restrict__ out)
{
    u64 acc = 0;
    for (u64 id = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; id < n; id += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        const u64* row = arena + id * W;
        u64 ch = 0;
        for (u32 w = 0; w < W; ++w)
        {
            u64 x = row[w];
            while (x)
            {
                const u32 s = w * 64 + static_cast<u32>(__builtin_ctzll(x));
                x &= x - 1;
                const u64 cid = slot_cid ? slot_cid[s] : s;
                ch ^= mix64(cid + 0x1234567ULL);
            }
        }
        acc ^= mix64(id * 0x9E3779B97F4A7C15ULL ^ ch);
    }
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1)
        acc ^= __shfl_xor(acc, d, kWave);
    if (lane_id() == 0 && acc)
        atomicXor(reinterpret_cast<unsigned long long*>(out), static_cast<unsigned long long>(acc));
}

__global__ void k_set_u64(u64* p, u64 v) { *p = v; }

constexpr int kSmall = 16;  // device scalars of the driver

/// A search's device buffers, freed in the order of its stream: a freed block is reused only once the work queued on
/// the stream before the free has completed, so ending a search waits for nothing and stalls no other stream.
struct Buffers
{
    explicit Buffers(hipStream_t s) : stream(s) {}
    Buffers(const Buffers&) = delete;
    Buffers& operator=(const Buffers&) = delete;
    hipStream_t stream;
    std::vector<void*> owned;
    u64* host = nullptr;  // pinned mirror of the device scalars
    template<class T>
    T* alloc(size_t n, const char* what)
    {
        T* p = dev_alloc<T>(n, what);
        owned.push_back(p);
        return p;
    }
    /// Frees one buffer of alloc() before the others (stream-ordered).
    void release(void* p)
    {
        const auto it = std::find(owned.begin(), owned.end(), p);
        if (it == owned.end())
            return;
        owned.erase(it);
        dev_free_async(p, stream);
    }
    ~Buffers()
    {
        for (void* p : owned)
            dev_free_async(p, stream);
        if (host)
        {
            // the pinned scalar block is handed to the next search only after this one's copies into it have landed
            (void)hipStreamSynchronize(stream);
            pinned_release(host);
        }
    }
};

using Clock = std::chrono::steady_clock;

/// The blocked states of a search on the device (BlockedView): the rows padded to the set's row width W, duplicates
/// dropped, the table built here with the state set's table hash (set_hash), slot and tag.
inline BlockedView upload_blocked(const std::vector<u64>& rows, u32 task_words, u32 W, u64 batch, Buffers& b, hipStream_t stream)
{
    const u64 k = task_words ? rows.size() / task_words : 0;
    if (k == 0)
        return BlockedView{};
    if (task_words > W)
        throw std::invalid_argument("mymyr_amd: brfs: blocked rows wider than the search's rows");
    std::vector<u64> uniq;
    std::vector<u64> table(2 * k + 2, 0);
    const u64 cap = table.size();
    std::vector<u64> row(W);
    for (u64 i = 0; i < k; ++i)
    {
        std::fill(row.begin(), row.end(), 0);
        std::copy(rows.begin() + i * task_words, rows.begin() + (i + 1) * task_words, row.begin());
        const u64 h = set_hash(row.data(), W);
        const u64 tag = h >> 32;
        u64 slot = slot_of_hash(h, cap);
        bool dup = false;
        for (; table[slot]; slot = slot + 1 == cap ? 0 : slot + 1)
            if ((table[slot] >> 32) == tag &&
                std::equal(row.begin(), row.end(), uniq.begin() + (static_cast<u32>(table[slot]) - 1) * W))
            {
                dup = true;
                break;
            }
        if (dup)
            continue;
        table[slot] = (tag << 32) | (uniq.size() / W + 1);
        uniq.insert(uniq.end(), row.begin(), row.end());
    }
    BlockedView v{};
    u64* d_table = b.alloc<u64>(cap, "blocked table");
    u64* d_rows = b.alloc<u64>(uniq.size(), "blocked rows");
    hip_check(hipMemcpyAsync(d_table, table.data(), cap * sizeof(u64), hipMemcpyHostToDevice, stream), "blocked table");
    hip_check(hipMemcpyAsync(d_rows, uniq.data(), uniq.size() * sizeof(u64), hipMemcpyHostToDevice, stream), "blocked rows");
    hip_check(hipStreamSynchronize(stream), "blocked states");
    v.table = d_table;
    v.capacity = cap;
    v.rows = d_rows;
    v.words = W;
    v.hit = b.alloc<u8>(batch, "blocked flags");
    return v;
}

/// The AnyOf goals of the options on the device (AnyOfDev{} when the task's goal decides).
inline AnyOfDev upload_any_of(const BrfsOptionsC& o, Buffers& b, hipStream_t stream)
{
    AnyOfDev d{};
    if (!o.any_of)
        return d;
    std::vector<u32> off{0}, slots;
    for (size_t k = 0; k < o.goal_pos.size(); ++k)
    {
        slots.insert(slots.end(), o.goal_pos[k].begin(), o.goal_pos[k].end());
        off.push_back(static_cast<u32>(slots.size()));
        slots.insert(slots.end(), o.goal_neg[k].begin(), o.goal_neg[k].end());
        off.push_back(static_cast<u32>(slots.size()));
    }
    u32* d_off = b.alloc<u32>(off.size(), "goal offsets");
    u32* d_slots = b.alloc<u32>(std::max<size_t>(1, slots.size()), "goal slots");
    hip_check(hipMemcpyAsync(d_off, off.data(), off.size() * sizeof(u32), hipMemcpyHostToDevice, stream), "goal offsets");
    if (!slots.empty())
        hip_check(hipMemcpyAsync(d_slots, slots.data(), slots.size() * sizeof(u32), hipMemcpyHostToDevice, stream), "goal slots");
    hip_check(hipStreamSynchronize(stream), "goals");
    d.off = d_off;
    d.slots = d_slots;
    d.count = static_cast<u32>(o.goal_pos.size());
    d.any = 1;
    return d;
}

/// The start state as a row of W words (BrfsOptionsC::start, else the task's initial state).
inline std::vector<u64> start_row(const CompiledTask& task, const BrfsOptionsC& o, u32 W)
{
    const std::vector<u64>& s = o.start.empty() ? task.initial : o.start;
    std::vector<u64> row(W, 0);
    std::copy(s.begin(), s.begin() + std::min<size_t>(s.size(), W), row.begin());
    return row;
}

/// max_seconds, the cancellation flag and the observer's on_progress (the reference's Control::check and keep_going,
/// src/mymyr/search/brfs.cpp:137-181): checked by the drivers before every batch with the counts so far; `why` keeps
/// the first reason (OutOfTime or Cancelled).
struct Halt
{
    const BrfsOptionsC& o;
    Clock::time_point t0, deadline;
    u64 next_progress;  // on_progress is asked once this many states were expanded
    i32 why = 0;
    Halt(const BrfsOptionsC& opt, Clock::time_point start)
        : o(opt), t0(start), next_progress(std::max<u64>(1, opt.progress_interval))
    {
        const double s = std::min(std::max(0.0, o.max_seconds), 1e9);
        deadline = t0 + std::chrono::duration_cast<Clock::duration>(std::chrono::duration<double>(s));
    }
    bool check(u64 expanded, u64 generated, u64 states)
    {
        if (why)
            return true;
        if (o.timed && Clock::now() >= deadline)
            why = kOutOfTime;
        else if (o.cancel && *o.cancel)
            why = kCancelled;
        else if (o.on_progress && expanded >= next_progress)
        {
            next_progress = expanded + std::max<u64>(1, o.progress_interval);
            if (!o.on_progress(expanded, generated, states, std::chrono::duration<double>(Clock::now() - t0).count()))
                why = kCancelled;
        }
        return why != 0;
    }
};

/// HIP-event timing of kernel classes on one stream; durations are read once the stream has drained.
class Timers
{
public:
    Timers(bool on, hipStream_t s, BrfsResultC& r) : m_on(on), m_s(s), m_r(r) {}
    ~Timers()
    {
        for (auto& e : m_ev)
        {
            event_release(e.a);
            event_release(e.b);
        }
    }
    void begin(int k)
    {
        if (!m_on)
            return;
        Pair p{k, nullptr, nullptr};
        p.a = event_acquire();
        p.b = event_acquire();
        hip_check(hipEventRecord(p.a, m_s), "event");
        m_ev.push_back(p);
    }
    void end(int k, u64 bytes)
    {
        m_r.kernel_bytes[k] += bytes;
        m_r.kernel_launches[k] += 1;
        if (!m_on)
            return;
        hip_check(hipEventRecord(m_ev.back().b, m_s), "event");
    }
    void bytes(int k, u64 b) { m_r.kernel_bytes[k] += b; }
    /// Adds the durations of the recorded pairs (the stream must have drained).
    void collect()
    {
        for (auto& e : m_ev)
        {
            float ms = 0;
            hip_check(hipEventElapsedTime(&ms, e.a, e.b), "event time");
            m_r.kernel_ms[e.k] += ms;
            event_release(e.a);
            event_release(e.b);
        }
        m_ev.clear();
    }

private:
    struct Pair
    {
        int k;
        hipEvent_t a, b;
    };
    bool m_on;
    hipStream_t m_s;
    BrfsResultC& m_r;
    std::vector<Pair> m_ev;
};

}  // namespace
}  // namespace mya
