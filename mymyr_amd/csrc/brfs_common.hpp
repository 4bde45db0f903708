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
#include <cmath>
#include <cstring>
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

/// SplitMix64 as the reference specifies it (include/mymyr/core/random.hpp:1-16, bit for bit): the state advances by
/// the golden gamma and each output is its mix64; bounded(n) is Lemire's multiply-shift with rejection; shuffle is
/// Fisher-Yates from the back (for i = n down to 2: swap a[i - 1] with a[bounded(i)]).
class SplitMix64
{
public:
    explicit SplitMix64(u64 seed) : m_state(seed) {}
    u64 next()
    {
        m_state += kGamma;
        return mix64(m_state);
    }
    u64 bounded(u64 n)
    {
        unsigned __int128 m = static_cast<unsigned __int128>(next()) * n;
        u64 low = static_cast<u64>(m);
        if (low < n)
        {
            const u64 threshold = (u64{0} - n) % n;  // 2^64 mod n
            while (low < threshold)
            {
                m = static_cast<unsigned __int128>(next()) * n;
                low = static_cast<u64>(m);
            }
        }
        return static_cast<u64>(m >> 64);
    }
    template<class T>
    void shuffle(std::vector<T>& a)
    {
        for (u64 i = a.size(); i > 1; --i)
            std::swap(a[i - 1], a[bounded(i)]);
    }

private:
    static constexpr u64 kGamma = 0x9e3779b97f4a7c15ull;
    u64 m_state;
};

/// The expansion order of BrFS layers under BrfsOptions::layers (the reference's LayerOrderer,
/// src/mymyr/search/layer_order_detail.hpp:26-200): a layer of n states (positions in id order) is reordered by the
/// kind and, with a beam, cut to its first beam_width entries. The generator persists across the layers of a search.
class LayerOrder
{
public:
    enum Kind : i32
    {
        kQueue = 0,
        kInOrder = 1,
        kReverse = 2,
        kRandomized = 3,
        kGoalCount = 4,
        kScored = 5,
    };
    explicit LayerOrder(const BrfsOptionsC& o) : m_o(o), m_rng(o.layer_seed) {}
    [[nodiscard]] bool ordered() const { return m_o.layer_kind != kQueue; }
    [[nodiscard]] bool limited() const { return ordered() && m_o.max_next_layer_states != ~u32{0}; }
    [[nodiscard]] bool ranked() const { return m_o.layer_kind == kGoalCount || m_o.layer_kind == kScored; }
    /// The positions of a layer of n states in expansion order (cut to the beam); `keys` (ranked kinds): each state's
    /// rank key, smaller first, ties by a random token (randomize_ties, drawn in position order) and then position.
    std::vector<u32> order(u32 n, const std::vector<u64>& keys)
    {
        std::vector<u32> out(n);
        for (u32 i = 0; i < n; ++i)
            out[i] = i;
        if (m_o.layer_kind == kReverse)
            std::reverse(out.begin(), out.end());
        else if (m_o.layer_kind == kRandomized)
            m_rng.shuffle(out);
        else if (ranked())
        {
            struct Ranked
            {
                u64 key, tie;
                u32 pos;
            };
            std::vector<Ranked> rk(n);
            for (u32 i = 0; i < n; ++i)
                rk[i] = {keys[i], m_o.randomize_ties ? m_rng.next() : 0, i};
            std::sort(rk.begin(), rk.end(), [](const Ranked& a, const Ranked& b) {
                return a.key != b.key ? a.key < b.key : a.tie != b.tie ? a.tie < b.tie : a.pos < b.pos;
            });
            for (u32 i = 0; i < n; ++i)
                out[i] = rk[i].pos;
        }
        if (m_o.beam_width != ~u32{0} && out.size() > m_o.beam_width)
            out.resize(m_o.beam_width);
        return out;
    }
    /// The rank key of a score: doubles ordered as unsigned integers (-inf first, +inf last; -0 as 0).
    static u64 score_key(double v)
    {
        u64 bits = 0;
        const double z = v == 0 ? 0.0 : v;
        std::memcpy(&bits, &z, sizeof(bits));
        return (bits >> 63) ? ~bits : bits | (u64{1} << 63);
    }

private:
    const BrfsOptionsC& m_o;
    SplitMix64 m_rng;
};

/// out[k] = v[ids[k] - first]: per-state bytes of a layer in its expansion order.
__global__ void k_gather_u8(const u8* __restrict__ v, const u64* __restrict__ ids, u64 first, u64 n, u8* __restrict__ out)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += static_cast<u64>(gridDim.x) * blockDim.x)
        out[i] = v[ids[i] - first];
}

/// GoalCount rank keys of rows [0, n) of W words: the task goal's unsatisfied literals (positive slots not set,
/// negative slots set; the masks hold each literal once), or their complement with prefer_less (fewest satisfied first).
__global__ void k_goal_keys(const u64* __restrict__ rows, u64 n, u32 W, const u64* __restrict__ pos, const u64* __restrict__ neg,
                            u32 prefer_less, u32* __restrict__ keys)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < n; i += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        const u64* r = rows + i * W;
        u32 unsat = 0;
        for (u32 w = 0; w < W; ++w)
            unsat += __popcll(pos[w] & ~r[w]) + __popcll(neg[w] & r[w]);
        keys[i] = prefer_less ? ~unsat : unsat;
    }
}

/// out[k] = rows[ids[k]] (W words each): a layer's rows in expansion order.
__global__ void k_gather_rows(const u64* __restrict__ rows, const u64* __restrict__ ids, u64 n, u32 W, u64* __restrict__ out)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < n * W; i += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        const u64 k = i / W, w = i % W;
        out[i] = rows[ids[k] * W + w];
    }
}

/// The device buffers of an observed search's per-state events (BrfsOptionsC::observed): per candidate of a batch its
/// probe result, its state's id and whether it entered the store. All null when the search is not observed.
struct EventBuffers
{
    bool on = false;
    u64* cand_slot = nullptr;
    i64* ids = nullptr;
    u8* is_new = nullptr;
    void init(bool observed, u64 chunk, Buffers& b)
    {
        on = observed;
        if (!on)
            return;
        cand_slot = b.alloc<u64>(chunk, "event probe results");
        ids = b.alloc<i64>(chunk, "event ids");
        is_new = b.alloc<u8>(chunk, "event new flags");
    }
};

/// A confirmed batch's events in the reference's order (src/mymyr/search/brfs.cpp:335-372): per parent p < np its
/// on_expand, then per successor of it (candidates in order; cand_parent[j] is j's parent) its on_generate and, for a
/// blocked one (hit[j]), its on_prune. ids [m] and is_new [m] come from the device; label(j, &schema, &binding,
/// &arity) gives a candidate's action and row(j, parent row) its successor row (host, W words).
template<class Label, class Row>
void emit_batch(const BrfsOptionsC& o, u32 W, u64 np, const std::vector<u64>& parent_rows, const std::vector<u64>& parent_ids,
                u64 m, const std::vector<u32>& cand_parent, const std::vector<i64>& ids, const std::vector<u8>& is_new,
                const std::vector<u8>& hit, Label&& label, Row&& row)
{
    u64 j = 0;
    for (u64 p = 0; p < np; ++p)
    {
        const u64* prow = parent_rows.data() + p * W;
        const u64 pid = parent_ids[p];
        if (o.on_expand)
            o.on_expand(pid, prow, W);
        for (; j < m && cand_parent[j] == p; ++j)
        {
            u32 schema = 0, arity = 0;
            const i32* binding = nullptr;
            label(j, &schema, &binding, &arity);
            const u64* crow = row(j, prow);
            const bool blocked = !hit.empty() && hit[j];
            if (o.on_generate)
                o.on_generate(pid, schema, binding, arity, blocked || ids[j] < 0 ? ~u64{0} : static_cast<u64>(ids[j]), crow, W,
                              !blocked && is_new[j] != 0);
            if (blocked && o.on_prune)
                o.on_prune(pid, schema, binding, arity, crow, W);
        }
    }
}

/// Device to host copy of n elements on the stream (synchronous).
template<class T>
std::vector<T> to_host(const T* d, u64 n, hipStream_t stream)
{
    std::vector<T> h(n);
    if (n)
    {
        hip_check(hipMemcpyAsync(h.data(), d, n * sizeof(T), hipMemcpyDeviceToHost, stream), "event copy");
        hip_check(hipStreamSynchronize(stream), "event copy");
    }
    return h;
}

/// A device buffer grown to the largest request of a search, freed in the order of its stream.
template<class T>
struct GrowBuf
{
    hipStream_t stream;
    T* p = nullptr;
    u64 cap = 0;
    explicit GrowBuf(hipStream_t s) : stream(s) {}
    GrowBuf(const GrowBuf&) = delete;
    GrowBuf& operator=(const GrowBuf&) = delete;
    T* get(u64 n, const char* what)
    {
        if (n > cap)
        {
            if (p)
                dev_free_async(p, stream);
            p = dev_alloc<T>(std::max<u64>(n, 1), what);
            cap = std::max<u64>(n, 1);
        }
        return p;
    }
    ~GrowBuf()
    {
        if (p)
            dev_free_async(p, stream);
    }
};

/// The expansion order of an ordered layer (BrfsOptions::layers): `ids` (host and device) holds the layer's state ids
/// in the order they are expanded, cut to the beam, and `rows` their rows gathered in that order, so that the
/// drivers expand positions [0, ids.size()) of it as they expand a layer of the arena. The start layer is never
/// reordered (src/mymyr/search/brfs.cpp:316-318).
struct LayerRows
{
    explicit LayerRows(hipStream_t s) : d_ids(s), rows(s), keys(s), masks(s) {}
    std::vector<u64> ids;
    GrowBuf<u64> d_ids;
    GrowBuf<u64> rows;
    GrowBuf<u32> keys;
    GrowBuf<u64> masks;

    /// Orders the layer [first, first + n) of the arena (W words per row) and gathers its rows.
    void order(LayerOrder& lo, const BrfsOptionsC& o, const CompiledTask& task, const u64* arena, u64 first, u64 n, u32 W, hipStream_t stream)
    {
        if (n > 0xFFFFFFFFull)
            throw std::length_error("mymyr_amd: brfs: an ordered layer of more than 2^32 - 1 states");
        std::vector<u64> key;
        if (o.layer_kind == LayerOrder::kGoalCount && n > 0)
        {
            // the task's goal (also under another search goal), each literal once (layer_ordering.hpp:93-96)
            std::vector<u64> m(2 * static_cast<size_t>(W), 0);
            for (u32 sl : task.goal_pos)
                if (sl < 64 * W)
                    m[sl >> 6] |= u64{1} << (sl & 63);
            for (u32 sl : task.goal_neg)
                if (sl < 64 * W)
                    m[W + (sl >> 6)] |= u64{1} << (sl & 63);
            u64* dm = masks.get(2 * W, "goal count masks");
            hip_check(hipMemcpyAsync(dm, m.data(), m.size() * sizeof(u64), hipMemcpyHostToDevice, stream), "goal count masks");
            u32* dk = keys.get(n, "goal count keys");
            hipLaunchKernelGGL(k_goal_keys, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(n, 256), 4096))), dim3(256), 0, stream,
                               arena + first * W, n, W, dm, dm + W, o.prefer_more_satisfied_goals ? 0u : 1u, dk);
            launch_check("goal count keys");
            std::vector<u32> hk(n);
            hip_check(hipMemcpyAsync(hk.data(), dk, n * sizeof(u32), hipMemcpyDeviceToHost, stream), "goal count keys");
            hip_check(hipStreamSynchronize(stream), "goal count keys");
            key.assign(hk.begin(), hk.end());
        }
        else if (o.layer_kind == LayerOrder::kScored && n > 0)
        {
            // one call of the scorer per layer with the layer's states in generation order (layer_ordering.hpp:98-104)
            std::vector<u64> hr(n * W);
            hip_check(hipMemcpyAsync(hr.data(), arena + first * W, hr.size() * sizeof(u64), hipMemcpyDeviceToHost, stream), "layer rows");
            hip_check(hipStreamSynchronize(stream), "layer rows");
            std::vector<double> sc(n, 0.0);
            o.scorer(hr.data(), n, W, sc.data());
            key.resize(n);
            for (u64 i = 0; i < n; ++i)
            {
                if (std::isnan(sc[i]))
                    throw std::invalid_argument("mymyr: a layer score is NaN");
                key[i] = LayerOrder::score_key(sc[i]);
            }
        }
        const std::vector<u32> pos = lo.order(static_cast<u32>(n), key);
        ids.resize(pos.size());
        for (size_t k = 0; k < pos.size(); ++k)
            ids[k] = first + pos[k];
        gather(arena, W, stream);
    }
    /// The ordered rows from the arena again (after the arena's rows were widened).
    void gather(const u64* arena, u32 W, hipStream_t stream)
    {
        const u64 k = ids.size();
        u64* di = d_ids.get(k, "layer order");
        u64* dr = rows.get(k * W, "ordered layer rows");
        if (k == 0)
            return;
        hip_check(hipMemcpyAsync(di, ids.data(), k * sizeof(u64), hipMemcpyHostToDevice, stream), "layer order");
        hipLaunchKernelGGL(k_gather_rows, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(k * W, 256), 8192))), dim3(256), 0, stream, arena,
                           di, k, W, dr);
        launch_check("ordered layer rows");
    }
};

}  // namespace
}  // namespace mya
