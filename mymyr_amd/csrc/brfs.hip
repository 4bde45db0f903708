// Device BrFS over ground actions (brfs.hpp). One thread per parent state: the parent row sits in LDS (transposed,
// conflict-free per lane) and in registers; the action loop is wave-uniform, so action records come through scalar
// loads. Per layer chunk: count -> exclusive scan -> generate (rows, hashes, parent, action) -> probe -> rank ->
// compact, all on one stream; the host reads a handful of counters per chunk.

#include "brfs.hpp"
#include "runtime.hpp"
#include "scan.hpp"
#include "state_set.hpp"

#include <algorithm>
#include <chrono>
#include <cstring>

namespace mya
{
namespace
{
constexpr int kGB = 128;  // threads per block of the ground kernels

struct GroundDev
{
    const u32* meta;
    const u32* off;
    const u32* slots;
    const u32* dom_off;  // witness pruning: dominators of each action (null: none)
    const u32* dom;
    u32 num;
};

struct GoalDev
{
    const u32* pos;
    const u32* neg;
    u32 npos, nneg;
    u32 unsat;
};

template<int W>
__device__ __forceinline__ bool lds_bit(const u64 (*st)[kGB], u32 slot)
{
    return (st[slot >> 6][threadIdx.x] >> (slot & 63)) & 1;
}

template<int W>
__device__ __forceinline__ bool applicable(const u64 (*st)[kGB], const u32* __restrict__ slots, u32 m, u32 o)
{
    const u32 npos = m & 0xFF, nneg = (m >> 8) & 0xFF;
    for (u32 i = 0; i < npos; ++i)
        if (!lds_bit<W>(st, slots[o + i]))
            return false;
    for (u32 i = 0; i < nneg; ++i)
        if (lds_bit<W>(st, slots[o + npos + i]))
            return false;
    return true;
}

/// Whether action a is a successor: applicable, and (witness pruning) no dominator is.
template<int W>
__device__ __forceinline__ bool emitted(const u64 (*st)[kGB], const GroundDev& g, u32 a, u32 m, u32 o)
{
    if (!applicable<W>(st, g.slots, m, o))
        return false;
    if (g.dom_off)
        for (u32 k = g.dom_off[a], e = g.dom_off[a + 1]; k < e; ++k)
        {
            const u32 d = g.dom[k];
            if (applicable<W>(st, g.slots, g.meta[d], g.off[d]))
                return false;
        }
    return true;
}

template<int W>
__global__ __launch_bounds__(kGB) void k_ground_count(const u64* __restrict__ arena, u64 first, u32 n, GroundDev g, GoalDev goal,
                                                     u32* __restrict__ counts, u8* __restrict__ goal_flags)
{
    __shared__ u64 st[W][kGB];
    const u32 t = blockIdx.x * kGB + threadIdx.x;
    const bool valid = t < n;
    const u64* row = arena + (first + t) * W;
#pragma unroll
    for (int w = 0; w < W; ++w)
        st[w][threadIdx.x] = valid ? row[w] : 0;
    bool gl = !goal.unsat;
    for (u32 i = 0; i < goal.npos; ++i)
        gl = gl && lds_bit<W>(st, goal.pos[i]);
    for (u32 i = 0; i < goal.nneg; ++i)
        gl = gl && !lds_bit<W>(st, goal.neg[i]);
    u32 cnt = 0;
    for (u32 a = 0; a < g.num; ++a)
        cnt += emitted<W>(st, g, a, g.meta[a], g.off[a]) ? 1u : 0u;
    if (valid)
    {
        counts[t] = cnt;
        goal_flags[t] = gl ? 1 : 0;
    }
}

template<int W>
__device__ __forceinline__ u64 hash_fixed(const u64 (&v)[W])
{
    u32 n = W;
#pragma unroll
    for (int i = W - 1; i >= 0; --i)
        if (n == static_cast<u32>(i + 1) && v[i] == 0)
            n = i;
    u64 h = kHashSeed ^ (static_cast<u64>(n) * kHashP1);
#pragma unroll
    for (int i = 0; i < W; i += 2)
    {
        if (static_cast<u32>(i + 1) < n)
            h = mulfold(h ^ v[i] ^ kHashP1, v[i + 1] ^ kHashP2);
        else if (static_cast<u32>(i) < n)
            h = mulfold(h ^ v[i] ^ kHashP1, kHashP2);
    }
    return mix64(h);
}

// Writes the successors of parents [first, first + n) at candidate positions offsets[t] - cand_base.
template<int W>
__global__ __launch_bounds__(kGB) void k_ground_generate(const u64* __restrict__ arena, u64 first, u32 n, GroundDev g,
                                                        const u64* __restrict__ offsets, u64 cand_base, u64* __restrict__ cand,
                                                        u64* __restrict__ cand_hash, u32* __restrict__ cand_parent,
                                                        u32* __restrict__ cand_action)
{
    __shared__ u64 st[W][kGB];
    const u32 t = blockIdx.x * kGB + threadIdx.x;
    const bool valid = t < n;
    const u64* row = arena + (first + t) * W;
    u64 r[W];
#pragma unroll
    for (int w = 0; w < W; ++w)
    {
        r[w] = valid ? row[w] : 0;
        st[w][threadIdx.x] = r[w];
    }
    u64 k = valid ? offsets[t] - cand_base : 0;
    const u32 parent = static_cast<u32>(first + t);
    for (u32 a = 0; a < g.num; ++a)
    {
        const u32 m = g.meta[a], o = g.off[a];
        if (!valid || !emitted<W>(st, g, a, m, o))
            continue;
        const u32 npos = m & 0xFF, nneg = (m >> 8) & 0xFF, nadd = (m >> 16) & 0xFF, ndel = m >> 24;
        u64 v[W];
#pragma unroll
        for (int w = 0; w < W; ++w)
            v[w] = r[w];
        const u32* adds = g.slots + o + npos + nneg;
        const u32* dels = adds + nadd;
        for (u32 i = 0; i < ndel; ++i)
        {
            const u32 s = dels[i];
#pragma unroll
            for (int w = 0; w < W; ++w)
                if (static_cast<u32>(w) == (s >> 6))
                    v[w] &= ~(u64{1} << (s & 63));
        }
        for (u32 i = 0; i < nadd; ++i)
        {
            const u32 s = adds[i];
#pragma unroll
            for (int w = 0; w < W; ++w)
                if (static_cast<u32>(w) == (s >> 6))
                    v[w] |= u64{1} << (s & 63);
        }
        u64* dst = cand + k * W;
#pragma unroll
        for (int w = 0; w < W; ++w)
            dst[w] = v[w];
        cand_hash[k] = hash_fixed<W>(v);
        cand_parent[k] = parent;
        cand_action[k] = a;
        ++k;
    }
}

// The winner whose exclusive rank equals `rank`: its candidate index.
__global__ void k_find_rank(const u32* __restrict__ flags, const u64* __restrict__ ranks, u64 n, u64 rank, u64* __restrict__ out)
{
    const u64 j = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (j < n && flags[j] && ranks[j] == rank)
        *out = j;
}

// The first index i in [lo, hi) with offsets[i] - base > limit (or hi): the parents whose successors fit a chunk.
__global__ void k_upper(const u64* __restrict__ offsets, u64 lo, u64 hi, u64 bound, u64* __restrict__ out)
{
    // one thread: binary search
    u64 a = lo, b = hi;
    while (a < b)
    {
        const u64 mid = a + (b - a) / 2;
        if (offsets[mid] <= bound)
            a = mid + 1;
        else
            b = mid;
    }
    *out = a;
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

struct Buffers
{
    u32* counts = nullptr;
    u8* goal = nullptr;
    u64* offsets = nullptr;
    u64* scan_scratch = nullptr;
    u64* cand = nullptr;
    u64* cand_hash = nullptr;
    u32* cand_parent = nullptr;
    u32* cand_action = nullptr;
    u64* small = nullptr;  // device scalars
    u64* host = nullptr;   // pinned mirror
    ~Buffers()
    {
        for (void* p : {static_cast<void*>(counts), static_cast<void*>(goal), static_cast<void*>(offsets), static_cast<void*>(scan_scratch),
                        static_cast<void*>(cand), static_cast<void*>(cand_hash), static_cast<void*>(cand_parent),
                        static_cast<void*>(cand_action), static_cast<void*>(small)})
            dev_free(p);
        if (host)
            (void)hipHostFree(host);
    }
};

using Clock = std::chrono::steady_clock;

/// HIP-event timing of kernel classes on one stream; durations are read once the stream has drained.
class Timers
{
public:
    Timers(bool on, hipStream_t s, BrfsResultC& r) : m_on(on), m_s(s), m_r(r) {}
    ~Timers()
    {
        for (auto& e : m_ev)
        {
            (void)hipEventDestroy(e.a);
            (void)hipEventDestroy(e.b);
        }
    }
    void begin(int k)
    {
        if (!m_on)
            return;
        Pair p{k, nullptr, nullptr};
        hip_check(hipEventCreate(&p.a), "event");
        hip_check(hipEventCreate(&p.b), "event");
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
            (void)hipEventDestroy(e.a);
            (void)hipEventDestroy(e.b);
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

template<int W>
BrfsResultC run(const CompiledTask& task, const GroundActions& ga, const BrfsOptionsC& o, std::vector<std::array<u64, 3>>& lc)
{
    BrfsResultC r;
    const auto t0 = Clock::now();
    hipStream_t stream = nullptr;
    hip_check(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "stream");
    struct StreamGuard
    {
        hipStream_t s;
        ~StreamGuard() { (void)hipStreamDestroy(s); }
    } sg{stream};
    Timers tm(o.timings != 0, stream, r);
    constexpr u64 R = W * 8;  // row bytes

    // ground table and goal
    u32* d_meta = dev_alloc<u32>(ga.meta.size(), "ground meta");
    u32* d_off = dev_alloc<u32>(ga.off.size(), "ground offsets");
    u32* d_slots = dev_alloc<u32>(ga.slots.size(), "ground slots");
    u32* d_dom_off = ga.dom_off.empty() ? nullptr : dev_alloc<u32>(ga.dom_off.size(), "ground dominators");
    u32* d_dom = ga.dom_off.empty() ? nullptr : dev_alloc<u32>(ga.dom.size(), "ground dominators");
    u32* d_gpos = dev_alloc<u32>(task.goal_pos.size(), "goal");
    u32* d_gneg = dev_alloc<u32>(task.goal_neg.size(), "goal");
    u64* d_slot_cid = task.mode == AtomMode::Dense ? nullptr : dev_alloc<u64>(task.slot_cid.size(), "slot cids");
    struct FreeAll
    {
        std::vector<void*> p;
        ~FreeAll()
        {
            for (void* x : p)
                dev_free(x);
        }
    } fa{{d_meta, d_off, d_slots, d_gpos, d_gneg, d_slot_cid, d_dom_off, d_dom}};
    auto up = [&](void* d, const void* h, size_t b) {
        if (b)
            hip_check(hipMemcpyAsync(d, h, b, hipMemcpyHostToDevice, stream), "upload");
    };
    up(d_meta, ga.meta.data(), ga.meta.size() * 4);
    up(d_off, ga.off.data(), ga.off.size() * 4);
    up(d_slots, ga.slots.data(), ga.slots.size() * 4);
    if (d_dom_off)
    {
        up(d_dom_off, ga.dom_off.data(), ga.dom_off.size() * 4);
        up(d_dom, ga.dom.data(), ga.dom.size() * 4);
    }
    up(d_gpos, task.goal_pos.data(), task.goal_pos.size() * 4);
    up(d_gneg, task.goal_neg.data(), task.goal_neg.size() * 4);
    if (d_slot_cid)
        up(d_slot_cid, task.slot_cid.data(), task.slot_cid.size() * 8);
    const GroundDev g{d_meta, d_off, d_slots, d_dom_off, d_dom, ga.size()};
    const GoalDev goal{d_gpos, d_gneg, static_cast<u32>(task.goal_pos.size()), static_cast<u32>(task.goal_neg.size()),
                       task.goal_unsat ? 1u : 0u};

    // capacity: the arena holds every stored state
    const bool bounded = o.max_states != ~u64{0};
    const u64 cap_states = bounded ? std::max<u64>(1, o.max_states) : (o.memory_states ? o.memory_states : (u64{1} << 26));
    const u64 chunk = std::max<u64>(o.chunk ? o.chunk : (u64{1} << 23), ga.size() + 1);
    StateSet set;
    state_set_create(set, cap_states, W, 0.5, chunk, stream, chunk);
    struct SetGuard
    {
        StateSet& s;
        ~SetGuard() { state_set_destroy(s); }
    } setg{set};
    Buffers b;
    b.counts = dev_alloc<u32>(cap_states, "layer counts");
    b.goal = dev_alloc<u8>(cap_states, "layer goal flags");
    b.offsets = dev_alloc<u64>(cap_states + 1, "layer offsets");
    b.scan_scratch = dev_alloc<u64>(scan_scratch_words(cap_states), "scan scratch");
    b.cand = dev_alloc<u64>(chunk * W, "candidate rows");
    b.cand_hash = dev_alloc<u64>(chunk, "candidate hashes");
    b.cand_parent = dev_alloc<u32>(chunk, "candidate parents");
    b.cand_action = dev_alloc<u32>(chunk, "candidate actions");
    b.small = dev_alloc<u64>(8, "scalars");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&b.host), 8 * sizeof(u64), hipHostMallocDefault), "pinned");

    auto read_small = [&](int idx) -> u64 {
        hip_check(hipMemcpyAsync(b.host + idx, b.small + idx, sizeof(u64), hipMemcpyDeviceToHost, stream), "read");
        hip_check(hipStreamSynchronize(stream), "sync");
        return b.host[idx];
    };
    auto set_small = [&](int idx, u64 v) { hipLaunchKernelGGL(k_set_u64, dim3(1), dim3(1), 0, stream, b.small + idx, v); };

    // the start state
    {
        std::vector<u64> s0(W, 0);
        std::copy(task.initial.begin(), task.initial.end(), s0.begin());
        hip_check(hipMemcpyAsync(b.cand, s0.data(), W * sizeof(u64), hipMemcpyHostToDevice, stream), "start state");
        u64 nn = 0;
        state_set_insert(set, b.cand, nullptr, 1, nullptr, nullptr, &nn, stream);
    }
    const auto td0 = Clock::now();
    u64 layer_begin = 0, layer_end = 1;
    bool stopped = false, budget_stopped = false;
    r.status = kExhausted;
    u64 pos = 0;  // states expanded or passed (the reference's queue position)
    while (!stopped)
    {
        if (pos >= set.size)
            break;
        if (bounded && set.size >= o.max_states)
        {
            r.status = kOutOfStates;
            break;
        }
        if (r.expanded >= o.max_expanded)
        {
            r.status = kOutOfStates;
            budget_stopped = true;
            break;
        }
        if (r.layers == o.max_depth)
            break;
        ++r.layers;
        layer_begin = pos;
        layer_end = set.size;
        const u64 ln = layer_end - layer_begin;
        std::array<u64, 3> row{0, 0, 0};
        const u64 size0 = set.size;
        // counts and goal flags of the whole layer
        tm.begin(kKCount);
        hipLaunchKernelGGL(k_ground_count<W>, dim3(blocks_for(ln, kGB)), dim3(kGB), 0, stream, set.v.arena, layer_begin,
                           static_cast<u32>(ln), g, goal, b.counts, b.goal);
        launch_check("ground count");
        tm.end(kKCount, ln * (R + 5));
        tm.begin(kKOther);
        launch_exclusive_scan(b.counts, b.offsets, ln, b.scan_scratch, b.small + 0, stream);
        tm.end(kKOther, 0);
        // offsets[ln] = total (for chunk searches)
        hip_check(hipMemcpyAsync(b.offsets + ln, b.small + 0, sizeof(u64), hipMemcpyDeviceToDevice, stream), "total");
        // the parents this layer expands: up to the first goal (stop_at_goal) and the expansion budget
        u64 expand_n = ln;
        set_small(1, ~u64{0});
        hipLaunchKernelGGL(k_first_u8, dim3(std::min<u64>(blocks_for(ln, 256), 4096)), dim3(256), 0, stream, b.goal, ln, b.small + 1);
        const u64 first_goal = read_small(1);
        bool goal_stop = false, budget_stop = false;
        if (o.stop_at_goal && first_goal != ~u64{0})
        {
            expand_n = first_goal;
            goal_stop = true;
        }
        // the budget check precedes the goal test of each state (brfs.cpp:138-144)
        if (o.max_expanded != ~u64{0} &&
            (goal_stop ? r.expanded + expand_n >= o.max_expanded : r.expanded + expand_n > o.max_expanded))
        {
            expand_n = o.max_expanded - r.expanded;
            budget_stop = true;
            goal_stop = false;
        }
        // chunks of parents whose successors fit the candidate buffers
        u64 p0 = 0;
        while (p0 < expand_n && !stopped)
        {
            set_small(2, 0);
            hip_check(hipMemcpyAsync(b.host + 3, b.offsets + p0, sizeof(u64), hipMemcpyDeviceToHost, stream), "offset");
            hip_check(hipStreamSynchronize(stream), "sync");
            const u64 base = b.host[3];
            // parents [p0, p1) end at offsets[p1] <= base + chunk: p1 + 1 is the first index past the bound
            hipLaunchKernelGGL(k_upper, dim3(1), dim3(1), 0, stream, b.offsets, p0, expand_n + 1, base + chunk, b.small + 2);
            u64 p1 = read_small(2) - 1;
            p1 = std::min<u64>(std::max<u64>(p1, p0 + 1), expand_n);
            hip_check(hipMemcpyAsync(b.host + 4, b.offsets + p1, sizeof(u64), hipMemcpyDeviceToHost, stream), "offset");
            hip_check(hipStreamSynchronize(stream), "sync");
            const u64 m = b.host[4] - base;
            const u32 np = static_cast<u32>(p1 - p0);
            tm.begin(kKGenerate);
            hipLaunchKernelGGL(k_ground_generate<W>, dim3(blocks_for(np, kGB)), dim3(kGB), 0, stream, set.v.arena, layer_begin + p0, np,
                               g, b.offsets + p0, base, b.cand, b.cand_hash, b.cand_parent, b.cand_action);
            launch_check("ground generate");
            tm.end(kKGenerate, np * (R + 8) + m * (R + 16));
            tm.begin(kKProbe);
            state_set_probe(set, b.cand, b.cand_hash, m, stream);
            tm.end(kKProbe, m * (R + 24));
            tm.begin(kKRank);
            state_set_rank(set, m, stream);
            tm.end(kKRank, m * 32);
            hip_check(hipMemcpyAsync(b.host + 5, set.d_total, sizeof(u64), hipMemcpyDeviceToHost, stream), "new");
            hip_check(hipMemcpyAsync(b.host + 6, set.d_status, sizeof(u32), hipMemcpyDeviceToHost, stream), "status");
            hip_check(hipStreamSynchronize(stream), "sync");
            if (static_cast<u32>(b.host[6]) & kStatusTableFull)
                throw std::length_error("mymyr_amd: brfs: state table full");
            const u64 fresh = b.host[5];
            tm.bytes(kKProbe, (m - fresh) * R);  // a duplicate compares its row with the stored one
            const u64 room = (bounded ? o.max_states : cap_states) - set.size;
            if (fresh >= room && fresh > 0 && bounded)
            {
                // the store fills at the winner of rank room - 1: stop inside its parent's expansion
                set_small(7, ~u64{0});
                hipLaunchKernelGGL(k_find_rank, dim3(blocks_for(m, 256)), dim3(256), 0, stream, set.flags, set.offsets, m, room - 1, b.small + 7);
                const u64 jcut = read_small(7);
                hip_check(hipMemcpyAsync(b.host + 3, b.cand_parent + jcut, sizeof(u32), hipMemcpyDeviceToHost, stream), "parent");
                hip_check(hipStreamSynchronize(stream), "sync");
                const u64 pcut = static_cast<u32>(b.host[3]) - layer_begin;  // index in the layer
                tm.begin(kKCompact);
                state_set_compact(set, b.cand, b.cand_hash, m, set.size, o.max_states, nullptr, nullptr, stream);
                tm.end(kKCompact, m * 12 + room * (2 * R + 24));
                row[0] += pcut - p0 + 1;
                row[1] += jcut + 1;
                set_small(0, 0);
                hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(pcut - p0 + 1, 256), 1024)), dim3(256), 0, stream, b.goal + p0,
                                   pcut - p0 + 1, b.small + 0);
                r.goal_states += read_small(0);
                set.size = o.max_states;
                r.status = kOutOfStates;
                stopped = true;
                break;
            }
            if (fresh > room)
                throw std::length_error("mymyr_amd: brfs: the search needs more than " + std::to_string(cap_states) +
                                        " states of device memory (set max_states or memory_states)");
            tm.begin(kKCompact);
            state_set_compact(set, b.cand, b.cand_hash, m, set.size, cap_states, nullptr, nullptr, stream);
            tm.end(kKCompact, m * 12 + fresh * (2 * R + 24));
            set.size += fresh;
            row[0] += np;
            row[1] += m;
            set_small(0, 0);
            hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(np, 256), 1024)), dim3(256), 0, stream, b.goal + p0, np, b.small + 0);
            r.goal_states += read_small(0);
            p0 = p1;
        }
        pos = layer_begin + row[0];
        r.expanded += row[0];
        r.generated += row[1];
        row[2] = set.size - size0;
        // the states this layer goal-tested: the expanded ones, plus the goal state a goal stop ends at
        const u64 tested = row[0] + ((goal_stop && !stopped) ? 1 : 0);
        if (first_goal != ~u64{0} && first_goal < tested && r.first_goal < 0)
            r.first_goal = static_cast<i64>(layer_begin + first_goal);
        if (goal_stop && !stopped)
        {
            r.goal_states += 1;  // the goal state is tested (and counted), then the search stops
            r.status = kSolved;
            stopped = true;
        }
        if (budget_stop && !stopped)
        {
            r.status = kOutOfStates;
            budget_stopped = true;
            stopped = true;
        }
        lc.push_back(row);
        if (!stopped)
            pos = layer_end;
    }
    r.states = set.size;
    r.exhausted = (!stopped && pos >= set.size) ? 1 : 0;
    // status as the reference's Control::finish (brfs.cpp:194-203): a tested goal state solves the search
    r.solved = r.first_goal >= 0 ? 1 : 0;
    if (r.solved)
        r.status = kSolved;
    else if (!budget_stopped)
        r.status = (r.exhausted || r.layers >= o.max_depth) ? kExhausted : kOutOfStates;
    hip_check(hipStreamSynchronize(stream), "brfs");
    r.device_s = std::chrono::duration<double>(Clock::now() - td0).count();
    tm.collect();
    if (o.fingerprint)
    {
        set_small(0, 0);
        hipLaunchKernelGGL(k_fingerprint, dim3(std::min<u64>(blocks_for(set.size, 256), 2048)), dim3(256), 0, stream, set.v.arena,
                           set.size, static_cast<u32>(W), d_slot_cid, b.small + 0);
        launch_check("fingerprint");
        r.fingerprint = read_small(0);
    }
    r.search_s = std::chrono::duration<double>(Clock::now() - t0).count();
    return r;
}
}  // namespace

BrfsResultC brfs_device(const CompiledTask& task, const BrfsOptionsC& o, std::vector<std::array<u64, 3>>& layer_counts)
{
    const GroundActions ga = ground_actions(task, o.witness_pruning != 0, u64{1} << 24);
    const u32 W = task.words;
    if (W <= 1)
        return run<1>(task, ga, o, layer_counts);
    if (W <= 2)
        return run<2>(task, ga, o, layer_counts);
    if (W <= 4)
        return run<4>(task, ga, o, layer_counts);
    if (W <= 8)
        return run<8>(task, ga, o, layer_counts);
    if (W <= 16)
        return run<16>(task, ga, o, layer_counts);
    throw std::invalid_argument("mymyr_amd: brfs: states of " + std::to_string(W) + " words (the device BrFS takes at most 16)");
}
}  // namespace mya
