// Device BrFS over ground actions (brfs.hpp).
//
// A layer's parents are expanded in chunks whose successors fit the candidate buffers. Per chunk, on one stream:
//   count   (thread per parent)     applicable-action counts and goal flags, for blocks of parents counted just ahead of
//                                   the expansion; a piecewise exclusive scan gives layer-relative successor offsets
//   emit    (thread per parent)     each parent's successors in action order as (parent, action) records at its
//                                   offsets: candidate index = order of first discovery (parent id, successor index)
//   insert  (group per candidate)   successor row = parent row with the action's delete and add masks, its state hash,
//                                   and the state set's probe: a successor equal to a stored state is dropped, equal
//                                   candidates keep the smallest index (rows of pending entries are recomputed from
//                                   their records, never stored)
//   rank / compact                  exclusive scan of the winner flags (new ids follow candidate order), winner rows
//                                   into the arena and their table entries settled
// The applicability test reads the parent from LDS byte planes (plane b holds byte b of every thread's row, so a
// wave reads 64 consecutive bytes per test) and the action records through scalar loads, eight actions at a time:
// an action with at most four positive preconditions, no negative one and no witness dominators is a single record
// of four precondition slots; the others take a general path over their slot lists.

#include "brfs.hpp"
#include "brfs_common.hpp"
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
constexpr int kTW = 4;        // waves per block of the per-parent kernels (64 parents per wave, one per lane)
constexpr int kLB = 256;      // threads per block of the per-candidate kernels
constexpr u64 kGeneral = 0x8000;  // fast-record flag: the action takes the general test
constexpr u64 kStrideBlocks = 4096;  // grid of the grid-stride kernels (16 blocks of 256 threads per CU)
constexpr int kCountPlanes = 7;    // bit planes of the per-lane successor counters (counts up to 64 between flushes)

struct GroundDev
{
    const u64* fast;     // [num_padded] four u16 precondition slots per action (kGeneral in the first)
    const u32* meta;     // npos | nneg << 8 | nadd << 16 | ndel << 24
    const u32* off;      // into slots
    const u32* slots;    // pos..., neg..., add..., del...
    const u32* dom_off;  // witness pruning: dominators of each action (null: none)
    const u32* dom;
    const u32* ce_off;   // conditional effects (null: none): action a's ground instances [ce_off[a], ce_off[a + 1])
    const u32* ce_meta;  // npos | nneg << 8 | nadd << 16 | ndel << 24 of each instance
    const u32* ce_soff;  // into ce_slots
    const u32* ce_slots; // pos..., neg..., add..., del...
    u32 num;
    u32 num_padded;      // a multiple of 64; the padding records never apply
};

struct GoalDev
{
    const u32* pos;
    const u32* neg;
    u32 npos, nneg;
    u32 unsat;
    AnyOfDev any;  // BrfsOptions::goal as GoalSpec::AnyOf (any.any set): it decides instead of the task's goal
};

/// Slot words of 64 parents, bit-sliced: word s holds bit s of each of the wave's 64 parents (bit t: parent t), for
/// s < 64W; word kOneSlot (= 64W) holds the wave's valid parents and word kZeroSlot (= 64W + 8) nothing, so a fast record
/// pads unused precondition slots with kOneSlot and padding actions with kZeroSlot.
template<int W>
struct Slices
{
    static constexpr u32 kOneSlot = W * 64;
    static constexpr u32 kZeroSlot = W * 64 + 8;
    static constexpr u32 kWords = W * 64 + 16;
};

/// Lane l ^ J's value, for J < 32: quad permutations (DPP) for 1 and 2, a bitmask swizzle within 32 lanes above.
template<int J>
__device__ __forceinline__ u32 xor_lane(u32 v)
{
    if constexpr (J == 1)
        return static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0xB1, 0xF, 0xF, false));  // [1,0,3,2]
    else if constexpr (J == 2)
        return static_cast<u32>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), 0x4E, 0xF, 0xF, false));  // [2,3,0,1]
    else
        return static_cast<u32>(__builtin_amdgcn_ds_swizzle(static_cast<int>(v), 0x1F | (J << 10)));  // and 31, xor J
}

/// One step of a 32x32 bit transpose over each half wave: lanes l and l ^ J swap the J-bit blocks that sit in the
/// wrong lane (the high J bits of each 2J-bit block of the lane without bit J, the low J bits of the other).
template<int J>
__device__ __forceinline__ u32 transpose_step(u32 x, u32 lane)
{
    constexpr u32 m = J == 16 ? 0x0000FFFFu : J == 8 ? 0x00FF00FFu : J == 4 ? 0x0F0F0F0Fu : J == 2 ? 0x33333333u : 0x55555555u;
    const u32 y = xor_lane<J>(x);
    const bool low = (lane & J) == 0;
    const u32 keep = low ? x : (y >> J), take = low ? (y << J) : x;
    return (keep & m) | (take & ~m);
}

/// 64x64 bit transpose across the wave: bit t of the result in lane s = bit s of x in lane t. The 32-bit halves
/// swap across the half waves first (the high word of lanes 0-31 with the low word of lanes 32-63, one lane-swap
/// instruction), then each word is a 32x32 transpose within its half wave; every step is branch-free.
__device__ __forceinline__ u64 transpose64(u64 x, u32 lane)
{
    u32 lo = static_cast<u32>(x), hi = static_cast<u32>(x >> 32);
    const auto sw = __builtin_amdgcn_permlane32_swap(lo, hi, false, false);  // lo of lanes 32-63 <-> hi of lanes 0-31
    lo = sw[0];
    hi = sw[1];
    lo = transpose_step<16>(lo, lane);
    hi = transpose_step<16>(hi, lane);
    lo = transpose_step<8>(lo, lane);
    hi = transpose_step<8>(hi, lane);
    lo = transpose_step<4>(lo, lane);
    hi = transpose_step<4>(hi, lane);
    lo = transpose_step<2>(lo, lane);
    hi = transpose_step<2>(hi, lane);
    lo = transpose_step<1>(lo, lane);
    hi = transpose_step<1>(hi, lane);
    return static_cast<u64>(lo) | (static_cast<u64>(hi) << 32);
}

/// Loads the rows of parents [first + base, + 64) (lane t: parent base + t, rows past n zero) bit-sliced into B.
/// Returns the mask of the valid parents.
template<int W>
__device__ __forceinline__ u64 load_slices(u64* B, const u64* __restrict__ arena, u64 first, u32 base, u32 n, u32 lane)
{
    const u32 t = base + lane;
    const bool valid = t < n;
    const u64* row = arena + (first + (valid ? t : 0)) * W;
#pragma unroll
    for (int w = 0; w < W; ++w)
        B[w * 64 + lane] = transpose64(valid ? row[w] : 0, lane);
    const u64 vm = __ballot(valid);
    if (lane < 16)
        B[W * 64 + lane] = lane < 8 ? vm : 0;
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    return vm;
}

/// The parents (bit mask) for which action a's precondition list holds.
__device__ __forceinline__ u64 holds_mask(const u64* B, const u32* __restrict__ slots, u32 m, u32 o, u64 vm)
{
    const u32 npos = m & 0xFF, nneg = (m >> 8) & 0xFF;
    u64 r = vm;
    for (u32 i = 0; i < npos; ++i)
        r &= B[slots[o + i]];
    for (u32 i = 0; i < nneg; ++i)
        r &= ~B[slots[o + npos + i]];
    return r;
}

/// The parents for which action a is a successor: its preconditions hold and (witness pruning) no dominator's do.
__device__ __noinline__ u64 general_mask(const u64* B, const u32* __restrict__ slots, const u32* __restrict__ meta, const u32* __restrict__ off,
                                        const u32* __restrict__ dom_off, const u32* __restrict__ dom, u32 a, u64 vm)
{
    u64 r = holds_mask(B, slots, meta[a], off[a], vm);
    if (dom_off && r)
        for (u32 k = dom_off[a], e = dom_off[a + 1]; k < e; ++k)
        {
            const u32 d = dom[k];
            r &= ~holds_mask(B, slots, meta[d], off[d], vm);
        }
    return r;
}

/// The successor mask over the wave's parents of the action in this lane (record rec).
template<int W>
__device__ __forceinline__ u64 action_mask(const u64* B, const GroundDev& g, u64 rec, u32 a, u64 vm)
{
    if (rec & kGeneral)
        return general_mask(B, g.slots, g.meta, g.off, g.dom_off, g.dom, a, vm);
    return B[rec & 0x7FFF] & B[(rec >> 16) & 0xFFFF] & B[(rec >> 32) & 0xFFFF] & B[rec >> 48];
}

// Successor counts and goal flags of parents [first, first + n): a wave takes 64 parents bit-sliced in LDS; each lane
// tests one action of a group of 64 against all 64 parents at once (an AND of the action's precondition slot words),
// and a transpose turns the group's masks into each parent's 64 action bits.
template<int W>
__global__ __launch_bounds__(kTW * kWave) void k_ground_count(const u64* __restrict__ arena, u64 first, u32 n, GroundDev g, GoalDev goal,
                                                             u32* __restrict__ counts, u8* __restrict__ goal_flags)
{
    __shared__ u64 Bs[kTW][Slices<W>::kWords];
    const u32 lane = lane_id(), wave = threadIdx.x / kWave;
    const u32 base = (blockIdx.x * kTW + wave) * kWave;
    if (base >= n)
        return;
    u64* B = Bs[wave];
    const u64 vm = load_slices<W>(B, arena, first, base, n, lane);
    u64 gm = 0;
    if (goal.any.any)
    {
        // AnyOf: the parents for which one of the goals holds, goal by goal over the bit slices
        for (u32 k = 0; k < goal.any.count; ++k)
        {
            u64 m = vm;
            for (u32 i = goal.any.off[2 * k]; i < goal.any.off[2 * k + 1]; ++i)
                m &= B[goal.any.slots[i]];
            for (u32 i = goal.any.off[2 * k + 1]; i < goal.any.off[2 * k + 2]; ++i)
                m &= ~B[goal.any.slots[i]];
            gm |= m;
        }
    }
    else
    {
        gm = goal.unsat ? 0 : vm;
        for (u32 i = 0; i < goal.npos; ++i)
            gm &= B[goal.pos[i]];
        for (u32 i = 0; i < goal.nneg; ++i)
            gm &= ~B[goal.neg[i]];
    }
    // Per lane (one action of each group), a bit-sliced counter over the 64 parents: plane k holds bit k of how many of
    // the lane's actions so far apply to each parent. Adding a group's mask is a ripple carry through the planes, and
    // only the final planes are transposed (bit k of parent t's count over the lanes = popcount of plane k's column t),
    // instead of one transpose per group. 64 groups at most between flushes keep every counter below 2^7.
    u64 plane[kCountPlanes] = {};
    u32 cnt = 0, groups = 0;
    auto add = [&](u64 m) {
#pragma unroll
        for (int k = 0; k < kCountPlanes; ++k)
        {
            const u64 c = plane[k] & m;
            plane[k] ^= m;
            m = c;
        }
    };
    auto flush = [&]() {
#pragma unroll
        for (int k = 0; k < kCountPlanes; ++k)
        {
            cnt += static_cast<u32>(__popcll(transpose64(plane[k], lane))) << k;
            plane[k] = 0;
        }
        groups = 0;
    };
    u32 a0 = 0;
    for (; a0 + 4 * kWave <= g.num_padded; a0 += 4 * kWave)
    {
        // four independent groups in flight
        u64 m[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            m[k] = action_mask<W>(B, g, g.fast[a0 + k * kWave + lane], a0 + k * kWave + lane, vm);
#pragma unroll
        for (int k = 0; k < 4; ++k)
            add(m[k]);
        groups += 4;
        if (groups == 64)
            flush();
    }
    for (; a0 < g.num_padded; a0 += kWave)
    {
        const u32 a = a0 + lane;
        add(action_mask<W>(B, g, g.fast[a], a, vm));
        if (++groups == 64)
            flush();
    }
    flush();
    const u32 t = base + lane;
    if (t < n)
    {
        counts[t] = cnt;
        goal_flags[t] = static_cast<u8>((gm >> lane) & 1);
    }
}

// (parent, action) records of the successors of parents [first, first + n) at their offsets (candidate index =
// offsets[t] - cand_base + rank in action order), 32 bits each: the parent index relative to `first` above the low
// `abits` bits, which hold the action (the driver keeps a chunk's parents below 2^(32 - abits)).
//
// Each parent's records are a run of its own (about 9 per parent and group of 256 actions here), so a lane writing its
// parent's records straight out makes every store touch as many memory lines as there are lanes. The wave stages the
// records of each 256-action step in LDS instead, parent after parent (a wave prefix sum of the parents' counts places
// them), with their candidate indices beside them, and writes them out in staging order: 64 consecutive staged records
// lie in a few parents' runs, a few lines per store. A step with more records than the stage holds writes directly.
constexpr u32 kEmitStage = 1024;  // staged records per wave (8 KiB of LDS with their indices)

template<int W>
__global__ __launch_bounds__(kTW * kWave) void k_ground_emit(const u64* __restrict__ arena, u64 first, u32 n, GroundDev g,
                                                            const u64* __restrict__ offsets, u64 cand_base, u32 abits,
                                                            u32* __restrict__ cand_pa)
{
    __shared__ u64 Bs[kTW][Slices<W>::kWords];
    __shared__ u64 Stage[kTW][kEmitStage];  // (candidate index << 32) | record
    const u32 lane = lane_id(), wave = threadIdx.x / kWave;
    const u32 base = (blockIdx.x * kTW + wave) * kWave;
    if (base >= n)
        return;
    u64* B = Bs[wave];
    u64* stage = Stage[wave];
    const u64 vm = load_slices<W>(B, arena, first, base, n, lane);
    const u32 t = base + lane;
    const bool valid = t < n;
    // candidate indices relative to the wave's first parent's (a wave holds at most 64 times the actions, below 2^32)
    const u64 kbase = offsets[base] - cand_base;
    u32 k = valid ? static_cast<u32>(offsets[t] - cand_base - kbase) : 0;
    const u32 hi = t << abits;
    for (u32 a0 = 0; a0 < g.num_padded; a0 += 4 * kWave)
    {
        // four groups in flight (num_padded is a multiple of 64; groups past it are empty)
        u64 mt[4];
#pragma unroll
        for (int q = 0; q < 4; ++q)
        {
            const u32 a = a0 + q * kWave + lane;
            mt[q] = a0 + q * kWave < g.num_padded ? action_mask<W>(B, g, g.fast[a], a, vm) : 0;
        }
        // every lane takes part in the transposes (cross-lane moves), invalid parents' masks cleared after them
#pragma unroll
        for (int q = 0; q < 4; ++q)
            mt[q] = transpose64(mt[q], lane);
#pragma unroll
        for (int q = 0; q < 4; ++q)
            mt[q] = valid ? mt[q] : 0;
        const u32 c = static_cast<u32>(__popcll(mt[0]) + __popcll(mt[1]) + __popcll(mt[2]) + __popcll(mt[3]));
        const u32 inc = wave_inclusive(c);
        const u32 total = __shfl(inc, kWave - 1, kWave);
        if (total > kEmitStage)
        {
#pragma unroll
            for (int q = 0; q < 4; ++q)
                while (mt[q])
                {
                    const u32 bit = static_cast<u32>(__builtin_ctzll(mt[q]));
                    mt[q] &= mt[q] - 1;
                    cand_pa[kbase + k++] = hi | (a0 + q * kWave + bit);
                }
            continue;
        }
        u32 pos = inc - c;
#pragma unroll
        for (int q = 0; q < 4; ++q)
            while (mt[q])
            {
                const u32 bit = static_cast<u32>(__builtin_ctzll(mt[q]));
                mt[q] &= mt[q] - 1;
                stage[pos++] = (static_cast<u64>(k++) << 32) | (hi | (a0 + q * kWave + bit));
            }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        for (u32 r = lane; r < total; r += kWave)
        {
            const u64 e = stage[r];
            cand_pa[kbase + (e >> 32)] = static_cast<u32>(e);
        }
        // the next step overwrites the stage only after every lane has read its share
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
}

/// The successor rows of (parent, action) records as the row source of the state set's probe and compaction:
/// candidate c's row = (parent row & ~delete mask) | add mask, recomputed wherever it is needed (the probe compares a
/// pending entry against it, the compaction writes it), so candidate rows are never stored before they are new states.
///
/// With conditional effects (kCE), the instances of the candidate's action whose conditions hold in the parent row add
/// their deletes and adds to the masks before the row is formed: every effect of the action is applied as "delete, then
/// add", the adds winning (include/mymyr/successor/successors.hpp:361-385).
template<int W, bool kCE = false>
struct ParentRows
{
    const u64* arena;
    u64 first;            // arena id of the chunk's first parent (records hold the parent relative to it)
    const u32* cand_pa;   // (parent << abits) | action
    const u64* masks;     // [actions, 2W]: delete mask, then add mask
    u32 abits;            // action bits of a record
    const u32* ce_off;    // kCE: GroundDev's conditional effect tables
    const u32* ce_meta;
    const u32* ce_soff;
    const u32* ce_slots;
    __device__ __forceinline__ u32 parent_of(u32 pa) const { return pa >> abits; }
    __device__ __forceinline__ u32 action_of(u32 pa) const { return pa & ((1u << abits) - 1); }
    template<int G, int K>
    __device__ __forceinline__ void load(u64 c, u32 q, Slice<G, K>& o) const
    {
        load_pa<G, K>(cand_pa[c], q, o);
    }
    /// The row of the candidate with record pa.
    template<int G, int K>
    __device__ __forceinline__ void load_pa(u32 pa, u32 q, Slice<G, K>& o) const
    {
        const u64* row = arena + (first + parent_of(pa)) * W;
        const u64* mk = masks + static_cast<u64>(action_of(pa)) * (2 * W);
        Slice<G, K> r, d, a;
        load_row<G, K>(row, W, q, r);
        load_row<G, K>(mk, W, q, d);
        load_row<G, K>(mk + W, W, q, a);
        if constexpr (kCE)
            fire_ces<G, K>(row, action_of(pa), q, d, a);
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            o.lo[k] = (r.lo[k] & ~d.lo[k]) | a.lo[k];
            o.hi[k] = (r.hi[k] & ~d.hi[k]) | a.hi[k];
        }
    }
    /// Sets slot s's bit in x if lane q holds its word (word w is in pair w / 2, pair p at lane p % G, index p / G).
    template<int G, int K>
    __device__ __forceinline__ static void set_slot(Slice<G, K>& x, u32 s, u32 q)
    {
        const u32 w = s >> 6, p = w >> 1;
        if (p % G != q)
            return;
        const u64 bit = u64{1} << (s & 63);
#pragma unroll
        for (int k = 0; k < K; ++k)
            if (p / G == static_cast<u32>(k))
            {
                if (w & 1)
                    x.hi[k] |= bit;
                else
                    x.lo[k] |= bit;
            }
    }
    /// The deletes and adds of action a's conditional effect instances whose conditions hold in `row` into d and a.
    template<int G, int K>
    __device__ __forceinline__ void fire_ces(const u64* row, u32 act, u32 q, Slice<G, K>& d, Slice<G, K>& a) const
    {
        for (u32 i = ce_off[act], e = ce_off[act + 1]; i < e; ++i)
        {
            const u32 m = ce_meta[i], o = ce_soff[i];
            const u32 npos = m & 0xFF, nneg = (m >> 8) & 0xFF, nadd = (m >> 16) & 0xFF, ndel = m >> 24;
            bool fires = true;
            for (u32 k = 0; k < npos && fires; ++k)
            {
                const u32 s = ce_slots[o + k];
                fires = (row[s >> 6] >> (s & 63)) & 1;
            }
            for (u32 k = 0; k < nneg && fires; ++k)
            {
                const u32 s = ce_slots[o + npos + k];
                fires = !((row[s >> 6] >> (s & 63)) & 1);
            }
            if (!fires)
                continue;
            for (u32 k = 0; k < nadd; ++k)
                set_slot<G, K>(a, ce_slots[o + npos + nneg + k], q);
            for (u32 k = 0; k < ndel; ++k)
                set_slot<G, K>(d, ce_slots[o + npos + nneg + nadd + k], q);
        }
    }
};

template<int W>
constexpr int kGroup = W >= 4 ? W / 4 : 1;  // lanes per candidate row (32 bytes each)
template<int W>
constexpr int kPairs = W >= 4 ? 2 : 1;  // word pairs per lane

// Candidates [0, m) of a chunk into the state set: a group of lanes per candidate forms its row, hashes it and probes
// the table (a stored equal row drops it; a pending equal row takes part in the smallest-index rule; an empty slot
// takes it as pending). Losers' flags are cleared, winners' stay 1.
template<int W, bool kCE>
__global__ __launch_bounds__(kLB) void k_ground_insert(StateSetView s, ParentRows<W, kCE> src, u64 m, u8* __restrict__ flags,
                                                      u32* __restrict__ status, BlockedView blocked, u64* __restrict__ cand_slot)
{
    constexpr int G = kGroup<W>;
    const u64 j = (static_cast<u64>(blockIdx.x) * kLB + threadIdx.x) / G;
    const u32 q = lane_id() % G, gbase = lane_id() - q;
    if (j >= m)
        return;
    Slice<G, kPairs<W>> me;
    src.load(j, q, me);
    const u64 h = group_set_hash<G, kPairs<W>>(me, q, gbase);
    if (blocked.capacity)
    {
        // the blocked test precedes the store (brfs.cpp:350-361): a blocked candidate takes no entry and no id
        const bool hit = group_blocked<G, kPairs<W>>(blocked, me, h, q, gbase);
        if (q == 0)
        {
            blocked.hit[j] = hit ? 1 : 0;
            if (hit)
                flags[j] = 0;
        }
        if (hit)
            return;
    }
    const ProbeResult r = probe_insert<G, kPairs<W>>(s, src, j, me, h, q, gbase, flags, status);
    if (q == 0 && r.lose)
        flags[j] = 0;
    if (q == 0 && cand_slot)
        cand_slot[j] = r.cand_slot;  // an observed search resolves every candidate's state id from it
}

// The chunk's winners (list order, ids from *size_now, their count size_next - size_now) below `limit` into the arena
// (rows recomputed from their records), with their search nodes: nodes[id] = (parent id << 32) | ground action, the
// first discovery of the state (the reference's node records, src/mymyr/search/brfs.cpp:235-268). A winner at or past
// `limit` sets kStatusCapacity.
template<int W, bool kCE>
__global__ __launch_bounds__(kLB) void k_ground_compact(StateSetView s, ParentRows<W, kCE> src, u64 m, const u32* __restrict__ list,
                                                       const u64* __restrict__ size_now, const u64* __restrict__ size_next, u64 limit,
                                                       const u64* __restrict__ parent_ids, u64* __restrict__ nodes, u32* __restrict__ status)
{
    constexpr int G = kGroup<W>;
    constexpr int K = kPairs<W>;
    constexpr int kBatch = 16;  // winners per group in flight (the list, record and row loads of each are independent)
    const u32 q = lane_id() % G;
    const u64 id0 = *size_now;
    const u64 winners = min(m, *size_next - id0);
    const u64 stride = static_cast<u64>(gridDim.x) * (kLB / G);
    // a grid sized for the whole chunk would mostly start waves that find no winner: a bounded grid strides instead
    for (u64 w0 = (static_cast<u64>(blockIdx.x) * kLB + threadIdx.x) / G; w0 < winners; w0 += kBatch * stride)
    {
        u32 pa[kBatch];
        bool live[kBatch];
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
        {
            const u64 w = w0 + b * stride;
            live[b] = w < winners && id0 + w < limit;
            if (w < winners && id0 + w >= limit && q == 0)
                atomicOr(status, kStatusCapacity);
            pa[b] = live[b] ? list[w] : 0;
        }
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
            pa[b] = live[b] ? src.cand_pa[pa[b]] : 0;
#pragma unroll
        for (int b = 0; b < kBatch; ++b)
        {
            if (!live[b])
                continue;
            const u64 id = id0 + w0 + b * stride;
            Slice<G, K> r;
            src.template load_pa<G, K>(pa[b], q, r);
            store_row<G, K>(s.arena + id * W, W, q, r);
            if (q == 0)
            {
                // parent rows gathered in an ordered layer's expansion order carry their ids in parent_ids
                const u64 p = src.first + src.parent_of(pa[b]);
                nodes[id] = ((parent_ids ? parent_ids[p] : p) << 32) | src.action_of(pa[b]);
            }
        }
    }
}

/// The fast records and the delete / add masks of the ground actions (host).
template<int W>
void build_action_tables(const GroundActions& ga, std::vector<u64>& fast, std::vector<u64>& masks)
{
    const u32 num = ga.size();
    const u32 padded = (num + 63) & ~63u;
    constexpr u64 one = Slices<W>::kOneSlot, zero = Slices<W>::kZeroSlot;
    fast.assign(padded, zero | (zero << 16) | (zero << 32) | (zero << 48));
    masks.assign(static_cast<size_t>(num) * 2 * W, 0);
    for (u32 a = 0; a < num; ++a)
    {
        const u32 m = ga.meta[a], o = ga.off[a];
        const u32 npos = m & 0xFF, nneg = (m >> 8) & 0xFF, nadd = (m >> 16) & 0xFF, ndel = m >> 24;
        const bool dominated = !ga.dom_off.empty() && ga.dom_off[a + 1] > ga.dom_off[a];
        u64 rec = 0;
        for (u32 i = 0; i < 4; ++i)
            rec |= (i < npos ? static_cast<u64>(ga.slots[o + i]) : one) << (16 * i);
        if (nneg || npos > 4 || dominated)
            rec = (rec & ~u64{0xFFFF}) | one | kGeneral;
        fast[a] = rec;
        u64* del = masks.data() + static_cast<size_t>(a) * 2 * W;
        u64* add = del + W;
        for (u32 i = 0; i < ndel; ++i)
        {
            const u32 s = ga.slots[o + npos + nneg + nadd + i];
            del[s >> 6] |= u64{1} << (s & 63);
        }
        for (u32 i = 0; i < nadd; ++i)
        {
            const u32 s = ga.slots[o + npos + nneg + i];
            add[s >> 6] |= u64{1} << (s & 63);
        }
    }
}

}  // namespace

struct BrfsTables;

namespace
{
/// Successor row of ground action a from a parent row on the host (an observed search's events): the instances of
/// its conditional effects that fire in the parent add their deletes and adds, then "delete, then add".
void host_successor(const std::vector<u64>& masks, const GroundActions& ga, const u64* parent, u32 a, u32 W, u64* out)
{
    std::vector<u64> del(masks.begin() + static_cast<size_t>(a) * 2 * W, masks.begin() + static_cast<size_t>(a) * 2 * W + W);
    std::vector<u64> add(masks.begin() + static_cast<size_t>(a) * 2 * W + W, masks.begin() + static_cast<size_t>(a + 1) * 2 * W);
    auto bit = [&](u32 sl) { return (parent[sl >> 6] >> (sl & 63)) & 1; };
    if (!ga.ce_meta.empty())
        for (u32 i = ga.ce_off[a]; i < ga.ce_off[a + 1]; ++i)
        {
            const u32 m = ga.ce_meta[i], o = ga.ce_soff[i];
            const u32 npos = m & 0xFF, nneg = (m >> 8) & 0xFF, nadd = (m >> 16) & 0xFF, ndel = m >> 24;
            bool fires = true;
            for (u32 k = 0; k < npos && fires; ++k)
                fires = bit(ga.ce_slots[o + k]);
            for (u32 k = 0; k < nneg && fires; ++k)
                fires = !bit(ga.ce_slots[o + npos + k]);
            if (!fires)
                continue;
            for (u32 k = 0; k < nadd; ++k)
            {
                const u32 sl = ga.ce_slots[o + npos + nneg + k];
                add[sl >> 6] |= u64{1} << (sl & 63);
            }
            for (u32 k = 0; k < ndel; ++k)
            {
                const u32 sl = ga.ce_slots[o + npos + nneg + nadd + k];
                del[sl >> 6] |= u64{1} << (sl & 63);
            }
        }
    for (u32 w = 0; w < W; ++w)
        out[w] = (parent[w] & ~del[w]) | add[w];
}
}  // namespace

struct BrfsTables
{
    int device = -1;
    u32 W = 0;
    GroundActions ga;
    GroundDev g{};
    GoalDev goal{};
    const u64* masks = nullptr;
    const u64* slot_cid = nullptr;
    std::vector<u64> host_masks;  // the delete and add masks on the host (an observed search's successor rows)
    std::vector<void*> owned;

    template<class T>
    const T* upload(const std::vector<T>& v)
    {
        if (v.empty())
            return nullptr;
        T* d = dev_alloc<T>(v.size(), "brfs tables");
        owned.push_back(d);
        hip_check(hipMemcpy(d, v.data(), v.size() * sizeof(T), hipMemcpyHostToDevice), "brfs tables");
        return d;
    }
    ~BrfsTables()
    {
        for (void* p : owned)
            dev_free(p);
    }
};

BrfsCache::BrfsCache() = default;
BrfsCache::~BrfsCache() = default;

namespace
{
template<int W>
std::unique_ptr<BrfsTables> build_tables(const CompiledTask& task, bool witness, int device)
{
    auto tb = std::make_unique<BrfsTables>();
    tb->device = device;
    tb->W = W;
    tb->ga = ground_actions(task, witness, u64{1} << 24);
    const GroundActions& ga = tb->ga;
    std::vector<u64> fast, masks;
    build_action_tables<W>(ga, fast, masks);
    // an action's conditional effect instances are evaluated where its successor rows are formed; tables without any
    // instance take the plain kernels
    const bool ces = !ga.ce_meta.empty();
    tb->g = GroundDev{tb->upload(fast),
                      tb->upload(ga.meta),
                      tb->upload(ga.off),
                      tb->upload(ga.slots),
                      tb->upload(ga.dom_off),
                      tb->upload(ga.dom),
                      ces ? tb->upload(ga.ce_off) : nullptr,
                      ces ? tb->upload(ga.ce_meta) : nullptr,
                      ces ? tb->upload(ga.ce_soff) : nullptr,
                      ces ? tb->upload(ga.ce_slots) : nullptr,
                      ga.size(),
                      static_cast<u32>(fast.size())};
    tb->masks = tb->upload(masks);
    tb->host_masks = std::move(masks);
    tb->goal = GoalDev{tb->upload(task.goal_pos), tb->upload(task.goal_neg), static_cast<u32>(task.goal_pos.size()),
                       static_cast<u32>(task.goal_neg.size()), task.goal_unsat ? 1u : 0u};
    tb->slot_cid = task.mode == AtomMode::Dense ? nullptr : tb->upload(task.slot_cid);
    return tb;
}

template<int W>
BrfsResultC run(const CompiledTask& task, const BrfsTables& tb, const BrfsOptionsC& o, std::vector<std::array<u64, 3>>& lc)
{
    const GroundActions& ga = tb.ga;
    BrfsResultC r;
    const auto t0 = Clock::now();
    hipStream_t stream = thread_stream();
    Timers tm(o.timings != 0, stream, r);
    constexpr u64 R = W * 8;  // row bytes
    Buffers b(stream);

    // ground tables and goal (device copies kept with the task)
    constexpr u32 S = 1;  // one count and one offset per parent
    const GroundDev& g = tb.g;
    const u64* d_masks = tb.masks;
    GoalDev goal = tb.goal;
    goal.any = upload_any_of(o, b, stream);
    const u64* d_slot_cid = tb.slot_cid;

    // capacity: the arena holds every stored state
    const bool bounded = o.max_states != ~u64{0};
    const u64 cap_states = bounded ? std::max<u64>(1, o.max_states) : (o.memory_states ? o.memory_states : (u64{1} << 26));
    // a chunk holds at most kMaxBatch candidates (the state set's candidate-coded entries) and one parent's successors
    if (ga.size() + 1 > kMaxBatch)
        throw std::invalid_argument("mymyr_amd: brfs: more than 2^25 - 1 ground actions");
    const u64 chunk = std::min<u64>(std::max<u64>(o.chunk ? o.chunk : kMaxBatch, ga.size() + 1), kMaxBatch);
    StateSet set;
    state_set_create(set, cap_states, W, 0.5, chunk, stream, chunk);
    struct SetGuard
    {
        StateSet& s;
        hipStream_t st;
        ~SetGuard() { state_set_destroy(s, st); }
    } setg{set, stream};
    // per-layer arrays (grown with the largest layer): counts [parents * S] per (parent, slice), goal flags per parent,
    // successor offsets [parents * S + 1] (layer-relative candidate indices)
    u32* counts = nullptr;
    u8* goal_flags = nullptr;
    u64* offsets = nullptr;
    u64* scan_scratch = nullptr;
    // sized once for the largest layer (no layer outgrows the store), so that no layer start waits for reallocation
    const u64 layer_cap = cap_states;
    counts = dev_alloc<u32>(layer_cap * S, "layer counts");
    goal_flags = dev_alloc<u8>(layer_cap, "layer goal flags");
    offsets = dev_alloc<u64>(layer_cap * S + 1, "layer offsets");
    scan_scratch = dev_alloc<u64>(scan_scratch_words(layer_cap * S), "scan scratch");
    struct LayerGuard
    {
        u32*& c;
        u8*& g;
        u64*& o;
        u64*& s;
        hipStream_t st;
        ~LayerGuard()
        {
            dev_free_async(c, st);
            dev_free_async(g, st);
            dev_free_async(o, st);
            dev_free_async(s, st);
        }
    } layer_guard{counts, goal_flags, offsets, scan_scratch, stream};
    // 32-bit candidate records: the action in the low abits bits, the parent relative to the chunk's first above them
    u32 abits = 1;
    while ((u64{1} << abits) < g.num_padded)
        ++abits;
    const u64 max_chunk_parents = u64{1} << (32 - abits);
    u32* cand_pa = b.alloc<u32>(chunk, "candidate records");
    u64* small = b.alloc<u64>(kSmall, "scalars");
    // search nodes: per stored state its first discovery (parent id << 32 | ground action); the start state has none
    u64* nodes = b.alloc<u64>(cap_states, "search nodes");
    r.memory_bytes = set.v.capacity * 8 + cap_states * (R + 8) + chunk * (4 + 8 + 1 + 4) + layer_cap * (S * 4 + 1 + S * 8 + 8);
    b.host = static_cast<u64*>(pinned_acquire(kSmall * sizeof(u64)));
    enum
    {
        kGoalSum = 0,   // goal states among the layer's expanded parents
        kFirstGoal = 1, // first goal flag of a counted block
        kChunkP = 2,    // chunk end parent, then its offset
        kChunkOff = 3,
        kSizeNow = 4,   // the set's size before the chunk's insert, then after it
        kSizeNext = 8,
        kChunkGoal = 10,  // goal states among a chunk's parents (read at the synchronization that confirms the chunk)
        kSpare = 9,     // the capacity status of a cut chunk's compaction (expected there, not an error)
        kCut = 5,       // the candidate of the state that fills the store
        kBlockTotal = 6,
        kFingerprint = 7,
        kChunkPruned = 11,  // blocked candidates of a chunk (read at the synchronization that confirms it)
        kCutPruned = 12,    // blocked candidates of a cut chunk up to the cut
    };
    auto set_small = [&](int idx, u64 v) { hipLaunchKernelGGL(k_set_u64, dim3(1), dim3(1), 0, stream, small + idx, v); };
    auto sync_small = [&] {
        hip_check(hipMemcpyAsync(b.host, small, kSmall * sizeof(u64), hipMemcpyDeviceToHost, stream), "read scalars");
        hip_check(hipStreamSynchronize(stream), "sync");
    };

    const BlockedView blocked = upload_blocked(o.blocked, task.words, W, chunk, b, stream);
    EventBuffers ev;
    ev.init(o.observed(), chunk, b);
    // the start state (stored even if blocked)
    {
        const std::vector<u64> s0 = start_row(task, o, W);
        u64* d_s0 = b.alloc<u64>(W, "start state");
        hip_check(hipMemcpyAsync(d_s0, s0.data(), W * sizeof(u64), hipMemcpyHostToDevice, stream), "start state");
        u64 nn = 0;
        state_set_insert(set, d_s0, 1, nullptr, nullptr, &nn, stream);
        hipLaunchKernelGGL(k_set_u64, dim3(1), dim3(1), 0, stream, nodes, ~u64{0});
        launch_check("root node");
    }
    const auto td0 = Clock::now();
    Halt halt(o, t0);
    LayerOrder lorder(o);
    LayerRows lrows(stream);
    bool stopped = false, budget_stopped = false;
    r.status = kExhausted;
    u64 pos = 0;                           // states expanded or passed (the reference's queue position)
    u64 seen_parents = 0, seen_cands = 0;  // counted so far (the successors-per-parent estimate)
    double new_rate = 1.0;                 // new states per candidate of the last confirmed chunk
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
        if (halt.check(r.expanded, r.generated, set.size))
        {
            stopped = true;
            break;
        }
        if (r.layers == o.max_depth)
            break;
        ++r.layers;
        const u64 layer_begin = pos, layer_end = set.size;
        const u64 ln = layer_end - layer_begin;
        std::array<u64, 3> row{0, 0, 0};
        const auto layer_t0 = Clock::now();
        const u64 size0 = set.size;
        // parent rows: the layer's rows in the arena, or an ordered layer's rows gathered in its expansion order (the
        // positions below are then expansion positions, pids their state ids)
        const u64* par = set.v.arena;
        u64 pbase = layer_begin;
        const u64* pids = nullptr;
        u64 keep = ln;
        if (lorder.ordered() && layer_begin > 0)
        {
            lrows.order(lorder, o, task, set.v.arena, layer_begin, ln, W, stream);
            par = lrows.rows.p;
            pbase = 0;
            pids = lrows.d_ids.p;
            keep = lrows.ids.size();
        }
        auto id_at = [&](u64 p) { return pids ? lrows.ids[p] : layer_begin + p; };
        // the id at which the store takes no more states: max_states, and with max_next_layer_states the layer's end
        // plus the limit (the layer is cut there and the search goes on, brfs.cpp:360-365)
        u64 cut_at = bounded ? o.max_states : ~u64{0};
        bool layer_cut = false, truncated = false;
        if (lorder.limited() && layer_end + o.max_next_layer_states < cut_at)
        {
            cut_at = layer_end + o.max_next_layer_states;
            layer_cut = true;
        }
        // the budget check precedes the goal test of each state (brfs.cpp:138-144): parents at or past the remaining
        // budget are neither tested nor expanded
        const u64 budget = o.max_expanded == ~u64{0} ? ~u64{0} : o.max_expanded - r.expanded;
        u64 lim = std::min(keep, budget);
        u64 counted = 0, counted_total = 0;  // parents [0, counted) counted; offsets[counted * S] on the host
        u64 first_goal = ~u64{0};
        bool goal_stop = false;
        u64 layer_goals = 0;   // goal states among the layer's expanded parents (confirmed chunks)
        u64 layer_pruned = 0;  // blocked successors of the confirmed chunks
        u64 p0 = 0, base = 0;  // base = offsets[p0 * S]
        constexpr int G = kGroup<W>;
        // The chunk whose kernels are queued but whose outcome (its winners) the host has not read yet: it is confirmed
        // at the next synchronization, which precedes the next chunk's emit and rank (its records and winner list are
        // intact until then), so the driver synchronizes once per chunk.
        struct Pending
        {
            bool live = false;
            u64 p0 = 0, np = 0, m = 0;
        } pend;
        // an observed search's events of a confirmed chunk: parents [p0e, p0e + npe) and candidates [0, me)
        auto emit = [&](u64 p0e, u64 npe, u64 me) {
            if (!ev.on)
                return;
            const std::vector<u64> prow = to_host(par + (pbase + p0e) * W, npe * W, stream);
            std::vector<u64> pid(npe);
            for (u64 p = 0; p < npe; ++p)
                pid[p] = id_at(p0e + p);
            const std::vector<u32> pa = to_host(cand_pa, me, stream);
            const std::vector<i64> ids = to_host(ev.ids, me, stream);
            const std::vector<u8> isn = to_host(ev.is_new, me, stream);
            const std::vector<u8> hit = blocked.capacity ? to_host(blocked.hit, me, stream) : std::vector<u8>{};
            std::vector<u32> cp(me);
            for (u64 j = 0; j < me; ++j)
                cp[j] = pa[j] >> abits;
            const u32 L = ga.label_width;
            std::vector<i32> bind(std::max<u32>(L, 1));
            std::vector<u64> crow(W);
            emit_batch(
                o, W, npe, prow, pid, me, cp, ids, isn, hit,
                [&](u64 j, u32* sc, const i32** bd, u32* ar) {
                    const u32 a = pa[j] & ((1u << abits) - 1);
                    *sc = ga.schema[a];
                    *ar = task.text.schemas[*sc].arity;
                    for (u32 k = 0; k < L; ++k)
                        bind[k] = static_cast<i32>(ga.binding[static_cast<size_t>(a) * L + k]);
                    *bd = bind.data();
                },
                [&](u64 j, const u64* parent) {
                    host_successor(tb.host_masks, ga, parent, pa[j] & ((1u << abits) - 1), W, crow.data());
                    return static_cast<const u64*>(crow.data());
                });
        };
        // confirms the pending chunk from the set's size and status read at the last synchronization; true if the
        // store filled inside it (the search stops there)
        auto confirm = [&](u64 size_dev, u32 status) {
            if (!pend.live)
                return false;
            pend.live = false;
            if (status & kStatusTableFull)
                throw std::length_error("mymyr_amd: brfs: state table full");
            const u64 winners = size_dev - set.size;
            const bool cuts = cut_at <= cap_states;  // a cut inside the arena (else only its capacity bounds the store)
            const u64 room = (cuts ? cut_at : cap_states) - set.size;
            // insert: every candidate's record, probe entry and slot, the parent rows, and the row each non-winner
            // compared equal to; compaction: per winner its list entry, record, slot, arena row and entry
            tm.bytes(kKInsert, pend.m * 20 + pend.np * R + (pend.m - std::min(winners, pend.m)) * R);
            tm.bytes(kKRank, pend.m * 9 + winners * 4);
            if (cuts && winners >= room && winners > 0)
            {
                // the store filled at winner room - 1 (id cut_at - 1): the search (max_states) or the layer
                // (max_next_layer_states) stops inside its parent's expansion; the compaction wrote ids below cut_at only
                tm.bytes(kKCompact, room * (2 * R + 24));
                u32 jc = 0;
                hip_check(hipMemcpyAsync(&jc, set.list + (room - 1), sizeof(u32), hipMemcpyDeviceToHost, stream), "cut");
                hip_check(hipStreamSynchronize(stream), "sync");
                u32 rec = 0;
                hip_check(hipMemcpyAsync(&rec, cand_pa + jc, sizeof(u32), hipMemcpyDeviceToHost, stream), "parent");
                hip_check(hipStreamSynchronize(stream), "sync");
                const u64 pc = rec >> abits;  // the parent, relative to the chunk's first
                row[0] += pc + 1;
                row[1] += u64{jc} + 1;
                set_small(kGoalSum, 0);
                hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(pc + 1, 256), 1024)), dim3(256), 0, stream, goal_flags + pend.p0,
                                   pc + 1, small + kGoalSum);
                if (blocked.capacity)
                {
                    set_small(kCutPruned, 0);
                    hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(u64{jc} + 1, 256), 1024)), dim3(256), 0, stream, blocked.hit,
                                       u64{jc} + 1, small + kCutPruned);
                }
                sync_small();
                layer_goals += b.host[kGoalSum];
                if (blocked.capacity)
                    layer_pruned += b.host[kCutPruned];
                emit(pend.p0, pc + 1, u64{jc} + 1);
                if (layer_cut)
                {
                    // the search goes on with the next layer: the cut winners' entries must not stand for states
                    state_set_cut(set, cut_at, stream);
                    truncated = true;
                    return true;
                }
                set.size = o.max_states;
                r.status = kOutOfStates;
                stopped = true;
                return true;
            }
            if (winners > room)
                throw std::length_error("mymyr_amd: brfs: the search needs more than " + std::to_string(cap_states) +
                                        " states of device memory (set max_states or memory_states)");
            tm.bytes(kKCompact, winners * (2 * R + 24));
            if (pend.m)
                new_rate = static_cast<double>(winners) / static_cast<double>(pend.m);
            set.size = size_dev;
            emit(pend.p0, pend.np, pend.m);
            row[0] += pend.np;
            row[1] += pend.m;
            layer_goals += b.host[kChunkGoal];
            if (blocked.capacity)
                layer_pruned += b.host[kChunkPruned];
            return false;
        };
        auto read_state = [&](const u64* block_total = nullptr) {
            hipLaunchKernelGGL(k_gather_small, dim3(1), dim3(1), 0, stream, small, int{kSizeNow}, state_set_size_now(set), int{kCut},
                               set.d_status, int{kBlockTotal}, block_total);
            launch_check("gather");
        };
        while (p0 < lim && !stopped)
        {
            if (halt.check(r.expanded + row[0], r.generated + row[1], set.size))
                break;  // the pending chunk is confirmed below; the layer ends at its last parent
            // count ahead when the counted parents past p0 hold less than a full chunk (and the layer has more)
            const bool count_now = counted < lim && counted_total - base < chunk;
            u64 nb = 0;
            if (count_now)
            {
                const u64 est = seen_parents ? std::max<u64>(1, (seen_cands + seen_parents - 1) / seen_parents) : 1;
                nb = std::min<u64>(lim - counted, std::max<u64>(u64{1} << 18, chunk / est));
                tm.begin(kKCount);
                hipLaunchKernelGGL(k_ground_count<W>, dim3(blocks_for(nb, kTW * kWave)), dim3(kTW * kWave), 0, stream, par, pbase + counted,
                                   static_cast<u32>(nb), g, goal, counts + counted * S, goal_flags + counted);
                launch_check("ground count");
                if (o.goal_test)
                    custom_goal_flags(o, par + (pbase + counted) * W, nb, W, goal_flags + counted, stream);
                tm.end(kKCount, nb * (R + 5));
                tm.begin(kKOther);
                launch_exclusive_scan(counts + counted * S, offsets + counted * S, nb * S, scan_scratch, offsets + (counted + nb) * S, stream,
                                      counted ? offsets + counted * S : nullptr);
                set_small(kFirstGoal, ~u64{0});
                hipLaunchKernelGGL(k_first_u8, dim3(std::min<u64>(blocks_for(nb, 256), 4096)), dim3(256), 0, stream, goal_flags + counted, nb,
                                   small + kFirstGoal);
                launch_check("count scan");
                tm.end(kKOther, 0);
            }
            // the chunk end over what is counted, and the pending chunk's outcome, in one synchronization
            hipLaunchKernelGGL(k_chunk_end, dim3(1), dim3(1), 0, stream, offsets, S, p0, std::min({counted + nb, lim, p0 + max_chunk_parents}),
                               base + chunk, small + kChunkP);
            launch_check("chunk end");
            read_state(count_now ? offsets + (counted + nb) * S : nullptr);
            sync_small();
            if (count_now)
            {
                const u64 total = b.host[kBlockTotal];
                seen_parents += nb;
                seen_cands += total - counted_total;
                counted_total = total;
                if (b.host[kFirstGoal] != ~u64{0})
                {
                    const u64 gi = counted + b.host[kFirstGoal];
                    if (first_goal == ~u64{0})
                        first_goal = gi;
                    if (o.stop_at_goal && gi < lim)
                    {
                        lim = gi;
                        goal_stop = true;
                    }
                }
                counted += nb;
            }
            if (confirm(b.host[kSizeNow], static_cast<u32>(b.host[kCut])))
                break;
            if (p0 >= lim)
                break;
            if (counted < lim && counted_total - base < chunk)
                continue;  // count more parents before this chunk
            u64 p1 = b.host[kChunkP], end_off = b.host[kChunkOff];
            if (p1 > lim)
            {
                // a goal found by this count ends the layer's expansion before the chunk end: the chunk ends there
                p1 = lim;
                hip_check(hipMemcpyAsync(b.host + kChunkOff, offsets + lim * S, sizeof(u64), hipMemcpyDeviceToHost, stream), "chunk end");
                hip_check(hipStreamSynchronize(stream), "sync");
                end_off = b.host[kChunkOff];
            }
            if (cut_at <= cap_states && p1 > p0 + 1)
            {
                // near a cut, a chunk of about the candidates the store's room needs at the last chunk's rate of new
                // states (with a margin): the chunk the store fills in then probes few candidates past the cut (chunk
                // boundaries change no result)
                const double room = static_cast<double>(cut_at - set.size);
                const double want = room / std::max(new_rate, 1.0 / 1024) * 1.25 + 65536.0;
                if (want < static_cast<double>(end_off - base))
                {
                    hipLaunchKernelGGL(k_chunk_end, dim3(1), dim3(1), 0, stream, offsets, S, p0, p1, base + static_cast<u64>(want), small + kChunkP);
                    launch_check("chunk end");
                    sync_small();
                    p1 = b.host[kChunkP];
                    end_off = b.host[kChunkOff];
                }
            }
            const u64 m = end_off - base;
            const u32 np = static_cast<u32>(p1 - p0);
            const ParentRows<W, false> src{par, pbase + p0, cand_pa, d_masks, abits};
            const ParentRows<W, true> src_ce{par, pbase + p0, cand_pa, d_masks, abits, g.ce_off, g.ce_meta, g.ce_soff, g.ce_slots};
            if (m > 0)
            {
                tm.begin(kKEmit);
                hipLaunchKernelGGL(k_ground_emit<W>, dim3(blocks_for(np, kTW * kWave)), dim3(kTW * kWave), 0, stream, par, pbase + p0, np, g,
                                   offsets + p0 * S, base, abits, cand_pa);
                launch_check("ground emit");
                tm.end(kKEmit, np * (R + 8) + m * 4);
                tm.begin(kKInsert);
                state_set_begin_batch(set, stream);
                if (g.ce_off)
                    hipLaunchKernelGGL((k_ground_insert<W, true>), dim3(blocks_for(m * G, kLB)), dim3(kLB), 0, stream, set.v, src_ce, m,
                                       set.flags, set.d_status, blocked, ev.cand_slot);
                else
                    hipLaunchKernelGGL((k_ground_insert<W, false>), dim3(blocks_for(m * G, kLB)), dim3(kLB), 0, stream, set.v, src, m,
                                       set.flags, set.d_status, blocked, ev.cand_slot);
                launch_check("ground insert");
                tm.end(kKInsert, 0);
                tm.begin(kKRank);
                state_set_rank(set, m, stream, ev.is_new);
                tm.end(kKRank, 0);
                // the winners' count is on the device (size next - size now); ids from max_states on are not written
                // (the store filled: the confirmation finds the cut)
                tm.begin(kKCompact);
                {
                    const dim3 grid(std::min<u64>(blocks_for(m * G, kLB), kStrideBlocks));
                    // winners past a cut are expected (the cut is confirmed on the host); past the arena an error
                    u32* const cstat = cut_at <= cap_states ? reinterpret_cast<u32*>(small + kSpare) : set.d_status;
                    const u64 climit = std::min(cut_at, cap_states);
                    if (g.ce_off)
                        hipLaunchKernelGGL((k_ground_compact<W, true>), grid, dim3(kLB), 0, stream, set.v, src_ce, m, set.list,
                                           state_set_size_now(set), state_set_size_next(set), climit, pids, nodes, cstat);
                    else
                        hipLaunchKernelGGL((k_ground_compact<W, false>), grid, dim3(kLB), 0, stream, set.v, src, m, set.list,
                                           state_set_size_now(set), state_set_size_next(set), climit, pids, nodes, cstat);
                }
                launch_check("ground compact");
                tm.end(kKCompact, 0);
                if (ev.on)
                    state_set_resolve_ids(set, ev.cand_slot, m, ev.ids, stream);
                state_set_flip(set);
            }
            // the chunk's goal states, read at the synchronization that confirms it
            set_small(kChunkGoal, 0);
            hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(np, 256), 1024)), dim3(256), 0, stream, goal_flags + p0, u64{np},
                               small + kChunkGoal);
            if (blocked.capacity)
            {
                set_small(kChunkPruned, 0);
                if (m > 0)
                    hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(m, 256), 1024)), dim3(256), 0, stream, blocked.hit, m,
                                       small + kChunkPruned);
            }
            pend = Pending{true, p0, np, m};
            p0 = p1;
            base = end_off;
            if (p0 >= lim)
                break;  // the layer's last chunk: its confirmation is the layer's last synchronization
        }
        if (!stopped && pend.live)
        {
            read_state();
            sync_small();
            confirm(b.host[kSizeNow], static_cast<u32>(b.host[kCut]));
        }
        if (halt.why)
            stopped = true;  // the time or the cancellation ended the layer after its confirmed chunks
        r.goal_states += layer_goals;
        r.pruned += layer_pruned;
        pos = layer_begin + row[0];
        r.expanded += row[0];
        r.generated += row[1];
        row[2] = set.size - size0;
        // the states this layer goal-tested: the expanded ones, plus the goal state a goal stop ends at
        const u64 tested = row[0] + ((goal_stop && !stopped && !truncated) ? 1 : 0);
        if (first_goal != ~u64{0} && first_goal < tested && r.first_goal < 0)
            r.first_goal = static_cast<i64>(id_at(first_goal));
        if (goal_stop && !stopped && !truncated)
        {
            r.goal_states += 1;  // the goal state is tested (and counted), then the search stops
            r.status = kSolved;
            stopped = true;
        }
        if (!goal_stop && !stopped && !truncated && lim < keep)
        {
            // the expansion budget ran out inside this layer
            r.status = kOutOfStates;
            budget_stopped = true;
            stopped = true;
        }
        lc.push_back(row);
        if (o.on_pass)
            o.on_pass(static_cast<u32>(lc.size() - 1), row, std::chrono::duration<double>(Clock::now() - layer_t0).count());
        if (!stopped)
            pos = layer_end;
    }
    r.states = set.size;
    r.exhausted = (!stopped && pos >= set.size) ? 1 : 0;
    // status as the reference's Control::finish (brfs.cpp:194-203): a tested goal state solves the search
    r.solved = r.first_goal >= 0 ? 1 : 0;
    if (r.solved)
        r.status = kSolved;
    else if (halt.why && !(set.size >= o.max_states && bounded))
        r.status = halt.why;
    else if (!budget_stopped)
        r.status = (r.exhausted || r.layers >= o.max_depth) ? kExhausted : kOutOfStates;
    hip_check(hipStreamSynchronize(stream), "brfs");
    r.device_s = std::chrono::duration<double>(Clock::now() - td0).count();
    tm.collect();
    if (o.fingerprint)
    {
        set_small(kFingerprint, 0);
        hipLaunchKernelGGL(k_fingerprint, dim3(std::min<u64>(blocks_for(set.size, 256), 2048)), dim3(256), 0, stream, set.v.arena,
                           set.size, static_cast<u32>(W), d_slot_cid, small + kFingerprint);
        launch_check("fingerprint");
        sync_small();
        r.fingerprint = b.host[kFingerprint];
    }
    if (r.solved)
    {
        // the plan to the first goal state tested, from the node records (first discoveries), and that state's row
        std::vector<u32> rev;
        for (u64 v = static_cast<u64>(r.first_goal);;)
        {
            u64 nd = 0;
            hip_check(hipMemcpy(&nd, nodes + v, sizeof(u64), hipMemcpyDeviceToHost), "plan node");
            if (nd == ~u64{0})
                break;
            rev.push_back(static_cast<u32>(nd));
            v = nd >> 32;
            if (rev.size() > r.layers)
                throw std::logic_error("mymyr_amd: brfs: the node records of the goal state form no path to the start");
        }
        const u32 L = ga.label_width;
        r.plan_width = L;
        for (auto it = rev.rbegin(); it != rev.rend(); ++it)
        {
            r.plan_schema.push_back(static_cast<i32>(ga.schema[*it]));
            for (u32 k = 0; k < L; ++k)
                r.plan_binding.push_back(static_cast<i32>(ga.binding[static_cast<size_t>(*it) * L + k]));
        }
        r.cost = static_cast<double>(rev.size());  // unit action costs (the device path takes tasks without a metric)
        r.goal_state.resize(W);
        hip_check(hipMemcpy(r.goal_state.data(), set.v.arena + static_cast<u64>(r.first_goal) * W, W * sizeof(u64), hipMemcpyDeviceToHost),
                  "goal state");
    }
    r.search_s = std::chrono::duration<double>(Clock::now() - t0).count();
    return r;
}
}  // namespace

namespace
{
template<int W>
BrfsResultC run_cached(const CompiledTask& task, const BrfsOptionsC& o, std::vector<std::array<u64, 3>>& lc, BrfsCache* cache)
{
    int device = 0;
    hip_check(hipGetDevice(&device), "hipGetDevice");
    const bool witness = o.witness_pruning != 0;
    if (!cache)
    {
        const auto tb = build_tables<W>(task, witness, device);
        return run<W>(task, *tb, o, lc);
    }
    const BrfsTables* tb = nullptr;
    std::unique_ptr<BrfsTables> local;
    {
        std::lock_guard lock(cache->mutex);
        std::unique_ptr<BrfsTables>& slot = cache->tables[witness ? 1 : 0];
        if (!slot)
            slot = build_tables<W>(task, witness, device);
        if (slot->device == device && slot->W == W)
            tb = slot.get();
    }
    if (!tb)
    {
        // another device than the cached tables': tables of its own for this search
        local = build_tables<W>(task, witness, device);
        tb = local.get();
    }
    return run<W>(task, *tb, o, lc);
}
}  // namespace

BrfsResultC brfs_device(const CompiledTask& task, const BrfsOptionsC& o, std::vector<std::array<u64, 3>>& layer_counts, BrfsCache* cache,
                        const TaskDev* dev, const LazyResolve* lazy)
{
    const u32 W = task.words;
    if (lazy)
    {
        if (!dev)
            throw std::invalid_argument("mymyr_amd: brfs: a task with lazy slots needs its device tables");
        return brfs_wide(task, *dev, o, layer_counts, lazy);
    }
    if (W <= 1)
        return run_cached<1>(task, o, layer_counts, cache);
    if (W <= 2)
        return run_cached<2>(task, o, layer_counts, cache);
    if (W <= 4)
        return run_cached<4>(task, o, layer_counts, cache);
    if (W <= 8)
        return run_cached<8>(task, o, layer_counts, cache);
    if (W <= 16)
        return run_cached<16>(task, o, layer_counts, cache);
    if (!dev)
        throw std::invalid_argument("mymyr_amd: brfs: states of " + std::to_string(W) + " words need the task's device tables");
    return brfs_wide(task, *dev, o, layer_counts);
}
}  // namespace mya
