// Device BrFS over rows wider than the ground driver's 16 words (brfs.hpp), for lifted tasks whose ground action lists
// are too large to test per parent (a transport instance grounds to hundreds of thousands of actions, few of them
// applicable in a state). A layer's parents are expanded by the lifted successor generator of the env path (the flat
// expansion's kernels: per parent a wave builds the state's view, counts the applicable bindings and writes each
// successor row in canonical order), in chunks whose successor rows fit the candidate buffer:
//   count    expansion pass 0 over the layer's parents: successor counts, an exclusive scan gives their offsets
//   emit     expansion pass 1 over a chunk of parents: successor rows, their parents, indices and goal flags
//   insert   the state set's probe over the candidate rows (stored equal rows drop a candidate; equal candidates keep
//            the smallest index), the winner list, and compaction: winner rows into the arena with their node records
//            (parent id, successor index: the reference's discoverer keys, src/mymyr/search/brfs.cpp:1362-1388) and
//            goal flags
// Every stored state's goal flag is written when the state is stored, so a layer's goal test reads flags. Ids, counts,
// cuts and statuses follow the ground driver (brfs.hip) and the reference's run_flat (brfs.cpp:274-404). With witness
// pruning on (the reference's default, include/mymyr/search/brfs.hpp:76) the expansion keeps, per effect-relevant
// binding of a schema with witness parameters, the one binding whose witnesses the reference's matcher finds first.

#include "brfs.hpp"
#include "brfs_common.hpp"
#include "env.hpp"
#include "runtime.hpp"
#include "scan.hpp"
#include "state_set.hpp"

#include <algorithm>
#include <cstring>

namespace mya
{
namespace
{
constexpr int kWB = 256;
constexpr u64 kWideStrideBlocks = 4096;

/// Calls f.template operator()<G, K>() for the lane-group shape of rows of W > 16 words.
template<class F>
void wide_shape(u32 W, F&& f)
{
    if (W <= 32)
        f.template operator()<16, 1>();
    else if (W <= 128)
        f.template operator()<64, 1>();
    else if (W <= 256)
        f.template operator()<64, 2>();
    else if (W <= 512)
        f.template operator()<64, 4>();
    else if (W <= 1024)
        f.template operator()<64, 8>();
    else if (W <= kLongRowWords)
        f.template operator()<64, 16>();
    else
        f.template operator()<64, 0>();  // long rows: copied from memory by a 64-lane group
}

// The chunk's winners (list order, ids from *size_now, their count size_next - size_now) below `limit` into the arena:
// candidate row list[w] becomes state id0 + w with its node record (parent id << 32 | successor index) and goal flag.
// A winner at or past `limit` sets kStatusCapacity.
template<int G, int K>
__global__ __launch_bounds__(kWB) void k_wide_compact(StateSetView s, const u64* __restrict__ rows, u64 m, const u32* __restrict__ list,
                                                     const u64* __restrict__ size_now, const u64* __restrict__ size_next, u64 limit,
                                                     const i32* __restrict__ parent, const i32* __restrict__ index,
                                                     const u8* __restrict__ goal, u64 first, const u64* __restrict__ parent_ids,
                                                     u64* __restrict__ nodes, u8* __restrict__ goal_id, u32* __restrict__ status)
{
    const u32 q = lane_id() % G;
    const u64 id0 = *size_now;
    const u64 winners = min(m, *size_next - id0);
    for (u64 w = (static_cast<u64>(blockIdx.x) * kWB + threadIdx.x) / G; w < winners; w += static_cast<u64>(gridDim.x) * (kWB / G))
    {
        const u64 id = id0 + w;
        if (id >= limit)
        {
            if (q == 0)
                atomicOr(status, kStatusCapacity);
            continue;
        }
        const u64 j = list[w];
        Slice<G, K> r;
        load_row<G, K>(rows + j * s.words, s.words, q, r);
        store_row<G, K>(s.arena + id * s.words, s.words, q, r);
        if (q == 0)
        {
            // parents gathered in an ordered layer's expansion order carry their ids in parent_ids
            const u64 p = first + static_cast<u64>(parent[j]);
            nodes[id] = ((parent_ids ? parent_ids[p] : p) << 32) | static_cast<u32>(index[j]);
            goal_id[id] = goal[j];
        }
    }
}

__global__ void k_read_u32(const u32* __restrict__ src, u64* __restrict__ dst) { *dst = *src; }

/// Rows [n, sw] into rows [n, dw] (dw >= sw), zero-padded.
__global__ void k_relayout(const u64* __restrict__ src, u32 sw, u64* __restrict__ dst, u32 dw, u64 n)
{
    for (u64 t = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; t < n * dw; t += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        const u64 i = t / dw;
        const u32 w = static_cast<u32>(t - i * dw);
        dst[t] = w < sw ? src[i * sw + w] : 0;
    }
}

/// Whether the task's goal holds in a row (host; the compiled goal lists).
bool goal_holds(const CompiledTask& task, const std::vector<u64>& row)
{
    if (task.goal_unsat)
        return false;
    auto bit = [&](u32 s) { return s / 64 < row.size() && ((row[s / 64] >> (s % 64)) & 1); };
    for (u32 s : task.goal_pos)
        if (!bit(s))
            return false;
    for (u32 s : task.goal_neg)
        if (bit(s))
            return false;
    return true;
}

}  // namespace

void custom_goal_flags(const BrfsOptionsC& o, const u64* rows, u64 n, u32 words, u8* flags, hipStream_t stream)
{
    // in pieces of at most 2^20 rows, so that the host copies stay bounded
    constexpr u64 kPiece = u64{1} << 20;
    std::vector<u8> f;
    for (u64 i0 = 0; i0 < n; i0 += kPiece)
    {
        const u64 m = std::min(kPiece, n - i0);
        const std::vector<u64> h = to_host(rows + i0 * words, m * words, stream);
        f.assign(m, 0);
        if (!o.goal_test(h.data(), m, words, f.data()))
            throw std::runtime_error("mymyr_amd: brfs: the goal test failed");
        for (u8& x : f)
            x = x ? 1 : 0;
        hip_check(hipMemcpyAsync(flags + i0, f.data(), m, hipMemcpyHostToDevice, stream), "goal flags");
        hip_check(hipStreamSynchronize(stream), "goal flags");
    }
}

bool any_of_holds(const BrfsOptionsC& o, const u64* row, u32 words)
{
    auto bit = [&](u32 s) { return s / 64 < words && ((row[s / 64] >> (s % 64)) & 1); };
    for (size_t k = 0; k < o.goal_pos.size(); ++k)
    {
        bool ok = true;
        for (u32 s : o.goal_pos[k])
            ok = ok && bit(s);
        for (u32 s : o.goal_neg[k])
            ok = ok && !bit(s);
        if (ok)
            return true;
    }
    return false;
}

BrfsResultC brfs_wide(const CompiledTask& task, const TaskDev& dev, const BrfsOptionsC& o, std::vector<std::array<u64, 3>>& lc,
                      const LazyResolve* lazy)
{
    TaskDev T = dev;  // lazy slots: refreshed after each interning
    const u32 TW0 = task.words;  // the width of the start and blocked rows
    u32 W = lazy ? lazy_row_words(TW0) : TW0;
    BrfsResultC r;
    const auto t0 = Clock::now();
    hipStream_t stream = thread_stream();
    Timers tm(o.timings != 0, stream, r);
    u64 R = static_cast<u64>(W) * 8;
    Buffers b(stream);
    const bool bounded = o.max_states != ~u64{0};
    // unbounded searches: an arena of at most 32 GiB by default (lazy slots: for rows of the task's largest width)
    const u64 R_max = lazy ? static_cast<u64>(lazy_row_words(words_for(task.layout.fluent_count))) * 8 : R;
    const u64 cap_states = bounded ? std::max<u64>(1, o.max_states)
                                   : (o.memory_states ? o.memory_states : std::min<u64>(u64{1} << 26, (u64{32} << 30) / R_max));
    // candidate rows per chunk: about 4 GiB of them by default
    auto chunk_for = [&](u64 row_bytes) {
        const u64 c = o.chunk ? o.chunk : std::clamp<u64>((u64{4} << 30) / row_bytes, u64{1} << 12, u64{1} << 22);
        return std::min<u64>(c, kMaxBatch - 1);
    };
    u64 chunk = chunk_for(R);
    StateSet set;
    state_set_create(set, cap_states, W, 0.5, chunk, stream, chunk);
    struct SetGuard
    {
        StateSet& s;
        hipStream_t st;
        ~SetGuard() { state_set_destroy(s, st); }
    } setg{set, stream};
    const u64 layer_cap = cap_states;
    u32* counts = b.alloc<u32>(layer_cap, "layer counts");
    u64* offsets = b.alloc<u64>(layer_cap + 1, "layer offsets");
    u64* scan_scratch = b.alloc<u64>(scan_scratch_words(layer_cap), "scan scratch");
    u8* goal_id = b.alloc<u8>(cap_states, "goal flags");
    u64* nodes = b.alloc<u64>(cap_states, "search nodes");
    u64* small = b.alloc<u64>(kSmall, "scalars");
    u32* xstatus = b.alloc<u32>(2, "expansion status");  // [0] words needed, [1] status
    b.host = static_cast<u64*>(pinned_acquire(kSmall * sizeof(u64)));
    // candidate buffers of one chunk (the state set's batch arrays hold as many)
    u64* cand_rows = b.alloc<u64>(chunk * W, "candidate rows");
    i32* cand_parent = b.alloc<i32>(chunk, "candidate parents");
    i32* cand_index = b.alloc<i32>(chunk, "candidate indices");
    u8* cand_goal = b.alloc<u8>(chunk, "candidate goal flags");
    auto memory_bytes = [&] { return set.v.capacity * 8 + cap_states * (R + 8 + 1) + layer_cap * (4 + 8 + 8) + chunk * (R + 4 + 4 + 1 + 1 + 4); };
    r.memory_bytes = memory_bytes();
    enum
    {
        kFirstGoal = 0,
        kChunkP = 1,  // chunk end parent, then its offset
        kChunkOff = 2,
        kSizeNow = 3,
        kStatus = 4,
        kTotal = 5,
        kGoalSum = 6,
        kFingerprint = 7,
        kSpare = 8,  // the capacity status of a cut chunk's compaction (expected there, not an error)
        kXStatus = 9,
        kPruned = 10,  // blocked candidates of a chunk (up to the cut of a cut chunk)
    };
    auto set_small = [&](int idx, u64 v) { hipLaunchKernelGGL(k_set_u64, dim3(1), dim3(1), 0, stream, small + idx, v); };
    auto sync_small = [&] {
        hip_check(hipMemcpyAsync(b.host, small, kSmall * sizeof(u64), hipMemcpyDeviceToHost, stream), "read scalars");
        hip_check(hipStreamSynchronize(stream), "sync");
    };
    auto read_state = [&](const u64* total) {
        hipLaunchKernelGGL(k_gather_small, dim3(1), dim3(1), 0, stream, small, int{kSizeNow}, state_set_size_now(set), int{kStatus},
                           set.d_status, int{kTotal}, total);
        hipLaunchKernelGGL(k_read_u32, dim3(1), dim3(1), 0, stream, xstatus + 1, small + kXStatus);
        launch_check("gather");
    };
    auto check_expansion = [&] {
        if (b.host[kXStatus] & ~u64{kStatusWideRow})
            throw std::runtime_error("mymyr_amd: brfs: expansion status " + std::to_string(b.host[kXStatus]));
        if (b.host[kStatus] & kStatusTableFull)
            throw std::length_error("mymyr_amd: brfs: state table full");
    };
    launch_fill_u32(xstatus, 2, 0, stream);
    BlockedView blocked = upload_blocked(o.blocked, TW0, W, chunk, b, stream);
    // an observed search's events: per candidate its probe result, id, new flag and action label
    EventBuffers ev;
    ev.init(o.observed(), chunk, b);
    const u32 EL = std::max<u32>(1, task.label_width);
    i32* ev_schema = ev.on ? b.alloc<i32>(chunk, "event schemas") : nullptr;
    i32* ev_binding = ev.on ? b.alloc<i32>(chunk * EL, "event bindings") : nullptr;
    // the start state (stored even if blocked)
    {
        const std::vector<u64> s0 = start_row(task, o, W);
        u64* d_s0 = b.alloc<u64>(W, "start state");
        hip_check(hipMemcpyAsync(d_s0, s0.data(), W * sizeof(u64), hipMemcpyHostToDevice, stream), "start state");
        u64 nn = 0;
        state_set_insert(set, d_s0, 1, nullptr, nullptr, &nn, stream);
        hipLaunchKernelGGL(k_set_u64, dim3(1), dim3(1), 0, stream, nodes, ~u64{0});
        const u8 g0 = (o.any_of ? any_of_holds(o, s0.data(), static_cast<u32>(s0.size())) : goal_holds(task, s0)) ? 1 : 0;
        hip_check(hipMemcpyAsync(goal_id, &g0, 1, hipMemcpyHostToDevice, stream), "start goal");
        hip_check(hipStreamSynchronize(stream), "start state");
    }
    ExpandArgs base_args{};
    base_args.T = T;
    base_args.words = W;
    base_args.out_words = W;
    base_args.label_width = 0;
    base_args.status = xstatus + 1;
    base_args.words_needed = xstatus;
    // witness pruning (the reference's default): one successor per effect-relevant binding, with the witnesses the
    // matcher binds first (tasks whose schemas have no witness parameter expand the same either way)
    base_args.witness = o.witness_pruning && T.witness ? 1 : 0;
    base_args.any_goal = upload_any_of(o, b, stream);
    // lazy slots: the stored states move to a set of rows of nw words in id order (so their ids stay), a chunk at a
    // time through new candidate rows of that width; the blocked table follows the width
    auto widen = [&](u32 nw) {
        const u64 nchunk = chunk_for(static_cast<u64>(nw) * 8);
        u64* rows = b.alloc<u64>(nchunk * nw, "candidate rows");
        StateSet grown;
        state_set_create(grown, cap_states, nw, 0.5, nchunk, stream, nchunk);
        for (u64 i = 0; i < set.size; i += nchunk)
        {
            const u64 k = std::min(nchunk, set.size - i);
            hipLaunchKernelGGL(k_relayout, dim3(std::min<u64>(blocks_for(k * nw, 256), 4096)), dim3(256), 0, stream, set.v.arena + i * W, W,
                               rows, nw, k);
            launch_check("relayout");
            u64 nn = 0;
            state_set_insert(grown, rows, k, nullptr, nullptr, &nn, stream);
            if (nn != k)
                throw std::logic_error("mymyr_amd: brfs: stored states merged when their rows were widened");
        }
        state_set_destroy(set, stream);
        set = grown;
        b.release(cand_rows);
        cand_rows = rows;
        W = nw;
        R = static_cast<u64>(nw) * 8;
        chunk = nchunk;
        blocked = upload_blocked(o.blocked, TW0, W, chunk, b, stream);
        base_args.words = W;
        base_args.out_words = W;
        r.memory_bytes = std::max(r.memory_bytes, memory_bytes());
    };
    const auto td0 = Clock::now();
    Halt halt(o, t0);
    LayerOrder lorder(o);
    LayerRows lrows(stream);
    GrowBuf<u8> lgoal(stream);  // an ordered layer's goal flags in its expansion order
    bool stopped = false, budget_stopped = false;
    r.status = kExhausted;
    u64 pos = 0;
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
        const u64 lb = pos, le = set.size, ln = le - lb;
        std::array<u64, 3> row{0, 0, 0};
        const auto layer_t0 = Clock::now();
        const u64 size0 = set.size;
        // parent rows and goal flags: the layer's in the arena, or an ordered layer's gathered in its expansion order
        // (positions below are then expansion positions)
        const bool ordered = lorder.ordered() && lb > 0;
        u64 keep = ln;
        if (o.goal_test)
            custom_goal_flags(o, set.v.arena + lb * W, ln, W, goal_id + lb, stream);
        const u8* gflags = goal_id + lb;
        if (ordered)
        {
            lrows.order(lorder, o, task, set.v.arena, lb, ln, W, stream);
            keep = lrows.ids.size();
            u8* g = lgoal.get(keep, "ordered layer goal flags");
            if (keep)
                hipLaunchKernelGGL(k_gather_u8, dim3(std::min<u64>(blocks_for(keep, 256), 4096)), dim3(256), 0, stream, goal_id + lb,
                                   lrows.d_ids.p, lb, keep, g);
            launch_check("ordered layer goal flags");
            gflags = g;
        }
        auto parents = [&](u64 p) { return ordered ? lrows.rows.p + p * W : set.v.arena + (lb + p) * W; };
        auto id_at = [&](u64 p) { return ordered ? lrows.ids[p] : lb + p; };
        // an observed search's events of a confirmed chunk: parents [p0e, p0e + npe) and candidates [0, me)
        auto emit = [&](u64 p0e, u64 npe, u64 me) {
            if (!ev.on)
                return;
            const std::vector<u64> prow = to_host(parents(p0e), npe * W, stream);
            std::vector<u64> pid(npe);
            for (u64 p = 0; p < npe; ++p)
                pid[p] = id_at(p0e + p);
            const std::vector<i32> par_rel = to_host(cand_parent, me, stream);
            std::vector<u32> cp(par_rel.begin(), par_rel.end());
            const std::vector<i64> ids = to_host(ev.ids, me, stream);
            const std::vector<u8> isn = to_host(ev.is_new, me, stream);
            const std::vector<u8> hit = blocked.capacity ? to_host(blocked.hit, me, stream) : std::vector<u8>{};
            const std::vector<i32> sch = to_host(ev_schema, me, stream);
            const std::vector<i32> bnd = to_host(ev_binding, me * EL, stream);
            const std::vector<u64> rows = to_host(cand_rows, me * W, stream);
            emit_batch(
                o, W, npe, prow, pid, me, cp, ids, isn, hit,
                [&](u64 j, u32* sc, const i32** bd, u32* ar) {
                    *sc = static_cast<u32>(sch[j]);
                    *ar = task.text.schemas[*sc].arity;
                    *bd = bnd.data() + j * EL;
                },
                [&](u64 j, const u64*) { return rows.data() + j * W; });
        };
        u64 cut_at = bounded ? o.max_states : ~u64{0};
        bool layer_cut = false, truncated = false;
        if (lorder.limited() && le + o.max_next_layer_states < cut_at)
        {
            cut_at = le + o.max_next_layer_states;
            layer_cut = true;
        }
        const u64 budget = o.max_expanded == ~u64{0} ? ~u64{0} : o.max_expanded - r.expanded;
        u64 lim = std::min(keep, budget);
        // the layer's first goal state among the parents to expand, and their successor counts
        set_small(kFirstGoal, ~u64{0});
        hipLaunchKernelGGL(k_first_u8, dim3(std::min<u64>(blocks_for(lim, 256), 4096)), dim3(256), 0, stream, gflags, lim,
                           small + kFirstGoal);
        launch_check("goal search");
        tm.begin(kKCount);
        ExpandArgs a = base_args;
        a.states = parents(0);
        a.rows = lim;
        a.pass = 0;
        a.counts = counts;
        launch_expand(a, stream);
        tm.end(kKCount, lim * (R + 4));
        tm.begin(kKOther);
        launch_exclusive_scan(counts, offsets, lim, scan_scratch, offsets + lim, stream);
        tm.end(kKOther, 0);
        read_state(offsets + lim);
        sync_small();
        check_expansion();
        const u64 first_goal = b.host[kFirstGoal];
        bool goal_stop = false;
        if (first_goal != ~u64{0} && o.stop_at_goal && first_goal < lim)
        {
            lim = first_goal;
            goal_stop = true;
        }
        u64 layer_goals = 0, layer_pruned = 0;
        u64 p0 = 0, base = 0;
        while (p0 < lim && !stopped)
        {
            if (halt.check(r.expanded + row[0], r.generated + row[1], set.size))
                break;
            hipLaunchKernelGGL(k_chunk_end, dim3(1), dim3(1), 0, stream, offsets, 1u, p0, lim, base + chunk, small + kChunkP);
            launch_check("chunk end");
            sync_small();
            const u64 p1 = b.host[kChunkP], end_off = b.host[kChunkOff];
            const u64 m = end_off - base;
            if (m > chunk)
                throw std::length_error("mymyr_amd: brfs: a state has " + std::to_string(m) + " successors, more than a chunk of " +
                                        std::to_string(chunk) + " candidates holds (raise the chunk option)");
            if (m > 0)
            {
                tm.begin(kKEmit);
                ExpandArgs e = base_args;
                e.states = parents(p0);
                e.rows = p1 - p0;
                e.pass = 1;
                e.offsets = offsets + p0;
                e.offset_base = base;
                e.capacity = m;
                e.succ = cand_rows;
                e.parent = cand_parent;
                e.index = cand_index;
                e.goal = cand_goal;
                e.counts = counts + p0;
                if (ev.on)
                {
                    e.schema = ev_schema;
                    e.binding = ev_binding;
                    e.label_width = EL;
                }
                launch_expand(e, stream);
                tm.end(kKEmit, (p1 - p0) * R + m * (R + 9));
                if (lazy)
                {
                    // added atoms without a slot: intern them (ascending canonical id), widen the rows if the task's
                    // rows outgrew them, and expand the chunk again (nothing of it is stored yet)
                    read_state(nullptr);
                    sync_small();
                    if (b.host[kXStatus] & kStatusNoSlot)
                    {
                        launch_fill_u32(xstatus, 2, 0, stream);
                        if (!(*lazy)(stream, &T))
                            throw std::logic_error("mymyr_amd: brfs: an added atom without a slot was not recorded");
                        base_args.T = T;
                        if (lazy_row_words(task.words) > W)
                        {
                            widen(lazy_row_words(task.words));
                            if (ordered)
                                lrows.gather(set.v.arena, W, stream);  // the ordered rows at the new width
                        }
                        continue;
                    }
                }
                tm.begin(kKInsert);
                state_set_begin_batch(set, stream);
                state_set_probe(set, cand_rows, m, stream, blocked.capacity ? &blocked : nullptr, ev.cand_slot);
                tm.end(kKInsert, m * (R + 8));
                tm.begin(kKRank);
                state_set_rank(set, m, stream, ev.is_new);
                tm.end(kKRank, m * 9);
                tm.begin(kKCompact);
                set_small(kSpare, 0);
                wide_shape(W, [&]<int G, int K>() {
                    hipLaunchKernelGGL((k_wide_compact<G, K>), dim3(std::min<u64>(blocks_for(m * G, kWB), kWideStrideBlocks)), dim3(kWB), 0, stream,
                                       set.v, cand_rows, m, set.list, state_set_size_now(set), state_set_size_next(set),
                                       std::min(cut_at, cap_states), cand_parent, cand_index, cand_goal, ordered ? p0 : lb + p0,
                                       ordered ? lrows.d_ids.p : nullptr, nodes, goal_id,
                                       cut_at <= cap_states ? reinterpret_cast<u32*>(small + kSpare) : set.d_status);
                });
                launch_check("wide compact");
                tm.end(kKCompact, 0);
                if (ev.on)
                    state_set_resolve_ids(set, ev.cand_slot, m, ev.ids, stream);
                state_set_flip(set);
            }
            // the chunk's goal parents, its outcome and the expansion's status in one synchronization
            set_small(kGoalSum, 0);
            hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(p1 - p0, 256), 1024)), dim3(256), 0, stream, gflags + p0,
                               p1 - p0, small + kGoalSum);
            if (blocked.capacity)
            {
                set_small(kPruned, 0);
                if (m > 0)
                    hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(m, 256), 1024)), dim3(256), 0, stream, blocked.hit, m,
                                       small + kPruned);
            }
            read_state(nullptr);
            sync_small();
            check_expansion();
            const u64 size_dev = b.host[kSizeNow];
            const u64 winners = size_dev - set.size;
            const bool cuts = cut_at <= cap_states;  // a cut inside the arena (else only its capacity bounds the store)
            const u64 room = (cuts ? cut_at : cap_states) - set.size;
            tm.bytes(kKCompact, std::min(winners, room) * (2 * R + 21));
            if (cuts && winners >= room && winners > 0)
            {
                // the store filled at winner room - 1 (id cut_at - 1): the search (max_states) or the layer
                // (max_next_layer_states) stops inside its parent's expansion
                u32 jc = 0;
                hip_check(hipMemcpy(&jc, set.list + (room - 1), sizeof(u32), hipMemcpyDeviceToHost), "cut");
                i32 pc = 0;
                hip_check(hipMemcpy(&pc, cand_parent + jc, sizeof(i32), hipMemcpyDeviceToHost), "cut parent");
                row[0] += static_cast<u64>(pc) + 1;
                row[1] += u64{jc} + 1;
                set_small(kGoalSum, 0);
                hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(static_cast<u64>(pc) + 1, 256), 1024)), dim3(256), 0, stream,
                                   gflags + p0, static_cast<u64>(pc) + 1, small + kGoalSum);
                if (blocked.capacity)
                {
                    set_small(kPruned, 0);
                    hipLaunchKernelGGL(k_sum_u8, dim3(std::min<u64>(blocks_for(u64{jc} + 1, 256), 1024)), dim3(256), 0, stream, blocked.hit,
                                       u64{jc} + 1, small + kPruned);
                }
                sync_small();
                layer_goals += b.host[kGoalSum];
                if (blocked.capacity)
                    layer_pruned += b.host[kPruned];
                emit(p0, static_cast<u64>(pc) + 1, u64{jc} + 1);
                if (layer_cut)
                {
                    // the search goes on with the next layer: the cut winners' entries must not stand for states
                    state_set_cut(set, cut_at, stream);
                    truncated = true;
                    break;
                }
                set.size = o.max_states;
                r.status = kOutOfStates;
                stopped = true;
                break;
            }
            if (winners > room)
                throw std::length_error("mymyr_amd: brfs: the search needs more than " + std::to_string(cap_states) +
                                        " states of device memory (set max_states or memory_states)");
            set.size = size_dev;
            emit(p0, p1 - p0, m);
            row[0] += p1 - p0;
            row[1] += m;
            layer_goals += b.host[kGoalSum];
            if (blocked.capacity)
                layer_pruned += b.host[kPruned];
            p0 = p1;
            base = end_off;
        }
        if (halt.why)
            stopped = true;  // the time or the cancellation ended the layer after its last full chunk
        r.goal_states += layer_goals;
        r.pruned += layer_pruned;
        pos = lb + row[0];
        r.expanded += row[0];
        r.generated += row[1];
        row[2] = set.size - size0;
        const u64 tested = row[0] + ((goal_stop && !stopped && !truncated) ? 1 : 0);
        if (first_goal != ~u64{0} && first_goal < tested && r.first_goal < 0)
            r.first_goal = static_cast<i64>(id_at(first_goal));
        if (goal_stop && !stopped && !truncated)
        {
            r.goal_states += 1;
            r.status = kSolved;
            stopped = true;
        }
        if (!goal_stop && !stopped && !truncated && lim < keep)
        {
            r.status = kOutOfStates;
            budget_stopped = true;
            stopped = true;
        }
        lc.push_back(row);
        if (o.on_pass)
            o.on_pass(static_cast<u32>(lc.size() - 1), row, std::chrono::duration<double>(Clock::now() - layer_t0).count());
        if (!stopped)
            pos = le;
    }
    r.states = set.size;
    r.exhausted = (!stopped && pos >= set.size) ? 1 : 0;
    r.solved = r.first_goal >= 0 ? 1 : 0;
    if (r.solved)
        r.status = kSolved;
    else if (halt.why && !(bounded && set.size >= o.max_states))
        r.status = halt.why;
    else if (!budget_stopped)
        r.status = (r.exhausted || r.layers >= o.max_depth) ? kExhausted : kOutOfStates;
    hip_check(hipStreamSynchronize(stream), "brfs");
    r.device_s = std::chrono::duration<double>(Clock::now() - td0).count();
    tm.collect();
    if (o.fingerprint)
    {
        const u64* d_slot_cid = nullptr;
        if (task.mode != AtomMode::Dense)
        {
            u64* c = b.alloc<u64>(task.slot_cid.size(), "slot canonical ids");
            hip_check(hipMemcpy(c, task.slot_cid.data(), task.slot_cid.size() * sizeof(u64), hipMemcpyHostToDevice), "slot ids");
            d_slot_cid = c;
        }
        set_small(kFingerprint, 0);
        hipLaunchKernelGGL(k_fingerprint, dim3(std::min<u64>(blocks_for(set.size, 256), 2048)), dim3(256), 0, stream, set.v.arena,
                           set.size, W, d_slot_cid, small + kFingerprint);
        launch_check("fingerprint");
        sync_small();
        r.fingerprint = b.host[kFingerprint];
    }
    if (r.solved)
    {
        // the plan from the node records: each names its parent and the successor's index in the parent's canonical
        // order; the label is that successor of the parent's expansion, generated again (brfs.cpp:1362-1388)
        std::vector<std::pair<u64, u32>> rev;
        for (u64 v = static_cast<u64>(r.first_goal);;)
        {
            u64 nd = 0;
            hip_check(hipMemcpy(&nd, nodes + v, sizeof(u64), hipMemcpyDeviceToHost), "plan node");
            if (nd == ~u64{0})
                break;
            rev.push_back({nd >> 32, static_cast<u32>(nd)});
            v = nd >> 32;
            if (rev.size() > r.layers)
                throw std::logic_error("mymyr_amd: brfs: the node records of the goal state form no path to the start");
        }
        const u32 L = std::max<u32>(1, task.label_width);
        r.plan_width = L;
        u64* zero = b.alloc<u64>(1, "plan offset");
        hip_check(hipMemset(zero, 0, sizeof(u64)), "plan offset");
        for (auto it = rev.rbegin(); it != rev.rend(); ++it)
        {
            ExpandArgs a = base_args;
            a.states = set.v.arena + it->first * W;
            a.rows = 1;
            a.pass = 0;
            a.counts = counts;
            launch_expand(a, stream);
            u32 c = 0;
            hip_check(hipMemcpyAsync(&c, counts, sizeof(u32), hipMemcpyDeviceToHost, stream), "plan count");
            hip_check(hipStreamSynchronize(stream), "plan count");
            if (it->second >= c)
                throw std::logic_error("mymyr_amd: brfs: a node record names a successor its parent does not have");
            i32* sch = b.alloc<i32>(c, "plan schemas");
            i32* bnd = b.alloc<i32>(static_cast<u64>(c) * L, "plan bindings");
            ExpandArgs e = a;
            e.pass = 1;
            e.offsets = zero;
            e.capacity = c;
            e.schema = sch;
            e.binding = bnd;
            e.label_width = L;
            launch_expand(e, stream);
            std::vector<i32> lab(1 + L);
            hip_check(hipMemcpyAsync(lab.data(), sch + it->second, sizeof(i32), hipMemcpyDeviceToHost, stream), "plan schema");
            hip_check(hipMemcpyAsync(lab.data() + 1, bnd + static_cast<u64>(it->second) * L, L * sizeof(i32), hipMemcpyDeviceToHost, stream),
                      "plan binding");
            hip_check(hipStreamSynchronize(stream), "plan label");
            r.plan_schema.push_back(lab[0]);
            r.plan_binding.insert(r.plan_binding.end(), lab.begin() + 1, lab.end());
        }
        r.cost = static_cast<double>(rev.size());
        r.goal_state.resize(task.words);
        hip_check(hipMemcpy(r.goal_state.data(), set.v.arena + static_cast<u64>(r.first_goal) * W, task.words * sizeof(u64),
                            hipMemcpyDeviceToHost), "goal state");
    }
    r.search_s = std::chrono::duration<double>(Clock::now() - t0).count();
    return r;
}
}  // namespace mya
