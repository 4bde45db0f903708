#pragma once
// Layer-synchronous breadth-first search on the device, bit-exact with the reference's BrFS (src/mymyr/search/brfs.cpp:
// run_flat 274-404 and brfs() 1809-1931): ids are ranks of first discovery by (parent id, successor index), every
// expanded state is goal-tested, layer_counts[d] = {expanded, generated, new}, max_states stops at the state that fills
// the store inside its parent's expansion, max_depth stores but does not expand the states of depth max_depth, and
// fingerprint = XOR over ids of mix64(id * phi ^ canonical_hash(state)) (brfs.cpp:34-37, task.cpp:387-404).

#include "task.hpp"

#include <hip/hip_runtime.h>

#include <array>
#include <functional>
#include <memory>
#include <mutex>
#include <vector>

namespace mya
{
struct BrfsOptionsC
{
    u32 max_depth = ~u32{0};
    i32 witness_pruning = 1;
    u64 max_states = ~u64{0};
    u64 max_expanded = ~u64{0};
    i32 stop_at_goal = 1;
    i32 fingerprint = 0;
    u64 chunk = 0;          // candidates per device batch (0: automatic)
    u64 memory_states = 0;  // arena capacity when max_states is unbounded (0: automatic)
    i32 timings = 0;        // time every kernel class with HIP events on the search's stream
    std::vector<u64> start;    // [task words] the start state (empty: the task's initial state)
    std::vector<u64> blocked;  // [k, task words] states never stored (the start state exempt)
    bool timed = false;        // stop with OutOfTime once max_seconds have passed
    double max_seconds = 0;
    const volatile i32* cancel = nullptr;  // stop with Cancelled once another thread sets it nonzero
    // BrfsOptions::goal as GoalSpec::AnyOf (include/mymyr/search/control.hpp:93-118): a state is a goal iff one of the
    // goals' positive slots all hold and its negative ones none (the goals that can never hold left out, so no goal at
    // all makes no state a goal); any_of false: the task's goal
    bool any_of = false;
    std::vector<std::vector<u32>> goal_pos, goal_neg;
    // the observer's events sent from inside the search (SearchObserver::on_pass and on_progress,
    // include/mymyr/search/control.hpp:157-186): the end of a layer with its {expanded, generated, new} counts and
    // seconds; before a batch once progress_interval more states were expanded, false stopping the search (Cancelled)
    std::function<void(u32 layer, const std::array<u64, 3>& counts, double seconds)> on_pass;
    std::function<bool(u64 expanded, u64 generated, u64 states, double seconds)> on_progress;
    u64 progress_interval = u64{1} << 16;
    // the per-state events (SearchObserver::on_expand, on_generate, on_prune), sent batch by batch in the reference's
    // order; child ~0: none (a blocked successor)
    std::function<void(u64 id, const u64* row, u32 words)> on_expand;
    std::function<void(u64 parent, u32 schema, const i32* binding, u32 arity, u64 child, const u64* row, u32 words, bool is_new)>
        on_generate;
    std::function<void(u64 parent, u32 schema, const i32* binding, u32 arity, const u64* row, u32 words)> on_prune;
    [[nodiscard]] bool observed() const { return on_expand || on_generate || on_prune; }
    // BrfsOptions::layers (include/mymyr/search/layer_ordering.hpp:63-113): kind 0 queue, 1 in order, 2 reverse,
    // 3 randomized, 4 goal count, 5 scored (the reference's Kind order); ~0: no limit / no beam
    i32 layer_kind = 0;
    u64 layer_seed = 0;
    u32 max_next_layer_states = ~u32{0};
    bool prefer_more_satisfied_goals = true;
    u32 beam_width = ~u32{0};
    bool randomize_ties = false;
    // scored layers: scores[i] of the layer's rows [n, words] (host), lower first
    std::function<void(const u64* rows, u64 n, u32 words, double* scores)> scorer;
    // GoalSpec::Custom: out[i] = whether host row i of [n, words] is a goal (instead of the task's goal or any_of); false
    // from it is an error that stops the search
    std::function<bool(const u64* rows, u64 n, u32 words, u8* out)> goal_test;
};

/// The custom goal test of rows [n, words] on the device into goal flags (device): a host round trip (BrfsOptionsC::goal_test).
void custom_goal_flags(const BrfsOptionsC& o, const u64* rows, u64 n, u32 words, u8* flags, hipStream_t stream);

/// Whether one of the AnyOf goals holds in a row of `words` words (host).
bool any_of_holds(const BrfsOptionsC& o, const u64* row, u32 words);

/// Kernel classes of the device BrFS (timed with HIP events when BrfsOptionsC::timings is set).
enum BrfsKernel : int
{
    kKCount = 0,    // applicability counts and goal flags of a block of parents
    kKEmit = 1,     // (parent, action) records of the successors, in candidate order
    kKInsert = 2,   // successor rows, hashes and the state-set probe (stored and pending equals, min-candidate winner)
    kKUnused = 3,
    kKRank = 4,     // winner flags and their exclusive scan
    kKCompact = 5,  // new states into the arena and the table
    kKOther = 6,    // scans of counts, goal searches, chunk bounds, fingerprint
    kKClasses = 7,
};

struct BrfsResultC
{
    i32 status = 0;  // SearchStatus of the reference (search/control.hpp:28-37)
    i32 solved = 0;
    i32 exhausted = 0;
    u32 layers = 0;
    u64 states = 0, expanded = 0, generated = 0, goal_states = 0, fingerprint = 0;
    i64 first_goal = -1;
    double search_s = 0;
    double device_s = 0;
    double kernel_ms[kKClasses] = {};
    u64 kernel_bytes[kKClasses] = {};  // algorithmic bytes per class (the per-launch formulas in brfs.hip)
    u64 kernel_launches[kKClasses] = {};
    u64 pruned = 0;        // successors equal to a blocked state
    u64 memory_bytes = 0;  // device bytes of the search's buffers (state set, arena, nodes, chunk and layer arrays)
    // a solved search: the plan to the first goal state tested as (schema, binding) labels ([len], [len, plan_width]
    // objects, -1 padded past a schema's arity), its cost and the goal state's words
    std::vector<i32> plan_schema;
    std::vector<i32> plan_binding;
    u32 plan_width = 0;
    double cost = 0;
    std::vector<u64> goal_state;
};

enum SearchStatus : i32
{
    kSolved = 0,
    kExhausted = 1,
    kOutOfStates = 2,
    kOutOfTime = 3,
    kCancelled = 4,
    kFailed = 5,
    kUnsolvable = 6,
};

/// Runs the BrFS on the current device; fills layer_counts with {expanded, generated, new} per expanded layer.
/// The device tables of a task's ground actions (grounding, witness dominators, fast precondition records, effect
/// masks, goal and slot tables), built on the first search per witness-pruning setting and device and kept with the
/// task: repeated searches skip grounding and uploads. Built under the mutex; read-only afterwards.
struct BrfsTables;
struct BrfsCache
{
    std::mutex mutex;
    std::unique_ptr<BrfsTables> tables[2];
    BrfsCache();
    ~BrfsCache();
};

struct TaskDev;

/// Lazy slots: interns the atoms the successor kernels recorded without a slot, brings the task's device image up to
/// date and stores its new pointer table in *T; returns whether any atom was interned.
using LazyResolve = std::function<bool(hipStream_t, TaskDev*)>;

/// Rows of at most 16 words: over the ground actions (brfs.hip). Wider rows, and tasks with lazy slots (`lazy` set):
/// over the lifted expansion (brfs_wide.hip), which needs the task's device tables `dev`.
BrfsResultC brfs_device(const CompiledTask& task, const BrfsOptionsC& o, std::vector<std::array<u64, 3>>& layer_counts,
                        BrfsCache* cache = nullptr, const TaskDev* dev = nullptr, const LazyResolve* lazy = nullptr);

/// The BrFS over the lifted expansion (witness pruning only for tasks without witness parameters). With lazy slots the
/// rows start at the task's current width (rounded up: lazy_row_words) and are widened, the stored states moved to
/// a set of the new width, when interned atoms outgrow them.
BrfsResultC brfs_wide(const CompiledTask& task, const TaskDev& dev, const BrfsOptionsC& o, std::vector<std::array<u64, 3>>& layer_counts,
                      const LazyResolve* lazy = nullptr);

/// Row words of a search over a task with lazy slots whose states have `words` words: powers of two through 64 words,
/// then whole multiples of 64 (the reference's arena buckets, cuda/src/brfs.cpp:33-34).
inline u32 lazy_row_words(u32 words)
{
    if (words > 64)
        return (words + 63) / 64 * 64;
    u32 w = 1;
    while (w < words)
        w *= 2;
    return w;
}
}  // namespace mya
