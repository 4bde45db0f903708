#pragma once
// The batched environment step on the device, bit-exact with HostEnv::step_row_impl (src/mymyr/rl/env.cpp:351-528):
// choose (given index or Philox draw over the canonical successor order), move, goal, dead end, reward, termination,
// truncation, successor count of the reached state, SAME_STEP autoreset. One wavefront per environment row, several
// waves per block sharing the LDS copy of the task's hot tables.

#include "lifted.hpp"

#include <hip/hip_runtime.h>

namespace mya
{
struct EnvCfg
{
    u32 max_steps;
    float step_reward, goal_reward, dead_end_reward;
    i32 dead_end_none;      // DeadEnd::None
    i32 dead_end_terminal;
    i32 autoreset;
};

/// What a step and a reset need of an instance besides its tables (device): the initial state, its count-cache row
/// and schema masks, and the goal as masks over the instance's words.
struct InstDev
{
    const u64* initial;     // [W]
    const u32* init_cache;  // [num_schemas + 2]
    const u8* init_masks;   // [num_schemas]
    const u64* goal_pos;    // [W]
    const u64* goal_neg;    // [W]
    u32 W;
    u32 init_count;
    u32 init_goal;
    u32 fluent_slots;
    u32 variant;  // the kernel variant that runs the instance's rows (staged | levels << 1)
    u32 reserved;
    u64 init_hash;  // hash_state of the initial state (its visited-table key)
};

/// Per-row visited tables (rl/visited.hpp): [rows, capacity] u64 keys by linear probing, counts [rows], a sticky
/// overflow status word ([1], or [rows] per row).
struct VisitedDev
{
    u64* table;
    i32* count;
    i32* status;
    u32 capacity;  // 0: no tables
    u32 status_per_row;
};

/// Rows of a batch over several instances grouped by instance (a counting sort of the task ids): order lists the rows
/// of instance 0, then of instance 1, ...; instance k's rows are order[starts[k], starts[k + 1]), cut into chunks of
/// kChunkRows rows numbered from chunk_start[k]. Rows whose task id names no instance are in no group.
struct RowGroups
{
    const u32* order;
    const u32* starts;       // [instances + 1]
    const u32* chunk_start;  // [instances + 1]
};
/// An instance sampler on the device (rl/sampling.hpp): instances 0 is off; m 0 draws uniformly.
struct SamplerDev
{
    u32 instances;
    u32 m;
    const u32* thresholds;  // [m - 1]
    const i32* indices;     // [m]
};

constexpr u32 kChunkRows = 4;  // rows of a chunk: one block's share (one per wave of a block of 4 waves)
constexpr u32 kMaxInstances = 65536;

struct EnvArgs
{
    TaskDev T;             // the instance of a one-instance batch
    const TaskDev* tasks;  // [instances] (device): every instance's tables, for a grouped launch
    const InstDev* inst;   // [instances] (device)
    u32 instances;
    u32 wave_words;        // LDS words per wave of a grouped launch (the largest of its instances)
    RowGroups groups;      // rows grouped by instance (order null: batch order, one instance)
    u32 instance;          // with groups, a one-instance launch's instance (T's): it steps that group's rows
    EnvCfg cfg;
    u64* states;
    u64 rows;
    u32 words;  // row words of the batch (>= every instance's W)
    i32* task_ids;             // [rows]: each row's instance (null: instance 0); an autoreset writes the new one
    const i32* next_task_ids;  // [rows]: the instance an autoresetting row restarts in (null: its own)
    const u64* seed;           // device word: the env's RNG key (set_seed writes it in stream order)
    const u64* seeds;          // [rows]: per-row keys of the random policy (null: *seed)
    const u32* env_ids;        // [rows]: per-row env ids (null: first_env + row)
    u32* reset_counts;         // [rows]: per-row reset counters (null: none), advanced by every autoreset

    i32* steps;
    u64* draws;
    u8* at_goal;
    u64 first_env;
    const i64* actions;  // null: the random policy
    // label mode (DeviceEnv::step with rl::Labels): row i's action is the label (label_schema[i], label_binding[i *
    // label_stride + k] for k below the schema's arity), applied where it is applicable (else the row is invalid)
    const i32* label_schema;
    const i32* label_binding;
    u32 label_stride;
    float* reward;
    u8* terminated;
    u8* truncated;
    i32* count;
    u64* final_states;
    u32 final_words;
    i32* schema;
    i32* binding;
    u32 label_width;
    u8* invalid;
    u8* goal;
    i32* atoms;       // [rows, max_atoms]: ascending true-atom slots of the observed state, -1 padded (optional)
    u32 max_atoms;
    u8* masks;        // [rows, num_schemas]: schemas with an applicable binding in the observed state (optional)
    u32* counts;      // [rows, cache_width]: the count cache (per-schema counts, then the state's fingerprint), optional
    u32 cache_width;  // the most schemas of any instance + 2
    u32 mask_width;   // the most schemas of any instance (columns of masks)
    u64* goal_pos;    // [rows, words]: per-env goal masks (optional, with goal_neg)
    u64* goal_neg;
    VisitedDev visited;
    u8* revisited;    // [rows]: the reached state's key was in the row's table before the step (optional)
    u32* status;
};

void launch_env_step(const EnvArgs& a, hipStream_t stream);

/// The masked rows' visited tables restarted with one key each (visited_clear + visited_insert): the initial state's
/// of the row's instance (a reset; run after launch_env_reset), or with `current` the hash of the row's state.
void launch_visited_restart(const VisitedDev& v, const InstDev* inst, u32 instances, const u64* states, u64 rows, u32 words,
                            const u8* mask, const i32* task_ids, bool current, hipStream_t stream);

/// Membership of successor hashes in visited tables (rl::visited_mask): out[j] = succ_hash[j] is in table row
/// parent[j] (or rows[parent[j]], rows having `parents` entries; without rows parents = table_rows); -1 and
/// out-of-range parents or rows read as not visited.
void launch_visited_mask(const u64* table, const i32* count, u64 table_rows, u32 capacity, const u64* succ_hash, const i32* parent,
                         const i32* rows, u64 parents, u64 size, u8* out, hipStream_t stream);

/// The arguments of a count over rows (refresh, the initial states, schema masks): count[i] (successors), goal[i],
/// masks [rows, num_schemas] and the count cache [rows, num_schemas + 2] of the rows (each may be null); goal_pos /
/// goal_neg [rows, words]: per-env goal masks (null: the instances' goal tests).
struct CountArgs
{
    TaskDev T;
    const TaskDev* tasks;
    const InstDev* inst;
    u32 instances;
    u32 wave_words;
    RowGroups groups;
    const u64* states;
    u64 rows;
    u32 words;
    const i32* task_ids;
    i32* count;
    u8* goal;
    u8* masks;        // [rows, mask_width]
    u32* cache;       // [rows, cache_width]
    u32 cache_width;  // the most schemas of any instance + 2
    u32 mask_width;   // the most schemas of any instance
    const u64* goal_pos;
    const u64* goal_neg;
    u32* status;
    u32 instance;  // the instance of a one-instance count (its fingerprint salt; with groups, the group it counts)
};

void launch_env_count(const CountArgs& a, hipStream_t stream);
/// A one-instance count of rows of instance `instance` (the common case of launch_env_count); masks and cache rows are
/// laid out for `schemas` schemas (0: the task's).
void launch_env_count(const TaskDev& T, const u64* states, u64 rows, u32 words, i32* count, u8* goal, u8* masks, u32* cache,
                      hipStream_t stream, const u64* goal_pos = nullptr, const u64* goal_neg = nullptr, u32* status = nullptr,
                      u32 instance = 0, u32 schemas = 0);

/// Groups the rows by task id (RowGroups): hist [instances + 1] and the three group arrays are device scratch; rows
/// with a task id outside [0, instances) set kStatusTaskId.
void launch_group_rows(const i32* task_ids, u64 rows, u32 instances, u32* hist, u32* order, u32* starts, u32* chunk_start,
                       u32* status, hipStream_t stream);

/// Tables of at most this many instances step with one launch per instance (the instance's tables as kernel arguments,
/// its group's rows from the row groups); larger tables with one launch per kernel variant (each block reads its
/// chunk's instance's tables from device memory).
constexpr u32 kPerInstanceLaunches = 16;

/// The kernel variant of an instance (InstDev::variant) and the block shape of a grouped launch over the instances of
/// one variant: waves per block and dynamic LDS bytes, from the largest hot tables and per-wave region among them.
u32 env_variant(const TaskDev& T);
unsigned grouped_shape(const TaskDev* const* tasks, u32 n, size_t* lds_bytes, u32* wave_words);
/// Raises the dynamic LDS limits of the step and count kernels an instance (or a variant's grouped launch) uses, so
/// that later launches make no runtime call besides the launch (HIP graph capture).
void prepare_env_launches(const TaskDev& T);
void prepare_grouped_launches(u32 v, size_t lds);
/// The grouped step / count of the rows of the instances of variant v (grid: enough blocks for every chunk).
void launch_env_step_grouped(const EnvArgs& a, u32 v, unsigned nw, size_t lds, hipStream_t stream);
void launch_env_count_grouped(const CountArgs& a, u32 v, unsigned nw, size_t lds, hipStream_t stream);

/// Ascending true-atom slots of each row, -1 padded to max_atoms (State::slots, include/mymyr/state/state.hpp:96-101).
void launch_encode_atoms(const u64* states, u64 rows, u32 words, u32 W, i32* out, u32 max_atoms, u32* status, hipStream_t stream);

/// Resets the rows with mask[i] != 0 (all if mask is null) to the initial state of their instance task_ids[i] (null:
/// instance 0; an id outside [0, instances) resets the row into instance 0, writes 0 there and sets kStatusTaskId):
/// the instance's initial state in its words and zeros up to the batch's, steps 0, at_goal, count and the count cache
/// row of the initial state; draws are kept (HostEnv::reset, src/mymyr/rl/env.cpp:179-205, 223-255).
void launch_env_reset(const InstDev* inst, u32 instances, u64* states, u64 rows, u32 words, const u8* mask, i32* task_ids, i32* steps,
                      u8* at_goal, i32* count, u32* cache, u32 cache_width, u32* status, hipStream_t stream);

/// Before a reset of the rows with mask[i] != 0: with `sample` their task ids drawn from the sampler (with the rows'
/// reset counters), then the counters advanced (HostEnv::reset, src/mymyr/rl/env.cpp:223-255).
void launch_env_reset_draw(const SamplerDev& sampler, const u64* seed, u64 first_env, u64 rows, const u8* mask, bool sample, i32* task_ids,
                           u32* reset_counts, const u64* sampling_seeds, const u32* env_ids, hipStream_t stream);

/// next[i] = the instance row i's next autoreset draws from the sampler (its current reset counter, its sampling key or
/// *seed, its env id or first_env + i): the next_task_ids of a step that restarts rows in sampled instances.
void launch_env_sample_next(const SamplerDev& sampler, const u64* seed, u64 first_env, u64 rows, const u32* reset_counts,
                            const u64* sampling_seeds, const u32* env_ids, i32* next, hipStream_t stream);

/// The random policy's next choices without a step: out[i] = the successor index a step would draw now for row i,
/// limited to max_actions, 0 where count[i] is 0 (DeviceEnv::random_actions, include/mymyr/cuda/env.hpp:189-192).
void launch_env_random_actions(const u64* seed, const u64* seeds, const u32* env_ids, u64 first_env, const u64* draws, const i32* count,
                               u64 rows, u32 max_actions, i64* out, hipStream_t stream);
/// kStatusTaskId if some ids[i] (device, [rows]; null: none) is outside [0, instances).
void launch_check_ids(const i32* ids, u64 rows, u32 instances, u32* status, hipStream_t stream);
/// *p = v in stream order (one thread).
void launch_set_word(u64* p, u64 v, hipStream_t stream);

/// Per-env goal masks at a reset of the rows with mask[i] != 0: the instance's goal written into them, or with
/// keep_goals the given masks kept, checked against the instance's fluent slots (kStatusGoalMask) and at_goal tested
/// on the initial state with them. Runs after launch_env_reset (it reads the rows' instances from task_ids).
void launch_env_reset_goals(const InstDev* inst, u32 instances, u64 rows, u32 words, const u8* mask, const i32* task_ids, u64* goal_pos,
                            u64* goal_neg, bool keep_goals, u8* at_goal, u32* status, hipStream_t stream);

/// The count cache's fingerprint salt of an instance: 0 for instance 0, so a row's cache entry stands for its state
/// and its instance.
__host__ __device__ inline u64 instance_salt(u32 k) { return static_cast<u64>(k) * 0xD6E8FEB86659FD93ull; }

/// Words of a count-cache row: the per-schema counts, then the 64-bit state fingerprint.
__host__ __device__ inline u32 cache_width(const TaskDev& T) { return T.num_schemas + 2; }

/// The flat expansion of rows (rl::expand, include/mymyr/rl/expand.hpp:1-130). Pass 0 counts each row's successors
/// (and, with drop_noops, its no-op successors) and checks that rows have no atoms past their instance's slots; pass 1
/// writes the successors of row i from offsets[i] on (kept rows only with drop_noops), up to capacity. Over a table,
/// one launch per instance expands that instance's group of rows.
struct ExpandArgs
{
    TaskDev T;
    RowGroups groups;  // rows grouped by instance (order null: batch order, one instance)
    u32 instance;      // with groups, the instance (T's) whose group this launch expands
    const u64* states;
    u64 rows;
    u32 words;
    u32 pass;
    u32 drop_noops;
    u32 out_words;    // words of the succ rows
    u32 label_width;  // columns of binding
    u32* counts;      // [rows]
    u32* noops;       // [rows]
    const u64* offsets;  // [rows]
    u64 offset_base;     // subtracted from offsets (a chunk of a longer expansion writes from its own position 0)
    u64 capacity;
    u64* succ;
    i32* parent;
    i32* schema;
    i32* binding;
    u8* goal;
    u64* succ_hash;
    u8* noop;
    i32* index;
    u32* words_needed;  // device word: the widest trimmed successor that did not fit out_words
    u32* status;
    u32 witness;        // witness pruning (one-instance launches): one successor per effect-relevant binding
    AnyOfDev any_goal;  // the goal flags' goal when any_goal.any is set (a search's GoalSpec::AnyOf), else the task's
};

void launch_expand(const ExpandArgs& a, hipStream_t stream);
/// kept[i] = counts[i] - noops[i], or counts[i] when every successor of row i is a no-op.
void launch_kept_counts(const u32* counts, const u32* noops, u64 rows, u32* kept, hipStream_t stream);

/// A flat expansion (device arrays; offsets [rows + 1]) and its padded [rows, k] view (rl::pad,
/// src/mymyr/rl/expand.cpp:799-873). Null destinations are not written; a null flat source pads its destination.
struct PadArgs
{
    u64 rows;
    u64 capacity;          // rows the flat arrays hold: successor j of a row is valid only below it
    const i32* offsets;    // [rows + 1]
    const u64* succ;       // [capacity, flat_words]
    u32 flat_words;
    u32 flat_label_width;
    const i32* schema;
    const i32* binding;    // [capacity, flat_label_width]
    const u8* goal;
    const u64* succ_hash;
    const u8* noop;
    const i32* index;      // positions in the parents' full successor order
    u32 k;
    u32 words;             // words of the padded succ rows (>= flat_words)
    u32 label_width;       // columns of the padded binding (>= flat_label_width)
    i32* out_index;        // [rows, k]: flat row, -1 padding
    u8* mask;
    i32* count;            // [rows]
    u64* out_succ;         // [rows, k, words], zero padding
    i32* out_schema;       // -1 padding
    i32* out_binding;      // [rows, k, label_width], -1 padding
    u8* out_goal;
    u64* out_succ_hash;
    u8* out_noop;
    i32* canonical;        // flat index, -1 padding
    u32* overflow;         // device word: set when a count exceeds k or a successor lies past capacity
};
void launch_pad(const PadArgs& a, hipStream_t stream);
/// actions[i] = the position of row i's label (label_schema[i], label_binding [rows, stride]) among its successors of a
/// flat expansion (offsets [rows + 1], schema, binding [., L]), or -1 when no successor carries it.
void launch_label_actions(const i32* offsets, const i32* schema, const i32* binding, u32 L, u64 rows, const i32* label_schema,
                          const i32* label_binding, u32 stride, i64* actions, hipStream_t stream);
/// dst[i] = src[i] for i < n (offsets fit int32 after the caller's checks).
void launch_offsets_i32(const u64* src, u64 n, i32* dst, hipStream_t stream);

/// Per-row successor listing in canonical order (schema [rows, cap], binding [rows, cap, L], successor rows
/// [rows, cap, words]) and counts [rows]; entries past cap are counted but not written.
void launch_successors(const TaskDev& T, const u64* states, u64 rows, u32 words, u32 cap, i32* count, i32* schema, i32* binding,
                       u64* succ, u32* status, hipStream_t stream);
}  // namespace mya
