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
    u64 seed;
    u32 max_steps;
    float step_reward, goal_reward, dead_end_reward;
    i32 dead_end_none;      // DeadEnd::None
    i32 dead_end_terminal;
    i32 autoreset;
};

struct EnvArgs
{
    TaskDev T;
    EnvCfg cfg;
    u64* states;
    u64 rows;
    u32 words;  // row words of the batch (>= T.W)
    i32* steps;
    u64* draws;
    u8* at_goal;
    u64 first_env;
    const i64* actions;  // null: the random policy
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
    u32* counts;      // [rows, num_schemas + 2]: the count cache (per-schema counts, then the state's fingerprint), optional
    u64* goal_pos;    // [rows, words]: per-env goal masks (optional, with goal_neg)
    u64* goal_neg;
    const u64* task_goal_pos;  // [W]: the task's goal as masks (device), written by an autoreset
    const u64* task_goal_neg;
    const u32* init_counts;  // [num_schemas + 2]: the initial state's cache row (device)
    const u8* init_masks;  // [num_schemas]: the initial state's masks (device)
    u32 init_count;
    u32 init_goal;
    u32* status;
};

void launch_env_step(const EnvArgs& a, hipStream_t stream);

/// count[i] (successors), goal[i], masks [rows, num_schemas] and the count cache [rows, num_schemas + 2] of rows (each
/// may be null).
void launch_env_count(const TaskDev& T, const u64* states, u64 rows, u32 words, i32* count, u8* goal, u8* masks, u32* cache,
                      hipStream_t stream, const u64* goal_pos = nullptr, const u64* goal_neg = nullptr, u32* status = nullptr);

/// Ascending true-atom slots of each row, -1 padded to max_atoms (State::slots, include/mymyr/state/state.hpp:96-101).
void launch_encode_atoms(const u64* states, u64 rows, u32 words, u32 W, i32* out, u32 max_atoms, u32* status, hipStream_t stream);

/// Resets the rows with mask[i] != 0 (all if mask is null) to the initial state: steps 0, at_goal = init_goal,
/// count = init_count, the count cache row = init_cache; draws are kept (HostEnv::reset, src/mymyr/rl/env.cpp:207-240).
void launch_env_reset(const TaskDev& T, u64* states, u64 rows, u32 words, const u8* mask, i32* steps, u8* at_goal, i32* count,
                      u32* cache, const u32* init_cache, u32 init_count, u32 init_goal, hipStream_t stream);

/// Per-env goal masks at a reset of the rows with mask[i] != 0: the task's goal (task_pos / task_neg [W]) written into
/// them, or with keep_goals the given masks kept, checked against the task's fluent slots (kStatusGoalMask) and
/// at_goal tested on the initial state with them.
void launch_env_reset_goals(const TaskDev& T, u64 rows, u32 words, const u8* mask, u64* goal_pos, u64* goal_neg, const u64* task_pos,
                            const u64* task_neg, bool keep_goals, u8* at_goal, u32* status, hipStream_t stream);

/// Words of a count-cache row: the per-schema counts, then the 64-bit state fingerprint.
__host__ __device__ inline u32 cache_width(const TaskDev& T) { return T.num_schemas + 2; }

/// The flat expansion of rows (rl::expand, include/mymyr/rl/expand.hpp:1-130). Pass 0 counts each row's successors
/// (and, with drop_noops, its no-op successors) and checks that rows have no atoms past the task's slots; pass 1 writes
/// the successors of row i from offsets[i] on (kept rows only with drop_noops), up to capacity.
struct ExpandArgs
{
    TaskDev T;
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
};

void launch_expand(const ExpandArgs& a, hipStream_t stream);
/// kept[i] = counts[i] - noops[i], or counts[i] when every successor of row i is a no-op.
void launch_kept_counts(const u32* counts, const u32* noops, u64 rows, u32* kept, hipStream_t stream);
/// dst[i] = src[i] for i < n (offsets fit int32 after the caller's checks).
void launch_offsets_i32(const u64* src, u64 n, i32* dst, hipStream_t stream);

/// Per-row successor listing in canonical order (schema [rows, cap], binding [rows, cap, L], successor rows
/// [rows, cap, words]) and counts [rows]; entries past cap are counted but not written.
void launch_successors(const TaskDev& T, const u64* states, u64 rows, u32 words, u32 cap, i32* count, i32* schema, i32* binding,
                       u64* succ, u32* status, hipStream_t stream);
}  // namespace mya
