#pragma once
// Device-side lifted matching over one state, executed by one wavefront (64 lanes) per state:
//   - the view: per fluent predicate of arity 1 one row, of arity 2 forward / backward rows, each row an object bitset
//     over the window of the other position's domain. Rows that are contiguous slices of the state (dense slots over
//     contiguous domains, forward direction) are read from the state row itself; the others are built in LDS from
//     the state's set bits;
//   - count(schema, plan j): the number of applicable full bindings extending a bound prefix, a nested loop over the
//     plan's parameters whose candidates are ANDs of 64-bit words (dom0, view rows, static rows), with k-ary literals
//     checked at the level that binds their last parameter;
//   - pick(schema, rank): the rank-th applicable binding in lexicographic parameter order, by prefix counting.
// The set of bindings is the reference's (all literals of the precondition hold; witness pruning off), and the
// lexicographic order is its canonical order (include/mymyr/successor/successors.hpp:8-10, 154-248).
//
// A block stages the task's hot tables (schemas, plans, constraints, checks, effects, view pairs, slot decoding,
// dom0, goal, per-predicate tables: the image's first hot_words words) in LDS once; each wave of the block then
// steps its environments with its own LDS region (state row, view, bindings, enumeration cursors).

#include "device_common.hpp"
#include "scan.hpp"
#include "task.hpp"

namespace mya
{
/// The task as the kernels see it: hot sections by word offset (in the image and, once staged, in LDS), cold tables
/// by global pointer.
struct TaskDev
{
    u64 off_schemas, off_steps, off_cons, off_checks, off_effects, off_pairs, off_decode, off_dom0;
    u64 off_goal_pos, off_goal_neg, off_pred_arity, off_pos_begin, off_pred_pairs, off_pred_offset;
    const u64* image;
    const u64* rs;
    const u32* slot_of;
    const u64* records;
    const u64* static_rows;
    const DevStaticMeta* static_meta;
    const u64* static_words;  // image base (static keys are image offsets)
    const u64* initial;
    u64 fluent_count;
    u32 hot_words;
    u32 n, ow, W, num_schemas, num_pairs, view_words, ngp, ngn, goal_unsat, dense, label_width, fluent_slots;
    u32 num_decode, decode_arith;
    u32 max_step_words;
    u32 lazy;      // lazy slots: an added atom without a slot is recorded in `missing`
    u64* missing;  // lazy slots: bit per canonical fluent atom (device; set by the successor kernels), else null
    const DevWitness* witness;  // per schema its witness parameters and plans (null: no schema has a witness)
};

/// Pointers into an uploaded image (host helper).
TaskDev task_dev(const u64* image_dev, const DevTaskHeader& h);

constexpr u32 kMaxEnvSchemas = 8192;  // schemas whose per-state counts a wave keeps in LDS
constexpr u32 kCap = 64;           // items per level of the level-synchronous count (one per lane)

/// Per-wave LDS words: the state row, the view, the uniform binding, the bindings and per-level enumeration cursors of
/// the 64 lanes' nested loops (A = the largest schema arity, at least 1), the effect scratch, the per-schema counts and
/// the successor enumeration's level cursors (A masks, A words);
/// with `levels`, also the two item levels of the level-synchronous count with their roots, root counts, root objects
/// and item makers.
__host__ __device__ inline u32 wave_lds_words(const TaskDev& t, bool levels)
{
    const u32 A = t.label_width ? t.label_width : 1;
    const u32 S = t.num_schemas;
    u32 w = t.W + t.view_words + (A + 1) / 2 + 32 * A + 64 * A + 32 * A + 32 + (S + 1) / 2 + A + (A + 1) / 2;
    if (levels)
        w += kCap * A + 5 * kCap / 2;
    return (w + 1) & ~1u;
}
}  // namespace mya
