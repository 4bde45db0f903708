#pragma once
// Device-side lifted matching over one state, executed by one wavefront (64 lanes) per state:
//   - the view: per fluent predicate of arity 1 one row, of arity 2 forward / backward rows, each row an object bitset
//     over the window of the other position's domain; built in LDS from the state's set bits (AtomIndex records);
//   - count(schema, plan j): the number of applicable full bindings extending a bound prefix, a nested loop over the
//     plan's parameters whose candidates are ANDs of 64-bit words (dom0, view rows, static rows), with k-ary literals
//     checked at the level that binds their last parameter;
//   - pick(schema, rank): the rank-th applicable binding in lexicographic parameter order, by prefix counting.
// The set of bindings is the reference's (all literals of the precondition hold; witness pruning off), and the
// lexicographic order is its canonical order (include/mymyr/successor/successors.hpp:8-10, 154-248).

#include "device_common.hpp"
#include "scan.hpp"
#include "task.hpp"

namespace mya
{
struct TaskDev
{
    const DevSchema* schemas;
    const DevStep* steps;
    const DevCons* cons;
    const DevCheck* checks;
    const DevEffect* effects;
    const DevPair* pairs;
    const u64* rs;
    const u32* slot_of;
    const u64* records;
    const u64* dom0;
    const u64* static_rows;
    const DevStaticMeta* static_meta;
    const u64* static_words;  // image base (static keys are image offsets)
    const u32* goal_pos;
    const u32* goal_neg;
    const u64* initial;
    const u32* pred_arity;
    const u32* pos_begin;
    const u64* pred_pairs;
    const u64* pred_offset;
    u64 fluent_count;
    u32 n, ow, W, num_schemas, num_pairs, view_words, ngp, ngn, goal_unsat, dense, label_width, fluent_slots;
};

/// Pointers into an uploaded image (host helper).
TaskDev task_dev(const u64* image_dev, const DevTaskHeader& h);

constexpr u32 kCountCache = 1024;  // per-schema counts kept in LDS for schemas below this count

/// LDS words (u64) a wave needs beyond the view: the bindings of 64 lanes, the per-schema counts, the enumeration
/// cursors of 64 lanes (bits and word index per level) and the effect scratch.
constexpr u32 kLdsExtraWords = (kMaxParams * 64) / 2 + kCountCache / 2 + kMaxParams * 64 + (kMaxParams * 64) / 2 + 32 + 32;

inline u32 lds_words(const DevTaskHeader& h) { return h.view_words + kLdsExtraWords; }
}  // namespace mya
