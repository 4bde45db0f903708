#pragma once
// Host side of a planning task: the text reader, the task compiler (typed-dense canonical atom layout, relaxed
// reachability, atom slots, initial state, goal) and the device image the HIP kernels read.
//
// Semantics follow the reference task build (maichmueller/mymyr):
//   text format                 src/mymyr/formalism/text_format.cpp:22-197
//   dom0 of a parameter         src/mymyr/task/compile.cpp:803-915 (the matcher's static domain)
//   canonical layout            src/mymyr/task/compile.cpp:1363-1455 (build_layout)
//   atom mode (dense/reachable) src/mymyr/task/task.cpp:106-143 (choose_atom_mode)
//   relaxed reachability        include/mymyr/reachability/relaxed_reachability.hpp:3-12 (rule semantics)
//   initial state               src/mymyr/task/task.cpp:216-232
// The code is this project's own: a single-threaded host compiler producing flat tables for the device.

#include <array>
#include <cstdint>
#include <map>
#include <memory>
#include <stdexcept>
#include <string>
#include <string_view>
#include <vector>

namespace mya
{
using u8 = std::uint8_t;
using u16 = std::uint16_t;
using u32 = std::uint32_t;
using u64 = std::uint64_t;
using i32 = std::int32_t;
using i64 = std::int64_t;

struct Error : std::runtime_error
{
    using std::runtime_error::runtime_error;
};

constexpr u32 kNone = ~u32{0};
constexpr u64 kNone64 = ~u64{0};

/// A literal: terms >= 0 are parameter indices, < 0 encode object o as -(o + 1).
struct Literal
{
    u32 pred = 0;
    bool positive = true;
    std::vector<i32> terms;
};

/// A conditional effect (the reference's ConditionalEffect, include/mymyr/formalism/task_data.hpp): for every binding of
/// its `extra` forall parameters (terms arity .. arity + extra - 1) under which `cond` holds in the state, the
/// literals `eff` apply (deletes, then adds, with the schema's own effects).
struct CondEffectText
{
    u32 extra = 0;
    std::vector<Literal> cond;
    std::vector<Literal> eff;
};

struct SchemaText
{
    std::string name;
    u32 arity = 0;
    std::vector<Literal> pre;
    std::vector<Literal> eff;           // the unconditional effects: positive = add, negative = delete
    std::vector<CondEffectText> ces;    // effects with a condition or forall parameters
};

struct PredicateText
{
    char kind = 'S';  // S static, F fluent, D derived
    u32 arity = 0;
    std::string name;
};

/// A parameter that normalization removed from its schema because nothing but its type mentions it (the reference's
/// CollapsedParameter, include/mymyr/formalism/task_data.hpp:194-206): the schema's actions bind the other parameters,
/// and the action as written names the representative at `position` of the parameter list before collapsing.
struct CollapsedText
{
    u32 schema = 0;
    u32 position = 0;
    bool written = false;
    i32 representative = -1;  // -1: none
};

/// A ground literal of the encoding goal (the goal that observation encodings show; the search goal is `goal`).
struct GroundLiteralText
{
    u32 pred = 0;
    bool positive = true;
    std::vector<u32> objects;
    bool operator<(const GroundLiteralText& o) const
    {
        if (positive != o.positive)
            return positive;  // positive literals first
        if (pred != o.pred)
            return pred < o.pred;
        return objects < o.objects;
    }
    bool operator==(const GroundLiteralText& o) const { return positive == o.positive && pred == o.pred && objects == o.objects; }
};

struct TaskText
{
    u32 objects = 0;
    std::vector<PredicateText> preds;
    std::vector<std::vector<u32>> static_init, fluent_init;  // [pred, args...]
    std::vector<Literal> goal;                                // ground
    std::vector<SchemaText> schemas;
    // the C section: collapsed parameters ascending in (schema, position); labels bind the schemas' own parameters
    bool unused_parameters_collapsed = false;
    std::vector<CollapsedText> collapsed;
    // the EG section: sorted and unique (positive first, predicate, objects)
    bool encoding_goal_recorded = false, encoding_goal_complete = false;
    std::vector<GroundLiteralText> encoding_goal;
};

/// Parses the reference's task text format (classical subset: no numeric sections, no axioms). Throws mya::Error naming
/// what is unsupported or malformed.
TaskText parse_task_text(std::string_view text);

/// Atom slots (include/mymyr/task/atom_index.hpp:12-22): Reachable and Dense are frozen (the slot table is a function of
/// the task); Lazy slots are assigned as atoms are met: the initial state's atoms at load, in the order of its atom
/// list (task.cpp:214-224), then the atoms that successors add without a slot, interned between device launches in
/// ascending canonical id (include/mymyr/cuda/generator.hpp:20-24).
enum class AtomMode : u32
{
    Reachable = 0,
    Dense = 1,
    Lazy = 2,
};
enum class AtomsOption : u32
{
    Auto = 0,
    Reachable = 1,
    Dense = 2,
    Lazy = 3,
};

/// Typed-dense canonical ids: cid(p, a) = offset[p] + sum_i rs[pos_begin[p] + i][a_i].
struct Layout
{
    static constexpr u64 kOutside = u64{1} << 40;
    std::vector<u64> offset;     // per predicate (kNone64 for static predicates)
    std::vector<u64> size;       // per predicate
    std::vector<u32> pos_begin;  // per predicate
    std::vector<std::vector<u64>> rs;      // per position: rank * stride or kOutside, per object
    std::vector<std::vector<u32>> domain;  // per position: objects in rank order
    u64 fluent_count = 0;
    [[nodiscard]] u64 encode(u32 p, const u32* args, u32 arity) const
    {
        u64 c = offset[p];
        for (u32 i = 0; i < arity; ++i)
            c += rs[pos_begin[p] + i][args[i]];
        return c;
    }
};

/// One constraint on the candidate objects of a parameter (an AND term of its candidate bitset).
enum class ConsKind : u32
{
    Dom0 = 0,        // the static domain (dom0) of the parameter
    ViewUnary = 1,   // the view row of a unary fluent predicate
    ViewRow = 2,     // a row of a binary fluent predicate, indexed by a bound parameter or a constant
    StaticRow = 3,   // a row of a binary static predicate, indexed by a bound parameter
};

/// A literal checked once all its parameters are bound (k-ary literals, repeated variables, ground fluents).
enum class CheckKind : u32
{
    Fluent = 0,  // canonical key -> slot -> state bit
    Static = 1,  // static relation membership (sorted keys)
};

// ---------------------------------------------------------------------------------------------------------------
// Device image. Everything below is POD and copied verbatim into one device buffer; offsets are in u64 words from
// the image start. The kernels index it directly.

struct DevCons
{
    u32 kind;   // ConsKind
    u32 neg;    // 1: AND with the complement (negative literal)
    u32 src;    // ViewRow / StaticRow: the source parameter, or kNone when `obj` is a constant
    u32 obj;    // constant source object (ViewRow with src == kNone)
    u32 table;  // Dom0: word offset of the dom0 bits; ViewUnary / ViewRow: view pair index; StaticRow: static row table
    u32 pad;
};

struct DevCheck
{
    u32 kind;  // CheckKind
    u32 pos;   // literal polarity
    u32 pred;  // predicate (Static: its relation index)
    u32 nterms;
    i32 terms[6];
};

/// One parameter to bind: its object window and the AND terms of its candidate set.
struct DevStep
{
    u32 param;
    u32 lo;      // first object of the window
    u32 words;   // window words
    u32 cons_begin, cons_end;    // into the schema's DevCons
    u32 check_begin, check_end;  // into the schema's DevCheck
    u32 pad;
};

constexpr u32 kMaxParams = 32;

/// Per schema: plans P_j (j = 0..arity) count the bindings with parameters [0, j) bound; filters F_i (i < arity) give
/// the candidates of parameter i with [0, i) bound (the lexicographic pick).
struct DevSchema
{
    u32 arity;
    u32 never;       // a static precondition fails, or a dom0 is empty
    u32 ground_begin, ground_end;  // ground fluent checks (DevCheck) of the precondition
    u32 plan_begin[kMaxParams + 2];  // into steps: plan j occupies [plan_begin[j], plan_begin[j + 1])
    u32 filter_step[kMaxParams];     // the DevStep of filter i
    u32 eff_begin, eff_end;          // into effects
    u32 nadd;                        // effects [eff_begin, eff_begin + nadd) add, the rest delete
    u32 affects;  // bit s: an action of this schema can change schema s's successor count (every bit past 32 schemas)
};

/// Witness pruning of a schema (the parameters no effect mentions, witnesses, bound last and only once per binding of
/// the others), in the order the reference's matcher binds the witnesses: filter[t] gives the candidates of param[t]
/// with the effect-relevant parameters and witnesses [0, t) bound; steps [plan_lo[t], plan_hi[t]) count the completions
/// of witnesses (t, n) once witnesses [0, t] are bound (empty for the last).
struct DevWitness
{
    u32 n;  // witness parameters (0: none)
    u32 param[kMaxParams];
    u32 filter[kMaxParams];
    u32 plan_lo[kMaxParams];
    u32 plan_hi[kMaxParams];
    u32 pad;
};

/// An effect pattern: cid = base + sum over parameter terms of rs[pos][object].
struct DevEffect
{
    u32 pred;
    u32 nvar;
    u64 base;
    u32 var_param[4];
    u32 var_pos[4];  // global position index into the rs tables
};

/// A view pair: the rows of a fluent predicate of arity 1 (one row) or 2 (forward: source position 0, or backward).
struct DevPair
{
    u32 pred;
    u32 dir;      // 0 forward (rows by position 0's object, bits of position 1), 1 backward; unary: 0
    u32 src_lo, src_n;   // source object window (rows)
    u32 dst_lo, dst_words;  // destination object window
    u32 offset;   // word offset of the pair's rows in the per-state view (not bulk)
    u32 bulk;     // 1: row r is the state's bits [bit0 + r * row_bits, + row_bits) (dense slots, contiguous domains)
    u64 bit0;     // bulk: first state bit of row 0
    u32 row_bits; // bulk: bits per row (the destination domain's size)
    u32 pad;
};

/// Slot decoding of a fluent predicate for the view build: a slot s in [offset, offset + size) is the atom with
/// position ranks (s - offset) / d1 and (s - offset) % d1; with contiguous domains the objects are lo0 + r0, lo1 + r1.
struct DevPredDecode
{
    u64 offset;
    u64 size;
    u32 pred;
    u32 arity;
    u32 d1;        // size of position 1's domain (1 for arity < 2)
    u32 lo0, lo1;
    u32 contiguous;  // every position's domain is a contiguous object range
    u32 has_scatter; // some view pair of the predicate is built by scattering set bits
    u32 pad;
};

struct DevTaskHeader
{
    u32 num_objects;
    u32 ow;             // words_for(num_objects)
    u32 words;          // state words W
    u32 fluent_slots;
    u32 dense;          // 1: slot = cid
    u32 num_schemas;
    u32 label_width;
    u32 num_pairs;
    u32 view_words;     // per-state view size (u64 words)
    u32 num_goal_pos, num_goal_neg;
    u32 goal_unsat;
    u64 fluent_count;
    // word offsets into the image
    u64 off_schemas, off_steps, off_cons, off_checks, off_effects, off_pairs;
    u64 off_rs, off_slot_of, off_records, off_dom0, off_static_rows, off_static_keys, off_static_meta;
    u64 off_goal_pos, off_goal_neg, off_initial;
    u64 off_pred_arity, off_pos_begin;
    u64 off_pred_pairs;   // per predicate: view pair of the unary / forward rows (low 32 bits), backward (high)
    u64 off_pred_offset;  // per predicate: first canonical id (u64)
    u64 off_decode;       // DevPredDecode per fluent predicate with atoms, ascending offset
    u64 hot_words;        // the image's first hot_words words hold everything the kernels read per state
                          // (staged in LDS); rs tables, slot tables, records, static rows and keys follow
    u32 num_positions;
    u32 num_decode;
    u32 decode_arith;     // 1: slots decode arithmetically (dense slots, contiguous domains)
    u32 init_count;     // successors of the initial state (filled once the device has counted them)
    u32 max_step_words; // the widest candidate window of any plan or filter step, in words
    u32 lazy;           // 1: lazy slots (slot_of, records, goal lists and initial row sized for every canonical atom)
    u32 pad;
    u64 off_witness;    // DevWitness per schema (0: no schema has a witness parameter)
};

/// Static k-ary relation: sorted keys sum(obj_i * n^(ar-1-i)) at [keys, keys + count).
struct DevStaticMeta
{
    u64 keys;
    u64 count;
    u32 arity;
    u32 pad;
};

struct CompiledTask
{
    TaskText text;
    u32 n = 0, ow = 1;
    Layout layout;
    AtomMode mode = AtomMode::Dense;
    u64 reachable_fluent = 0;
    u32 fluent_slots = 0, words = 1;
    std::vector<u32> slot_of;     // per cid (fluent_count entries): slot or kNone
    std::vector<u64> slot_cid;    // per slot
    std::vector<u64> initial;     // [words]
    std::vector<u32> goal_pos, goal_neg;  // goal slots
    bool goal_unsat = false;              // no state is a goal under the current slots
    // the goal's fluent literals in order (polarity, canonical id: at least fluent_count for an atom outside the
    // typed-dense domains), and whether the goal fails whatever the state (a static literal that fails, or one atom
    // wanted both true and false: the reference's compiled goal.unsatisfiable, compile.cpp:1322-1343)
    std::vector<std::pair<bool, u64>> goal_fluent;
    bool goal_fixed_unsat = false;
    // conditional effects: per schema, per conditional effect, the static domains of its forall parameters
    bool has_ce = false;
    std::vector<std::vector<std::vector<std::vector<u64>>>> ce_dom0;
    u32 label_width = 0;
    std::vector<std::vector<std::vector<u64>>> dom0;  // per schema, per parameter: object bits (ow words)
    std::vector<u8> never;                            // per schema
    std::vector<std::vector<u64>> static_keys;        // per static predicate: sorted packed keys of its atoms
    std::vector<u64> image;                           // the device image (DevTaskHeader first)
    [[nodiscard]] const DevTaskHeader& header() const { return *reinterpret_cast<const DevTaskHeader*>(image.data()); }
    [[nodiscard]] bool static_holds(u32 pred, const u32* objs) const;
    [[nodiscard]] u32 slot_of_atom(u32 pred, const u32* objs) const;  // kNone: no slot
};

std::unique_ptr<CompiledTask> compile_task(TaskText text, AtomsOption atoms);

/// The device record of canonical fluent atom `cid`: predicate | a0 << 16 | a1 << 32 | a2 << 48.
u64 atom_record(const CompiledTask& task, u64 cid);

/// Lazy slots: gives the next slots to the atoms `cids` (canonical fluent ids without a slot, ascending), in that order,
/// and brings the slot tables, the goal, the initial row's width and the device image up to date. Returns the image's
/// changed word ranges [first, end), for the device copy.
std::vector<std::pair<u64, u64>> intern_atoms(CompiledTask& task, const std::vector<u64>& cids);

/// Ground actions in canonical order (schema, then lexicographic binding), with their static preconditions evaluated
/// and fluent ones resolved to slots. An action whose positive fluent precondition has no slot is dropped (it never
/// applies); a negative one without a slot always holds.
struct GroundActions
{
    std::vector<u32> meta;   // npos | nneg << 8 | nadd << 16 | ndel << 24
    std::vector<u32> off;    // into slots
    std::vector<u32> slots;  // pos..., neg..., add..., del...
    std::vector<u32> schema;
    std::vector<u32> binding;  // [num, label_width]
    /// Witness pruning: action a is emitted only if none of dom[dom_off[a], dom_off[a + 1]) applies (the actions with
    /// its effect-relevant binding and a smaller witness object). Empty without witness pruning.
    std::vector<u32> dom_off;
    std::vector<u32> dom;
    /// Conditional effects: action a's ground instances are [ce_off[a], ce_off[a + 1]) (empty without conditional
    /// effects); instance k fires in a state where its condition slots ce_slots[ce_soff[k] ..] hold (npos positive, then
    /// nneg negative; ce_meta[k] = npos | nneg << 8 | nadd << 16 | ndel << 24), and then adds and deletes its slots.
    std::vector<u32> ce_off;
    std::vector<u32> ce_meta;
    std::vector<u32> ce_soff;
    std::vector<u32> ce_slots;
    u32 label_width = 0;
    [[nodiscard]] u32 size() const { return static_cast<u32>(meta.size()); }
};

/// Grounds every schema (static literals filter the bindings). Throws if more than `limit` actions result, or if an
/// action has more than 255 atoms in one list. With `witness_pruning`, the parameters no effect mentions (witnesses)
/// are pruned as the reference's matcher does: among the applicable actions with one effect-relevant binding the
/// successor is the one whose witness objects come first in the matcher's witness order, the binding it finds first
/// (include/mymyr/successor/detail/engine.hpp:345-356; the order: src/mymyr/task/compile.cpp:916-946).
GroundActions ground_actions(const CompiledTask& task, bool witness_pruning, u64 limit);

/// The effect-relevant parameters of a schema: those its effects or its conditional effects' conditions and effects
/// mention (src/mymyr/task/compile.cpp:1140-1162); the others are witnesses.
std::vector<u8> effect_relevant(const SchemaText& s);

/// The witness parameters of schema si (those `relevant` does not mark) in the order the reference's matcher binds them
/// (src/mymyr/task/compile.cpp:916-946).
std::vector<u32> witness_order(const CompiledTask& task, u32 si, const std::vector<u8>& relevant);

inline u32 words_for(u64 bits) { return static_cast<u32>((bits + 63) >> 6); }
}  // namespace mya
