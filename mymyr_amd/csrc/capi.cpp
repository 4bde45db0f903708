// The C ABI (include/mymyr_amd.h): argument checks, exception-to-status translation, and the calls into the task
// compiler, the state set and the drivers.

#include "../../include/mymyr_amd.h"

#include "brfs.hpp"
#include "capi_internal.hpp"
#include "device_common.hpp"
#include "runtime.hpp"
#include "state_set.hpp"
#include "lifted.hpp"
#include "task.hpp"

#include <cstdio>
#include <cstring>
#include <fstream>
#include <sstream>

namespace mya
{
thread_local std::string g_error;

void set_error(const std::string& m) { g_error = m; }

const DeviceTask& device_task(mya_task* t)
{
    // the lifted device tables (environment, successor listing, the wide and lazy searches) carry no conditional
    // effects: only the ground search (states of at most 16 words) evaluates them
    if (t->compiled->has_ce)
        throw std::invalid_argument("mymyr_amd: conditional effects are supported by the ground breadth-first search only (states of "
                                    "at most 16 words); the environment, the successor listing and the wide search refuse them");
    std::lock_guard lock(t->mutex);
    if (!t->dev.image)
    {
        int dev = 0;
        hip_check(hipGetDevice(&dev), "hipGetDevice");
        const auto& img = t->compiled->image;
        t->dev.image = dev_alloc<u64>(img.size(), "task image");
        hip_check(hipMemcpy(t->dev.image, img.data(), img.size() * sizeof(u64), hipMemcpyHostToDevice), "upload task image");
        t->dev.device = dev;
        t->dev.words = img.size();
        t->dev.thost = std::make_unique<TaskDev>(task_dev(t->dev.image, t->compiled->header()));
        if (t->compiled->mode == AtomMode::Lazy)
        {
            const u64 nw = std::max<u64>(1, words_for(t->compiled->layout.fluent_count));
            t->dev.missing = dev_alloc<u64>(nw, "lazy slot bitmap");
            hip_check(hipMemset(t->dev.missing, 0, nw * sizeof(u64)), "lazy slot bitmap");
            t->dev.thost->missing = t->dev.missing;
        }
    }
    return t->dev;
}

bool resolve_missing(mya_task* t, hipStream_t s)
{
    const DeviceTask& d = device_task(t);
    std::lock_guard lock(t->mutex);
    CompiledTask& C = *t->compiled;
    const u64 nw = std::max<u64>(1, words_for(C.layout.fluent_count));
    std::vector<u64> bits(nw);
    hip_check(hipMemcpyAsync(bits.data(), d.missing, nw * sizeof(u64), hipMemcpyDeviceToHost, s), "lazy slot bitmap");
    hip_check(hipStreamSynchronize(s), "lazy slot bitmap");
    std::vector<u64> cids;
    for (u64 w = 0; w < nw; ++w)
        for (u64 x = bits[w]; x; x &= x - 1)
            cids.push_back(w * 64 + static_cast<u64>(__builtin_ctzll(x)));
    if (cids.empty())
        return false;
    launch_fill_u32(reinterpret_cast<u32*>(d.missing), 2 * nw, 0, s);
    const auto ranges = intern_atoms(C, cids);
    for (const auto& [a, b] : ranges)
        if (b > a)
            hip_check(hipMemcpyAsync(d.image + a, C.image.data() + a, (b - a) * sizeof(u64), hipMemcpyHostToDevice, s), "task image");
    hip_check(hipStreamSynchronize(s), "task image");
    *t->dev.thost = task_dev(d.image, C.header());
    t->dev.thost->missing = d.missing;
    return true;
}
}  // namespace mya

using namespace mya;

extern "C" {

const char* mya_last_error(void) { return g_error.c_str(); }

int mya_abi_version(void) { return MYA_ABI_VERSION; }

int mya_memory_usage_get(mya_memory_usage* out)
{
    return guarded([&] {
        if (!out)
            throw std::invalid_argument("mymyr_amd: memory_usage_get: null argument");
        const MemoryUsage u = memory_usage();
        *out = mya_memory_usage{u.reserved, u.used, u.reserved_high, u.used_high, u.allocations, u.driver_allocations};
    });
}

int mya_task_load_text(const char* text, size_t len, int atoms, mya_task** out)
{
    return guarded([&] {
        if (!text || !out)
            throw std::invalid_argument("mymyr_amd: task_load_text: null argument");
        if (atoms < 0 || atoms > 3)
            throw std::invalid_argument("mymyr_amd: task_load_text: atoms must be 0 (auto), 1 (reachable), 2 (dense) or 3 (lazy)");
        auto t = std::make_unique<mya_task>();
        t->compiled = compile_task(parse_task_text(std::string_view(text, len)), static_cast<AtomsOption>(atoms));
        *out = t.release();
    });
}

int mya_task_load_file(const char* path, int atoms, mya_task** out)
{
    return guarded([&] {
        if (!path)
            throw std::invalid_argument("mymyr_amd: task_load_file: null path");
        std::ifstream in(path, std::ios::binary);
        if (!in)
            throw std::invalid_argument(std::string("mymyr_amd: cannot open ") + path);
        std::stringstream ss;
        ss << in.rdbuf();
        const std::string s = ss.str();
        if (mya_task_load_text(s.data(), s.size(), atoms, out) != 0)
            throw std::runtime_error(g_error);
    });
}

void mya_task_free(mya_task* task)
{
    if (!task)
        return;
    dev_free(task->dev.image);
    dev_free(task->dev.missing);
    delete task;
}

int mya_task_info_get(const mya_task* task, mya_task_info* out)
{
    return guarded([&] {
        if (!task || !out)
            throw std::invalid_argument("mymyr_amd: task_info: null argument");
        std::lock_guard lock(const_cast<mya_task*>(task)->mutex);  // lazy slots change words and fluent_slots
        const CompiledTask& c = *task->compiled;
        std::memset(out, 0, sizeof(*out));
        out->words = c.words;
        out->fluent_slots = c.fluent_slots;
        out->atom_mode = static_cast<uint32_t>(c.mode);
        out->num_schemas = static_cast<uint32_t>(c.text.schemas.size());
        out->label_width = c.label_width;
        out->num_objects = c.n;
        u32 ma = 0;
        for (const auto& p : c.text.preds)
            if (p.kind == 'F')
                ma = std::max(ma, p.arity);
        out->max_arity = ma;
        out->goal_unsat = c.goal_unsat ? 1 : 0;
        out->dense_fluent = c.layout.fluent_count;
        out->reachable_fluent = c.reachable_fluent;
        out->view_words = c.header().view_words;
    });
}

int mya_task_slots(const mya_task* task, uint32_t* rec, uint64_t* cid)
{
    return guarded([&] {
        if (!task)
            throw std::invalid_argument("mymyr_amd: task_slots: null task");
        std::lock_guard lock(const_cast<mya_task*>(task)->mutex);
        const CompiledTask& c = *task->compiled;
        u32 ma = 0;
        for (const auto& p : c.text.preds)
            if (p.kind == 'F')
                ma = std::max(ma, p.arity);
        const u32 stride = 1 + std::max<u32>(1, ma);
        for (u32 s = 0; s < c.fluent_slots; ++s)
        {
            const u64 id = c.slot_cid[s];
            if (cid)
                cid[s] = id;
            if (!rec)
                continue;
            // decode: the predicate whose block holds the id, then mixed-radix ranks (last position stride 1)
            u32 p = kNone;
            for (u32 q = 0; q < c.text.preds.size(); ++q)
                if (c.text.preds[q].kind == 'F' && c.layout.size[q] > 0 && c.layout.offset[q] <= id && id < c.layout.offset[q] + c.layout.size[q])
                    p = q;
            u32* r = rec + static_cast<size_t>(s) * stride;
            std::memset(r, 0, stride * sizeof(u32));
            r[0] = p;
            u64 rem = id - c.layout.offset[p];
            const u32 ar = c.text.preds[p].arity;
            for (u32 i = ar; i-- > 0;)
            {
                const auto& dom = c.layout.domain[c.layout.pos_begin[p] + i];
                r[1 + i] = dom[rem % dom.size()];
                rem /= dom.size();
            }
        }
    });
}

int mya_task_initial(const mya_task* task, uint64_t* row, uint32_t words)
{
    return guarded([&] {
        if (!task || !row)
            throw std::invalid_argument("mymyr_amd: task_initial: null argument");
        std::lock_guard lock(const_cast<mya_task*>(task)->mutex);
        const CompiledTask& c = *task->compiled;
        if (words < c.words)
            throw std::invalid_argument("mymyr_amd: task_initial: rows of " + std::to_string(words) + " words; the task needs " +
                                        std::to_string(c.words));
        std::memset(row, 0, words * sizeof(uint64_t));
        std::memcpy(row, c.initial.data(), c.words * sizeof(uint64_t));
    });
}

int mya_hash_rows(const uint64_t* rows, uint64_t n, uint32_t words, uint64_t* out, void* stream)
{
    return guarded([&] {
        if (n && (!rows || !out))
            throw std::invalid_argument("mymyr_amd: hash_rows: null array");
        launch_hash_rows(rows, n, words, out, static_cast<hipStream_t>(stream));
    });
}

uint64_t mya_hash_words(const uint64_t* w, uint32_t n, uint64_t seed) { return hash_words(w, n, seed); }
uint64_t mya_hash_state(const uint64_t* w, uint32_t n) { return hash_state(w, n); }

void mya_philox(uint64_t seed, uint64_t env, uint64_t draw, uint32_t purpose, uint32_t out[4])
{
    const Block4 b = philox4x32_10(Block4{{static_cast<u32>(draw), static_cast<u32>(draw >> 32), static_cast<u32>(env), purpose}},
                                   static_cast<u32>(seed), static_cast<u32>(seed >> 32));
    for (int i = 0; i < 4; ++i)
        out[i] = b.v[i];
}

uint32_t mya_successor_index(uint64_t seed, uint64_t env, uint64_t draw, uint32_t count)
{
    return successor_index(seed, env, draw, count);
}

int32_t mya_instance_draw(uint64_t seed, uint64_t env, uint32_t reset_count, uint32_t instances, const uint32_t* thresholds,
                          const int32_t* indices, uint32_t m)
{
    return instance_draw(seed, env, reset_count, instances, thresholds, indices, m);
}

int mya_hashset_create(uint64_t max_states, uint32_t words, double max_load, uint64_t batch, mya_hashset** out)
{
    return guarded([&] {
        if (!out)
            throw std::invalid_argument("mymyr_amd: hashset_create: null output");
        auto h = std::make_unique<mya_hashset>();
        state_set_create(h->set, max_states, words, max_load, batch ? batch : (u64{1} << 20), nullptr);
        hip_check(hipStreamSynchronize(nullptr), "hashset create");
        *out = h.release();
    });
}

void mya_hashset_free(mya_hashset* set)
{
    if (set)
        hashset_unref(set);
}

int mya_hashset_insert(mya_hashset* set, const uint64_t* rows, uint64_t n, int64_t* ids, uint8_t* is_new, uint64_t* new_count,
                       void* stream)
{
    return guarded([&] {
        if (!set || (n && !rows))
            throw std::invalid_argument("mymyr_amd: hashset_insert: null argument");
        state_set_insert(set->set, rows, n, ids, is_new, new_count, static_cast<hipStream_t>(stream));
    });
}

int mya_hashset_size(mya_hashset* set, uint64_t* size)
{
    return guarded([&] {
        if (!set || !size)
            throw std::invalid_argument("mymyr_amd: hashset_size: null argument");
        state_set_sync(set->set);
        *size = set->set.size;
    });
}

int mya_hashset_rows(const mya_hashset* set, const uint64_t** rows)
{
    return guarded([&] {
        if (!set || !rows)
            throw std::invalid_argument("mymyr_amd: hashset_rows: null argument");
        *rows = set->set.v.arena;
    });
}

int mya_hashset_clear(mya_hashset* set, void* stream)
{
    return guarded([&] {
        if (!set)
            throw std::invalid_argument("mymyr_amd: hashset_clear: null set");
        state_set_clear(set->set, static_cast<hipStream_t>(stream));
    });
}

int mya_dedup_rows(uint64_t start, uint64_t count, uint32_t words, uint64_t seed, double dup, uint64_t* out, void* stream)
{
    return guarded([&] {
        if (count && !out)
            throw std::invalid_argument("mymyr_amd: dedup_rows: null output");
        if (!(dup >= 0.0 && dup < 1.0))
            throw std::invalid_argument("mymyr_amd: dedup_rows: dup must be in [0, 1)");
        if (start + count > (u64{1} << 32))
            throw std::invalid_argument("mymyr_amd: dedup_rows: rows beyond 2^32");
        launch_dedup_rows(start, count, words, seed, dup, out, static_cast<hipStream_t>(stream));
    });
}

int mya_random_ops(uint64_t* table, uint64_t words, uint64_t n, int kind, uint64_t seed, uint64_t* sink, void* stream)
{
    return guarded([&] {
        if (!table || !sink)
            throw std::invalid_argument("mymyr_amd: random_ops: null array");
        if (words == 0 || (words & (words - 1)))
            throw std::invalid_argument("mymyr_amd: random_ops: the table's words must be a power of two");
        if (kind < 0 || kind > 3)
            throw std::invalid_argument("mymyr_amd: random_ops: kind must be 0 (load), 1 (CAS), 2 (atomic min) or 3 (store)");
        launch_random_ops(table, words, n, kind, seed, sink, static_cast<hipStream_t>(stream));
    });
}

namespace
{
[[noreturn]] void condition_error(const std::string& what) { throw std::invalid_argument("mymyr: condition: " + what); }

/// BrfsOptions::goal as GoalSpec::AnyOf (search::any_of, src/mymyr/search/goal.cpp:14-70): each condition's literals
/// are checked first (GroundCondition::validate, src/mymyr/successor/conditions.cpp:757-766), then resolved in order: a
/// static literal decided against the static facts (false: the condition can never hold and is left out), a fluent
/// atom outside its predicate's domains or without a slot is never true (a positive literal leaves its condition out, a
/// negative one is dropped), any other fluent literal becomes its slot.
/// Lazy slots: the slot of canonical atom `cid`, interned now (the next slot) if it has none, with the task's device
/// image brought up to date when it is on the device (AtomIndex::slot_if_any, include/mymyr/task/atom_index.hpp:169).
u32 intern_goal_atom(mya_task* t, u64 cid)
{
    std::lock_guard lock(t->mutex);
    CompiledTask& C = *t->compiled;
    if (C.slot_of[cid] != kNone)
        return C.slot_of[cid];
    const auto ranges = intern_atoms(C, {cid});
    if (t->dev.image)
    {
        for (const auto& [a, b] : ranges)
            if (b > a)
                hip_check(hipMemcpy(t->dev.image + a, C.image.data() + a, (b - a) * sizeof(u64), hipMemcpyHostToDevice), "task image");
        *t->dev.thost = task_dev(t->dev.image, C.header());
        t->dev.thost->missing = t->dev.missing;
    }
    return C.slot_of[cid];
}

void resolve_any_of(mya_task* task, const mya_brfs_options& op, BrfsOptionsC& o)
{
    const CompiledTask& C = *task->compiled;
    if (op.goal_test)
    {
        // GoalSpec::Custom: the caller's test decides (brfs.cpp:43-52)
        if (op.goal_kind != 0)
            throw std::invalid_argument("mymyr_amd: brfs: a custom goal test takes goal_kind 0 (no goal conditions)");
        auto fn = op.goal_test;
        void* user = op.goal_test_user;
        o.goal_test = [fn, user](const u64* rows, u64 n, u32 words, u8* out) { return fn(user, rows, n, words, out) == 0; };
        return;
    }
    if (op.goal_kind == 0)
        return;
    if (op.goal_kind != 1)
        throw std::invalid_argument("mymyr_amd: brfs: goal_kind must be 0 (the task's goal) or 1 (any of goal_count conditions)");
    if (op.goal_count && !op.goal_offsets)
        throw std::invalid_argument("mymyr_amd: brfs: goal_count without goal_offsets");
    const TaskText& T = C.text;
    o.any_of = true;
    for (u32 k = 0; k < op.goal_count; ++k)
    {
        const u32 lo = op.goal_offsets[k], hi = op.goal_offsets[k + 1];
        if (hi < lo)
            throw std::invalid_argument("mymyr_amd: brfs: goal_offsets must not decrease");
        if (hi > lo && !op.goal_literals)
            throw std::invalid_argument("mymyr_amd: brfs: goal literals missing");
        auto rec = [&](u32 l) { return op.goal_literals + static_cast<size_t>(l) * MYA_GOAL_LITERAL_INTS; };
        for (u32 l = lo; l < hi; ++l)
        {
            const int32_t* r = rec(l);
            const std::string where = "literal " + std::to_string(l - lo);
            if (r[0] < 0 || static_cast<u32>(r[0]) >= T.preds.size())
                condition_error(where + ": predicate index " + std::to_string(r[0]) + " out of range");
            const PredicateText& P = T.preds[static_cast<u32>(r[0])];
            if (r[2] < 0 || static_cast<u32>(r[2]) != P.arity)
                condition_error(where + ": " + P.name + " takes " + std::to_string(P.arity) + " arguments, got " + std::to_string(r[2]));
            if (P.arity > MYA_GOAL_LITERAL_INTS - 3)
                throw std::invalid_argument("mymyr_amd: brfs: goal literals hold at most 6 objects");
            for (u32 i = 0; i < P.arity; ++i)
                if (r[3 + i] < 0 || static_cast<u32>(r[3 + i]) >= T.objects)
                    condition_error(where + ": object index " + std::to_string(r[3 + i]) + " out of range");
        }
        std::vector<u32> pos, neg;
        bool possible = true;
        for (u32 l = lo; l < hi && possible; ++l)
        {
            const int32_t* r = rec(l);
            const u32 p = static_cast<u32>(r[0]);
            const bool positive = r[1] != 0;
            const PredicateText& P = T.preds[p];
            u32 objs[6] = {};
            for (u32 i = 0; i < P.arity; ++i)
                objs[i] = static_cast<u32>(r[3 + i]);
            if (P.kind == 'S')
            {
                if (C.static_holds(p, objs) != positive)
                    possible = false;
                continue;
            }
            if (P.kind != 'F')
                throw std::invalid_argument("mymyr_amd: brfs: goal literals over derived predicates are not supported");
            u32 slot = kNone;
            if (C.layout.size[p])
            {
                // frozen slots: the atom's slot if it has one; lazy slots: interned now, in the literals' order
                const u64 cid = C.layout.encode(p, objs, P.arity);
                if (cid < C.layout.fluent_count)
                    slot = lazy_task(task) ? intern_goal_atom(task, cid) : C.slot_of[cid];
            }
            if (slot == kNone)
            {
                if (positive)
                    possible = false;
                continue;
            }
            (positive ? pos : neg).push_back(slot);
        }
        if (possible)
        {
            o.goal_pos.push_back(std::move(pos));
            o.goal_neg.push_back(std::move(neg));
        }
    }
}
}  // namespace

int mya_brfs(mya_task* task, const mya_brfs_options* options, mya_brfs_result* result, uint64_t* layer_counts, uint32_t cap,
             mya_brfs_plan* plan)
{
    int layers = -1;
    const int rc = guarded([&] {
        if (!task || !options || !result)
            throw std::invalid_argument("mymyr_amd: brfs: null argument");
        // lazy slots: the search interns atoms into the task; it holds the task for its whole run
        std::unique_lock<std::mutex> lazy_lock;
        LazyResolve resolve;
        if (lazy_task(task))
        {
            lazy_lock = std::unique_lock<std::mutex>(task->lazy_mutex);
            resolve = [task](hipStream_t s, TaskDev* T) {
                const bool any = resolve_missing(task, s);
                *T = *device_task(task).thost;
                return any;
            };
        }
        BrfsOptionsC o;
        o.max_depth = options->max_depth;
        o.witness_pruning = options->witness_pruning;
        o.max_states = options->max_states;
        o.max_expanded = options->max_expanded;
        o.stop_at_goal = options->stop_at_goal;
        o.fingerprint = options->fingerprint;
        o.chunk = options->chunk;
        o.memory_states = options->memory_states;
        o.timings = options->timings;
        const u32 TW = task->compiled->words;
        if ((options->start || options->blocked_count) && options->words != TW)
            throw std::invalid_argument("mymyr_amd: brfs: start and blocked rows have " + std::to_string(options->words) +
                                        " words, the task's rows " + std::to_string(TW));
        if (options->blocked_count && !options->blocked)
            throw std::invalid_argument("mymyr_amd: brfs: blocked_count without blocked rows");
        if (options->start)
            o.start.assign(options->start, options->start + TW);
        if (options->blocked_count)
            o.blocked.assign(options->blocked, options->blocked + options->blocked_count * TW);
        o.timed = options->timed != 0;
        o.max_seconds = options->max_seconds;
        o.cancel = options->cancel;
        resolve_any_of(task, *options, o);
        // the observer (search::SearchObserver, include/mymyr/search/control.hpp:157-186): on_start here, on_pass and
        // on_progress from inside the drivers, on_solution and on_end once the result is known (Control::finish,
        // src/mymyr/search/brfs.cpp:193-211)
        const mya_search_observer* obs = options->observer;
        o.progress_interval = options->progress_interval ? options->progress_interval : u64{1} << 16;
        if (obs && obs->on_pass)
            o.on_pass = [obs](u32 layer, const std::array<u64, 3>& c, double seconds) {
                const mya_search_statistics st{c[0], c[1], c[2], 0, seconds, 0};
                obs->on_pass(obs->user, layer, &st);
            };
        if (obs && obs->on_progress)
            o.on_progress = [obs](u64 expanded, u64 generated, u64 states, double seconds) {
                const mya_search_statistics st{expanded, generated, states, 0, seconds, 0};
                return obs->on_progress(obs->user, &st) != 0;
            };
        if (obs && obs->on_expand)
            o.on_expand = [obs](u64 id, const u64* row, u32 words) { obs->on_expand(obs->user, id, row, words); };
        if (obs && obs->on_generate)
            o.on_generate = [obs](u64 parent, u32 schema, const i32* binding, u32 arity, u64 child, const u64* row, u32 words, bool is_new) {
                obs->on_generate(obs->user, parent, static_cast<i32>(schema), binding, arity, child, row, words, is_new ? 1 : 0);
            };
        if (obs && obs->on_prune)
            o.on_prune = [obs](u64 parent, u32 schema, const i32* binding, u32 arity, const u64* row, u32 words) {
                obs->on_prune(obs->user, parent, static_cast<i32>(schema), binding, arity, row, words);
            };
        if (obs && obs->on_start)
        {
            const std::vector<u64>& s0 = o.start.empty() ? task->compiled->initial : o.start;
            obs->on_start(obs->user, s0.data(), static_cast<u32>(s0.size()));
        }
        // BrfsOptions::layers with the reference's checks (check_layers, include/mymyr/search/layer_ordering.hpp:117-134)
        {
            const i32 k = options->layer_kind;
            const u32 limit = options->max_next_layer_states ? options->max_next_layer_states : ~u32{0};
            const u32 beam = options->beam_width ? options->beam_width : ~u32{0};
            auto bad = [](const std::string& m) { throw std::invalid_argument("mymyr brfs: " + m); };
            if (k < 0 || k > 5)
                bad("layer_kind must be 0 (queue) .. 5 (scored)");
            if (k == 0 && limit != ~u32{0})
                bad("max_next_layer_states needs an ordered layer order (any but the queue)");
            if (beam != ~u32{0} && k == 0)
                bad("beam_width needs an ordered layer order (any but the queue)");
            if (beam != ~u32{0} && limit != ~u32{0})
                bad("beam_width and max_next_layer_states exclude each other");
            if (options->beam_novelty < 0 || options->beam_novelty > 2)
                bad("beam_novelty must be 0 (all tested), 1 (survivors only) or 2 (relaxed survivors only)");
            if (beam == ~u32{0} && options->beam_novelty != 0)
                bad("a beam novelty other than all-tested needs a beam (beam_width)");
            if (options->randomize_ties && k != 4 && k != 5)
                bad("randomize_ties needs a layer order with scores (goal count or a scorer)");
            if ((k == 5) != (options->layer_scorer != nullptr))
                bad("a scorer is needed by the scored layer order and taken by no other");
            if (options->beam_novelty == 2)
            {
                if (k != 4)
                    bad("the relaxed survivors-only beam novelty needs the goal-count layer order (it ranks by score)");
                throw std::invalid_argument("mymyr_amd: brfs: the relaxed survivors-only beam is not supported by the device search");
            }
            o.layer_kind = k;
            o.layer_seed = options->layer_seed;
            o.max_next_layer_states = limit;
            o.prefer_more_satisfied_goals = options->prefer_fewer_satisfied_goals == 0;
            o.beam_width = beam;
            o.randomize_ties = options->randomize_ties != 0;
            if (k == 5)
            {
                auto fn = options->layer_scorer;
                void* user = options->layer_scorer_user;
                o.scorer = [fn, user](const u64* rows, u64 n, u32 words, double* scores) { fn(user, rows, n, words, scores); };
            }
        }
        std::vector<std::array<u64, 3>> lc;
        BrfsResultC r;
        bool searched = true;
        if (o.stop_at_goal && !o.any_of && !o.goal_test && task->compiled->goal_fixed_unsat)
        {
            // the task's goal fails in every state: the start state alone, nothing expanded (brfs.cpp:1851-1861)
            r.status = kUnsolvable;
            r.states = 1;
            searched = false;
        }
        else
        {
            const bool lifted = resolve || task->compiled->words > 16;
            r = brfs_device(*task->compiled, o, lc, &task->brfs, lifted ? device_task(task).thost.get() : nullptr,
                            resolve ? &resolve : nullptr);
        }
        std::memset(result, 0, sizeof(*result));
        result->status = r.status;
        result->solved = r.solved;
        result->exhausted = r.exhausted;
        result->layers = r.layers;
        result->states = r.states;
        result->expanded = r.expanded;
        result->generated = r.generated;
        result->goal_states = r.goal_states;
        result->fingerprint = r.fingerprint;
        result->first_goal = r.first_goal;
        result->search_s = r.search_s;
        result->device_s = r.device_s;
        result->pruned = r.pruned;
        result->memory_bytes = r.memory_bytes;
        result->words = task->compiled->words;
        result->fluent_slots = task->compiled->fluent_slots;
        result->threads_used = 1;
        std::snprintf(result->store, sizeof(result->store), "%s", searched ? "device" : "none");
        if (plan)
        {
            if (plan->binding && plan->label_width < r.plan_width)
                throw std::invalid_argument("mymyr_amd: brfs: plan label width " + std::to_string(plan->label_width) +
                                            " is below the task's " + std::to_string(r.plan_width));
            const u32 len = static_cast<u32>(r.plan_schema.size());
            plan->length = len;
            plan->cost = r.cost;
            plan->goal_words = static_cast<u32>(r.goal_state.size());
            for (u32 i = 0; i < len && i < plan->cap; ++i)
            {
                if (plan->schema)
                    plan->schema[i] = r.plan_schema[i];
                if (plan->binding)
                    for (u32 k = 0; k < plan->label_width; ++k)
                        plan->binding[static_cast<size_t>(i) * plan->label_width + k] =
                            k < r.plan_width ? r.plan_binding[static_cast<size_t>(i) * r.plan_width + k] : -1;
            }
            if (plan->goal_state)
                for (u32 w = 0; w < plan->goal_cap; ++w)
                    plan->goal_state[w] = w < r.goal_state.size() ? r.goal_state[w] : 0;
        }
        for (int k = 0; k < kKClasses; ++k)
        {
            result->kernel_ms[k] = r.kernel_ms[k];
            result->kernel_bytes[k] = r.kernel_bytes[k];
            result->kernel_launches[k] = r.kernel_launches[k];
        }
        if (layer_counts)
            for (size_t i = 0; i < lc.size() && i < cap; ++i)
                for (int j = 0; j < 3; ++j)
                    layer_counts[i * 3 + j] = lc[i][j];
        layers = static_cast<int>(lc.size());
        if (obs && obs->on_solution && r.solved)
            obs->on_solution(obs->user, r.plan_schema.data(), r.plan_binding.data(), static_cast<u32>(r.plan_schema.size()),
                             r.plan_width, r.cost);
        if (obs && obs->on_end)
        {
            const mya_search_statistics st{r.expanded, r.generated, r.states, r.pruned, r.search_s, 0};
            obs->on_end(obs->user, r.status, &st);
        }
    });
    return rc == 0 ? layers : -1;
}

}  // extern "C"
