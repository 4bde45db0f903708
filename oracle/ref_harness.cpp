// Test infrastructure, not product code: a C-ABI harness over the reference CPU core (maichmueller/mymyr), compiled
// together with the reference's own sources by oracle/Makefile into oracle/_ref/libmymyr_ref.so. Only tests/,
// the smoke check and bench.py's CPU-baseline leg load it; the product library never links or calls it.
//
// Every entry point is a thin call into the reference API it names:
//   task loading          Task::from_text_file           include/mymyr/task/task.hpp:166-167
//   slot records          AtomIndex::record / canonical  include/mymyr/task/atom_index.hpp:167-172
//   successors            Successors::generate           include/mymyr/successor/successors.hpp:154-248
//   hashes                hash::words / hash::state      include/mymyr/core/hash.hpp:38-60
//   Philox                rl::rng::block                 include/mymyr/rl/rng.hpp:45-83
//   env step / reset      rl::HostEnv                    include/mymyr/rl/env.hpp:181-278
//   env pool              rl::CpuEnvPool                 include/mymyr/rl/pool.hpp:114-172 (reset, send, recv, recv_ticket)
//   BrFS                  brfs(Task, BrfsOptions)        include/mymyr/search/brfs.hpp:140
//   dedup                 FlatStateStore::insert         include/mymyr/state/flat_store.hpp:44-115
//                         ConcurrentStateStore::insert   include/mymyr/state/concurrent_store.hpp:79-177
// Errors: functions return a negative value (or null) and mref_last_error() holds the message.

#include "mymyr/core/hash.hpp"
#include "mymyr/rl/env.hpp"
#include "mymyr/rl/expand.hpp"
#include "mymyr/rl/pool.hpp"
#include "mymyr/rl/rng.hpp"
#include "mymyr/rl/task_suite.hpp"
#include "mymyr/rl/task_table.hpp"
#include "mymyr/rl/visited.hpp"
#include "mymyr/core/team.hpp"
#include "mymyr/search/brfs.hpp"
#include "mymyr/search/goal.hpp"
#include "mymyr/state/concurrent_store.hpp"
#include "mymyr/state/flat_store.hpp"
#include "mymyr/successor/successors.hpp"
#include "mymyr/task/task.hpp"
#include "mymyr/task/workspace.hpp"

#include <algorithm>
#include <atomic>
#include <chrono>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <exception>
#include <memory>
#include <string>
#include <vector>

using namespace mymyr;

namespace
{
thread_local std::string g_error;

template<class F>
auto guarded(F&& f, decltype(f()) on_error) -> decltype(f())
{
    try
    {
        return f();
    }
    catch (const std::exception& e)
    {
        g_error = e.what();
    }
    catch (...)
    {
        g_error = "unknown exception";
    }
    return on_error;
}
}  // namespace

struct mref_task
{
    TaskPtr task;
    rl::TaskTablePtr table;
};

struct mref_env
{
    std::unique_ptr<rl::HostEnv> env;
    std::unique_ptr<ThreadPool> pool;
};

extern "C" {

struct mref_env_config
{
    uint64_t seed;
    uint32_t max_steps;
    float step_reward;
    float goal_reward;
    float dead_end_reward;
    int32_t dead_end;  // 0 no_successors, 1 none
    int32_t dead_end_terminal;
    int32_t autoreset;
    int32_t canonical_order;
    int32_t witness_pruning;
    int32_t label_actions;  // ActionSpace::Label
};

struct mref_brfs_options
{
    uint32_t threads;
    uint32_t max_depth;
    uint64_t max_states;
    int32_t witness_pruning;
    int32_t canonical_order;
    int32_t stop_at_goal;
    int32_t fingerprint;
    uint64_t max_expanded;
    const uint64_t* start;    // [words] (null: the task's initial state)
    const uint64_t* blocked;  // [blocked_count, words]
    uint64_t blocked_count;
    uint32_t words;
    uint32_t reserved;
    double max_seconds;       // BrfsOptions::max_seconds (infinity: unbounded)
    // BrfsOptions::goal: goal_kind 1 = search::any_of over goal_count ground conditions, condition k's literals the
    // 8-int32 records [goal_offsets[k], goal_offsets[k + 1]) of goal_literals: predicate, positive, then the objects
    int32_t goal_kind;
    uint32_t goal_count;
    const uint32_t* goal_offsets;
    const int32_t* goal_literals;
    // BrfsOptions::layers: kind (LayerOrdering::Kind order), seed, max_next_layer_states / beam_width (0: none),
    // prefer_fewer (prefer_more_satisfied_goals false), randomize_ties, and for the scored kind a scorer over host rows
    int32_t layer_kind;
    int32_t prefer_fewer;
    uint64_t layer_seed;
    uint32_t max_next_layer_states;
    uint32_t beam_width;
    int32_t randomize_ties;
    int32_t record_events;  // record the observer's events (mref_brfs_events)
    void (*scorer)(void* user, const uint64_t* rows, uint64_t n, uint32_t words, double* scores);
    void* scorer_user;
    // goal_kind 2: GoalSpec::Custom, a state is a goal iff its hash_state % goal_mod == goal_res (a test that no atom
    // goal expresses); goal_kind 3: GoalSpec::Custom, iff the state has goal_res true atoms
    uint64_t goal_mod;
    uint64_t goal_res;
};

namespace
{
/// The events of search::SearchObserver as 7-word records: kind (0 start, 1 expand, 2 generate, 3 prune, 4 pass,
/// 5 solution, 6 end) then its fields; states by their hash_state, bindings by a polynomial hash of their objects
/// (h = arity, then h = h * 1000003 + object).
struct EventLog final : search::SearchObserver
{
    std::vector<uint64_t> ev;
    void rec(uint64_t a, uint64_t b = 0, uint64_t c = 0, uint64_t d = 0, uint64_t e = 0, uint64_t f = 0, uint64_t g = 0)
    {
        ev.insert(ev.end(), {a, b, c, d, e, f, g});
    }
    static uint64_t sh(StateView s) { return hash::state(s.w, s.nw, s.num, s.nnum); }
    static uint64_t bh(const Action& a)
    {
        uint64_t h = a.binding.size();
        for (ObjectId o : a.binding)
            h = h * 1000003ull + o.v;
        return h;
    }
    void on_start(StateView s) override { rec(0, sh(s)); }
    void on_expand(u64 id, StateView s) override { rec(1, id, sh(s)); }
    void on_generate(u64 parent, const Action& a, u64 child, StateView s, bool is_new) override
    {
        rec(2, parent, a.schema.v, bh(a), child, sh(s), is_new ? 1 : 0);
    }
    void on_prune(u64 parent, const Action& a, StateView s) override { rec(3, parent, a.schema.v, bh(a), 0, sh(s)); }
    void on_pass(u32 layer, const search::SearchStatistics& st) override { rec(4, layer, st.expanded, st.generated, st.states); }
    void on_solution(std::span<const Action> plan, double cost) override
    {
        uint64_t h = plan.size();
        for (const Action& a : plan)
            h = h * 1000003ull + a.schema.v * 7919ull + bh(a);
        rec(5, plan.size(), h, static_cast<uint64_t>(cost));
    }
    void on_end(search::SearchStatus status, const search::SearchStatistics& st) override
    {
        rec(6, static_cast<uint64_t>(status), st.expanded, st.generated, st.states, st.pruned);
    }
};
thread_local std::vector<uint64_t> g_events;
}  // namespace

/// The events recorded by the last mref_brfs with record_events: count records of 7 words (copied up to cap records).
uint64_t mref_brfs_events(uint64_t* out, uint64_t cap)
{
    const uint64_t n = g_events.size() / 7;
    if (out)
        std::memcpy(out, g_events.data(), std::min(n, cap) * 7 * sizeof(uint64_t));
    return n;
}

struct mref_brfs_result
{
    uint64_t states, expanded, generated, goal_states, fingerprint;
    uint32_t layers;
    int32_t status;
    int32_t solved;
    int32_t exhausted;
    double seconds;
    double cost;
    uint64_t pruned;
    uint32_t plan_len;  // actions of the plan (those past plan_cap are not written)
    uint32_t goal_words;  // words of goal_state (0: none)
    uint32_t words;         // BrfsResult::words
    uint32_t fluent_slots;  // BrfsResult::fluent_slots
    uint32_t threads_used;  // BrfsResult::threads_used
    uint32_t reserved;
    char store[16];         // BrfsResult::store
    char message[256];      // BrfsResult::message
};

const char* mref_last_error() { return g_error.c_str(); }

// atoms: 0 auto, 1 reachable, 2 dense, 3 lazy (a lazy task has no table: TaskTable refuses lazy slots)
mref_task* mref_task_load(const char* path, int atoms)
{
    return guarded(
        [&]() -> mref_task*
        {
            TaskOptions o;
            o.atoms = atoms == 1   ? TaskOptions::Atoms::Reachable
                      : atoms == 2 ? TaskOptions::Atoms::Dense
                      : atoms == 3 ? TaskOptions::Atoms::Lazy
                                   : TaskOptions::Atoms::Auto;
            auto t = new mref_task;
            t->task = Task::from_text_file(path, o);
            if (atoms != 3)
                t->table = rl::TaskTable::single(t->task);
            return t;
        },
        nullptr);
}

void mref_task_free(mref_task* t) { delete t; }

// out: words, fluent_slots, mode (0 reachable, 1 dense, 2 lazy), num_schemas, label_width, num_objects, max_arity,
// table_words, dense_fluent (typed-dense canonical fluent count)
int mref_task_info(mref_task* t, uint64_t* out)
{
    return guarded(
        [&]() -> int
        {
            const Task& k = *t->task;
            out[0] = k.words();
            out[1] = k.atoms().fluent_slots();
            out[2] = static_cast<uint64_t>(k.atoms().mode());
            out[3] = k.num_schemas();
            u32 lw = 0;
            for (const auto& sc : k.data().schemas)
                lw = std::max(lw, sc.arity());
            out[4] = t->table ? t->table->label_width() : lw;
            out[5] = k.data().num_objects();
            out[6] = k.atoms().layout().max_arity;
            out[7] = t->table ? t->table->words() : k.words();
            out[8] = k.atoms().layout().fluent_count;
            return 0;
        },
        -1);
}

// rec: [fluent_slots, 1 + max(1, max_arity)] = predicate then arguments; cid: [fluent_slots]
int mref_task_slots(mref_task* t, uint32_t* rec, uint64_t* cid)
{
    return guarded(
        [&]() -> int
        {
            const AtomIndex& a = t->task->atoms();
            const u32 n = a.fluent_slots();
            const u32 stride = 1 + std::max<u32>(1, a.layout().max_arity);
            for (u32 s = 0; s < n; ++s)
            {
                const u32* r = a.record(AtomKind::Fluent, s);
                for (u32 j = 0; j < stride; ++j)
                    rec[static_cast<usize>(s) * stride + j] = j <= a.layout().arity[r[0]] ? r[j] : 0;
                cid[s] = a.canonical(AtomKind::Fluent, s);
            }
            return 0;
        },
        -1);
}

// the initial state, zero-padded to `words`
int mref_task_initial(mref_task* t, uint64_t* row, uint32_t words)
{
    return guarded(
        [&]() -> int
        {
            const State& s = t->task->initial_state();
            std::memset(row, 0, words * sizeof(uint64_t));
            const auto w = s.words();
            if (w.size() > words)
                throw std::length_error("initial state wider than the row");
            std::memcpy(row, w.data(), w.size() * sizeof(uint64_t));
            return 0;
        },
        -1);
}

int mref_task_goal(mref_task* t, const uint64_t* row, uint32_t nw)
{
    return guarded([&]() -> int { return t->task->is_goal(StateView{row, bits::trimmed_size(row, nw), nullptr, 0}) ? 1 : 0; }, -1);
}

uint64_t mref_canonical_hash(mref_task* t, const uint64_t* row, uint32_t nw)
{
    return t->task->canonical_hash(StateView{row, bits::trimmed_size(row, nw), nullptr, 0});
}

// The successors of a state in the generator's order: schema [cap], binding [cap, L] (-1 padded), rows [cap, W]
// (zero padded; W >= the task's words). Returns the successor count (which may exceed cap; only cap are written).
int64_t mref_successors(mref_task* t, const uint64_t* row, uint32_t nw, int witness, int canonical, int32_t* schema,
                        int32_t* binding, uint32_t L, uint64_t* rows, uint32_t W, uint64_t cap)
{
    return guarded(
        [&]() -> int64_t
        {
            const WorkspaceLease lease = t->task->workspace();
            Successors& succ = lease->successors();
            const u32 n = bits::trimmed_size(row, nw);
            succ.prepare(StateView{row, n, nullptr, 0});
            std::vector<u64> next;
            int64_t count = 0;
            succ.generate<false>(
                [&](u32 s, const ObjectId* b, const Delta& d) -> bool
                {
                    if (static_cast<uint64_t>(count) < cap)
                    {
                        if (schema)
                            schema[count] = static_cast<int32_t>(s);
                        if (binding)
                            for (u32 k = 0; k < L; ++k)
                                binding[count * L + k] = k < succ.arity(s) ? static_cast<int32_t>(b[k].v) : -1;
                        if (rows)
                        {
                            const u32 m = apply_delta(row, n, d, next);
                            if (m > W)
                                throw std::length_error("successor wider than the row");
                            uint64_t* dst = rows + count * W;
                            std::memset(dst, 0, W * sizeof(uint64_t));
                            std::memcpy(dst, next.data(), m * sizeof(uint64_t));
                        }
                    }
                    ++count;
                    return true;
                },
                witness != 0, canonical != 0);
            return count;
        },
        -1);
}

uint64_t mref_hash_words(const uint64_t* w, uint32_t n, uint64_t seed) { return hash::words(w, n, seed); }
uint64_t mref_hash_state(const uint64_t* w, uint32_t n) { return hash::state(w, n, nullptr, 0); }
// hash_state of each of n rows of `words` words, `stride` words apart
void mref_hash_rows(const uint64_t* rows, uint64_t n, uint32_t words, uint32_t stride, uint64_t* out)
{
    for (uint64_t i = 0; i < n; ++i)
        out[i] = hash::state(rows + i * stride, words, nullptr, 0);
}
uint64_t mref_hash_mix64(uint64_t x) { return hash::mix64(x); }

void mref_philox(uint64_t seed, uint64_t env, uint64_t draw, uint32_t purpose, uint32_t* out)
{
    const rl::rng::Block4 b = rl::rng::block(seed, env, draw, purpose);
    for (int i = 0; i < 4; ++i)
        out[i] = b.v[i];
}

void mref_philox_raw(const uint32_t* counter, uint32_t k0, uint32_t k1, uint32_t* out)
{
    const rl::rng::Block4 b = rl::rng::philox4x32_10(rl::rng::Block4{{counter[0], counter[1], counter[2], counter[3]}}, k0, k1);
    for (int i = 0; i < 4; ++i)
        out[i] = b.v[i];
}

uint32_t mref_successor_index(uint64_t seed, uint64_t env, uint64_t draw, uint32_t count)
{
    return rl::rng::successor_index(seed, env, draw, count);
}

static rl::EnvConfig env_config(const mref_env_config* c)
{
    rl::EnvConfig e;
    e.seed = c->seed;
    e.max_steps = c->max_steps;
    e.step_reward = c->step_reward;
    e.goal_reward = c->goal_reward;
    e.dead_end_reward = c->dead_end_reward;
    e.dead_end = c->dead_end == 1 ? rl::DeadEnd::None : rl::DeadEnd::NoSuccessors;
    e.dead_end_terminal = c->dead_end_terminal != 0;
    e.autoreset = c->autoreset != 0;
    e.canonical_order = c->canonical_order != 0;
    e.witness_pruning = c->witness_pruning != 0;
    e.actions = c->label_actions ? rl::ActionSpace::Label : rl::ActionSpace::Index;
    return e;
}

mref_env* mref_env_create(mref_task* t, const mref_env_config* c, uint32_t threads)
{
    return guarded(
        [&]() -> mref_env*
        {
            auto e = new mref_env;
            e->env = std::make_unique<rl::HostEnv>(t->table, env_config(c));
            if (threads > 1)
                e->pool = std::make_unique<ThreadPool>(threads);
            return e;
        },
        nullptr);
}

void mref_env_free(mref_env* e) { delete e; }

int mref_env_reset(mref_env* e, uint64_t* states, uint64_t rows, uint32_t words, int32_t* steps, uint64_t* draws,
                   uint8_t* at_goal, int32_t* count, uint64_t first_env)
{
    return guarded(
        [&]() -> int
        {
            rl::EnvBatch b;
            b.states = states;
            b.rows = rows;
            b.words = words;
            b.steps = steps;
            b.draws = draws;
            b.at_goal = at_goal;
            b.first_env = first_env;
            e->env->reset(b, nullptr, count);
            return 0;
        },
        -1);
}

// actions: null for the random policy
int mref_env_step(mref_env* e, uint64_t* states, uint64_t rows, uint32_t words, int32_t* steps, uint64_t* draws,
                  uint8_t* at_goal, uint64_t first_env, const int64_t* actions, float* reward, uint8_t* terminated,
                  uint8_t* truncated, int32_t* count, int32_t* schema, int32_t* binding, uint32_t label_width,
                  uint8_t* goal, uint8_t* invalid, uint64_t* final_states)
{
    return guarded(
        [&]() -> int
        {
            rl::EnvBatch b;
            b.states = states;
            b.rows = rows;
            b.words = words;
            b.steps = steps;
            b.draws = draws;
            b.at_goal = at_goal;
            b.first_env = first_env;
            rl::StepOutputs o;
            o.reward = reward;
            o.terminated = terminated;
            o.truncated = truncated;
            o.count = count;
            o.schema = schema;
            o.binding = binding;
            o.label_width = label_width;
            o.goal = goal;
            o.invalid = invalid;
            o.final_states = final_states;
            rl::Actions a;
            a.v64 = actions;
            e->env->step(b, o, a, nullptr, e->pool.get());
            return 0;
        },
        -1);
}

// A HostEnv over TaskTable::create(tasks) (include/mymyr/rl/task_table.hpp:69-75): several instances of one domain
// (suite: over TaskSuite::group(tasks), include/mymyr/rl/task_suite.hpp:62-64, instances of several domains),
// with an instance sampler (rl/sampling.hpp) when sampled_instances > 0 (m = 0: uniform; else thresholds [m - 1] and
// indices [m]). Null (and the table's message in mref_last_error) when the tasks are not of one domain.
mref_env* mref_table_env_create(mref_task* const* tasks, uint32_t n, const mref_env_config* c, uint32_t sampled_instances,
                                const uint32_t* thresholds, const int32_t* indices, uint32_t m, int suite)
{
    return guarded(
        [&]() -> mref_env*
        {
            std::vector<TaskPtr> v;
            for (uint32_t i = 0; i < n; ++i)
                v.push_back(tasks[i]->task);
            rl::EnvConfig cfg = env_config(c);
            cfg.sampling.instances = sampled_instances;
            if (m)
            {
                cfg.sampling.thresholds.assign(thresholds, thresholds + m - 1);
                cfg.sampling.indices.assign(indices, indices + m);
            }
            auto e = new mref_env;
            if (suite)  // TaskSuite::group: several domains, global ids in task order
                e->env = std::make_unique<rl::HostEnv>(rl::TaskSuite::group(std::move(v)), cfg);
            else
                e->env = std::make_unique<rl::HostEnv>(rl::TaskTable::create(std::move(v)), cfg);
            return e;
        },
        nullptr);
}

// The arrays of a table batch (rl::EnvBatch, include/mymyr/rl/env.hpp:96-135); null arrays are absent.
struct mref_table_batch
{
    uint64_t* states;
    uint64_t rows;
    uint32_t words;
    uint32_t reserved;
    int32_t* steps;
    uint64_t* draws;
    uint8_t* at_goal;
    uint64_t first_env;
    int32_t* task_ids;
    uint64_t* goal_pos;
    uint64_t* goal_neg;
    uint32_t* reset_counts;
    const uint64_t* seeds;
    const uint32_t* env_ids;
    const uint64_t* sampling_seeds;
    uint64_t* visited;        // [rows, visited_capacity] (null: no visited tables)
    int32_t* visited_count;   // [rows]
    int32_t* visited_status;  // [1]
    uint32_t visited_capacity;
    uint32_t reserved2;
};

static rl::EnvBatch table_batch(const mref_table_batch* t)
{
    rl::EnvBatch b;
    b.states = t->states;
    b.rows = t->rows;
    b.words = t->words;
    b.steps = t->steps;
    b.draws = t->draws;
    b.at_goal = t->at_goal;
    b.first_env = t->first_env;
    b.task_ids = t->task_ids;
    b.goal_pos = t->goal_pos;
    b.goal_neg = t->goal_neg;
    b.reset_counts = t->reset_counts;
    b.seeds = t->seeds;
    b.env_ids = t->env_ids;
    b.sampling_seeds = t->sampling_seeds;
    b.visited = t->visited;
    b.visited_count = t->visited_count;
    b.visited_status = t->visited_status;
    b.visited_capacity = t->visited ? t->visited_capacity : 0;
    return b;
}

// HostEnv::clear_visited over a table batch (include/mymyr/rl/env.hpp:210-211): mask [rows] (null: all rows).
int mref_table_env_clear_visited(mref_env* e, const mref_table_batch* t, const uint8_t* mask)
{
    return guarded(
        [&]() -> int
        {
            rl::EnvBatch b = table_batch(t);
            e->env->clear_visited(b, mask);
            return 0;
        },
        -1);
}

// HostEnv::reset over a table batch: mask [rows] (null: all), keep_goals, sample (draw the reset rows' instances).
int mref_table_env_reset(mref_env* e, const mref_table_batch* t, int32_t* count, const uint8_t* mask, int keep_goals, int sample)
{
    return guarded(
        [&]() -> int
        {
            rl::EnvBatch b = table_batch(t);
            e->env->reset(b, mask, count, keep_goals != 0, sample != 0);
            return 0;
        },
        -1);
}

// HostEnv::step over a table batch: actions (null: the random policy), next_task_ids [rows] (null: an autoreset restarts
// in the row's next sampled instance with reset counters and a sampler, else in its own); final_states
// [rows, final_words] (final_words 0: the batch's words).
int mref_table_env_step(mref_env* e, const mref_table_batch* t, const int64_t* actions, const int32_t* next_task_ids, float* reward,
                        uint8_t* terminated, uint8_t* truncated, int32_t* count, int32_t* schema, int32_t* binding,
                        uint32_t label_width, uint8_t* goal, uint8_t* invalid, uint64_t* final_states, uint32_t final_words,
                        uint8_t* revisited)
{
    return guarded(
        [&]() -> int
        {
            rl::EnvBatch b = table_batch(t);
            rl::StepOutputs o;
            o.reward = reward;
            o.terminated = terminated;
            o.truncated = truncated;
            o.count = count;
            o.schema = schema;
            o.binding = binding;
            o.label_width = label_width;
            o.goal = goal;
            o.invalid = invalid;
            o.final_states = final_states;
            o.words = final_words;
            o.revisited = revisited;
            rl::Actions a;
            a.v64 = actions;
            e->env->step(b, o, a, next_task_ids, nullptr);
            return 0;
        },
        -1);
}

// HostEnv::step with explicit labels (include/mymyr/rl/env.hpp:216-219) on an env created with label actions: schema
// [rows], binding [rows, stride].
int mref_table_env_step_labels(mref_env* e, const mref_table_batch* t, const int32_t* label_schema, const int32_t* label_binding,
                               uint32_t stride, const int32_t* next_task_ids, float* reward, uint8_t* terminated, uint8_t* truncated,
                               int32_t* count, int32_t* schema, int32_t* binding, uint32_t label_width, uint8_t* goal, uint8_t* invalid,
                               uint64_t* final_states, uint32_t final_words, uint8_t* revisited)
{
    return guarded(
        [&]() -> int
        {
            rl::EnvBatch b = table_batch(t);
            rl::StepOutputs o;
            o.reward = reward;
            o.terminated = terminated;
            o.truncated = truncated;
            o.count = count;
            o.schema = schema;
            o.binding = binding;
            o.label_width = label_width;
            o.goal = goal;
            o.invalid = invalid;
            o.final_states = final_states;
            o.words = final_words;
            o.revisited = revisited;
            rl::Labels l{label_schema, label_binding, stride};
            e->env->step(b, o, l, next_task_ids, nullptr);
            return 0;
        },
        -1);
}

// rl::expand over TaskSuite::group(tasks) (include/mymyr/rl/expand.hpp:133-150; one domain: its table): states [rows, words], task_ids [rows];
// outputs of `capacity` rows (succ [capacity, words], parent, schema, binding [capacity, label_width], goal, succ_hash,
// noop, index) and offsets [rows + 1]. Returns generated; total through *total.
int64_t mref_table_expand(mref_task* const* tasks, uint32_t n, const uint64_t* states, const int32_t* task_ids, uint64_t rows,
                          uint32_t words, int drop_noops, uint64_t capacity, uint64_t* succ, int32_t* parent, int32_t* schema,
                          int32_t* binding, uint32_t label_width, uint8_t* goal, uint64_t* succ_hash, uint8_t* noop, int32_t* index,
                          int32_t* offsets, uint64_t* total)
{
    return guarded(
        [&]() -> int64_t
        {
            std::vector<TaskPtr> v;
            for (uint32_t i = 0; i < n; ++i)
                v.push_back(tasks[i]->task);
            const rl::TaskSuitePtr suite = rl::TaskSuite::group(std::move(v));
            rl::StateBatchView in;
            in.data = states;
            in.rows = rows;
            in.words = words;
            rl::Expansion out;
            out.capacity = capacity;
            out.words = words;
            out.label_width = label_width;
            out.succ = succ;
            out.parent = parent;
            out.schema = schema;
            out.binding = binding;
            out.goal = goal;
            out.succ_hash = succ_hash;
            out.noop = noop;
            out.index = index;
            out.offsets = offsets;
            rl::ExpandOptions o;
            o.drop_noops = drop_noops != 0;
            rl::expand(*suite, in, task_ids, out, o);
            *total = out.total;
            return static_cast<int64_t>(out.generated);
        },
        -1);
}

// rl::pad (include/mymyr/rl/expand.hpp:155-183) of the full flat expansion of a suite batch (rl::expand with capacity for
// every successor, drop_noops as given) into [rows, k] arrays: index, mask, count [rows], succ [rows, k, words], schema,
// binding [rows, k, label_width], goal, succ_hash, noop, canonical. Returns the overflow flag (or -1).
int mref_table_pad(mref_task* const* tasks, uint32_t n, const uint64_t* states, const int32_t* task_ids, uint64_t rows, uint32_t words,
                   int drop_noops, uint32_t k, uint32_t label_width, int32_t* index, uint8_t* mask, int32_t* count, uint64_t* succ,
                   int32_t* schema, int32_t* binding, uint8_t* goal, uint64_t* succ_hash, uint8_t* noop, int32_t* canonical)
{
    return guarded(
        [&]() -> int
        {
            std::vector<TaskPtr> v;
            for (uint32_t i = 0; i < n; ++i)
                v.push_back(tasks[i]->task);
            const rl::TaskSuitePtr suite = rl::TaskSuite::group(std::move(v));
            rl::StateBatchView in;
            in.data = states;
            in.rows = rows;
            in.words = words;
            rl::ExpandOptions o;
            o.drop_noops = drop_noops != 0;
            std::vector<int32_t> off(rows + 1);
            rl::Expansion probe;
            probe.offsets = off.data();
            probe.words = words;
            rl::expand(*suite, in, task_ids, probe, o);
            const u64 cap = probe.generated;
            std::vector<u64> fs(cap * words);
            std::vector<int32_t> fp(cap), fsch(cap), fb(cap * label_width), fix(cap);
            std::vector<u8> fg(cap), fn(cap);
            std::vector<u64> fh(cap);
            rl::Expansion flat;
            flat.capacity = cap;
            flat.words = words;
            flat.label_width = label_width;
            flat.succ = fs.data();
            flat.parent = fp.data();
            flat.schema = fsch.data();
            flat.binding = fb.data();
            flat.goal = fg.data();
            flat.succ_hash = fh.data();
            flat.noop = fn.data();
            flat.index = fix.data();
            flat.offsets = off.data();
            rl::expand(*suite, in, task_ids, flat, o);
            rl::PaddedExpansion out;
            out.k = k;
            out.index = index;
            out.mask = mask;
            out.count = count;
            out.words = words;
            out.succ = succ;
            out.schema = schema;
            out.label_width = label_width;
            out.binding = binding;
            out.goal = goal;
            out.succ_hash = succ_hash;
            out.noop = noop;
            out.canonical = canonical;
            rl::pad(flat, rows, out);
            return out.overflow ? 1 : 0;
        },
        -1);
}

// rl::visited_insert (include/mymyr/rl/visited.hpp:31-52) of `n` hashes into one table of H slots: present[i] for each.
void mref_visited_insert(uint64_t* table, uint32_t H, int32_t* count, const uint64_t* hashes, uint64_t n, uint8_t* present)
{
    for (uint64_t i = 0; i < n; ++i)
        present[i] = rl::visited_insert(table, H, *count, hashes[i]) ? 1 : 0;
}

// rl::visited_mask (include/mymyr/rl/visited.hpp:63-74).
void mref_visited_mask(const uint64_t* table, const int32_t* count, uint32_t H, const uint64_t* succ_hash, const int32_t* parent,
                       const int32_t* rows, uint64_t size, uint8_t* out)
{
    rl::visited_mask(table, count, H, succ_hash, parent, rows, size, out);
}

// rl::rng::instance_draw (include/mymyr/rl/rng.hpp:94-115)
int32_t mref_instance_draw(uint64_t seed, uint64_t env, uint32_t reset_count, uint32_t instances, const uint32_t* thresholds,
                           const int32_t* indices, uint32_t m)
{
    return rl::rng::instance_draw(seed, env, reset_count, instances, thresholds, indices, m);
}

// The CPU env pool (CpuEnvPool, `threads` workers) over `num_envs` envs: reset, then `steps` random-policy steps of
// every env. seconds: wall time of the steps only. checksum: hash of the final pool states, rewards and counts.
int mref_pool_run(mref_task* t, const mref_env_config* c, uint32_t num_envs, uint32_t threads, uint32_t steps,
                  double* seconds, uint64_t* checksum)
{
    return guarded(
        [&]() -> int
        {
            rl::PoolOptions po;
            po.threads = threads;
            rl::CpuEnvPool pool(t->table, env_config(c), num_envs, po);
            rl::PoolBatch b = pool.reset(nullptr, 0, nullptr);
            pool.recycle(std::move(b));
            u64 h = 0;
            const auto t0 = std::chrono::steady_clock::now();
            for (u32 k = 0; k < steps; ++k)
            {
                rl::PoolBatch r = pool.step(nullptr, 0, rl::Actions{}, nullptr);
                if (k + 1 == steps)
                {
                    h = hash::words(r.states.data(), static_cast<u32>(r.states.size()));
                    h = hash::combine(h, hash::words(reinterpret_cast<const u64*>(r.count.data()), static_cast<u32>(r.count.size() / 2)));
                }
                pool.recycle(std::move(r));
            }
            *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            *checksum = h;
            return 0;
        },
        -1);
}

// BrFS over the task; layer_counts [cap, 3] receives {expanded, generated, new} per expanded layer.
// plan_schema [plan_cap], plan_binding [plan_cap, binding_width], goal_state [goal_cap] (all optional): the plan's
// actions as (schema, objects padded with -1) and the goal state's words.
int mref_brfs(mref_task* t, const mref_brfs_options* o, mref_brfs_result* r, uint64_t* layer_counts, uint32_t cap,
              int32_t* plan_schema, int32_t* plan_binding, uint32_t binding_width, uint32_t plan_cap, uint64_t* goal_state,
              uint32_t goal_cap)
{
    return guarded(
        [&]() -> int
        {
            BrfsOptions b;
            b.threads = o->threads;
            b.max_depth = o->max_depth;
            b.max_states = o->max_states;
            b.max_expanded = o->max_expanded;
            b.witness_pruning = o->witness_pruning != 0;
            if (o->start)
                b.start = State(std::span<const u64>(o->start, o->words));
            for (uint64_t k = 0; k < o->blocked_count; ++k)
                b.blocked_states.push_back(State(std::span<const u64>(o->blocked + k * o->words, o->words)));
            b.max_seconds = o->max_seconds;
            if (o->goal_kind == 1)
            {
                std::vector<GroundCondition> conds(o->goal_count);
                const formalism::TaskData& td = t->task->data();
                for (u32 k = 0; k < o->goal_count; ++k)
                    for (u32 l = o->goal_offsets[k]; l < o->goal_offsets[k + 1]; ++l)
                    {
                        const int32_t* rec = o->goal_literals + static_cast<usize>(l) * 8;
                        GroundLiteral gl;
                        gl.atom.predicate = PredicateId{static_cast<u32>(rec[0])};
                        gl.positive = rec[1] != 0;
                        const u32 ar = td.predicates.at(static_cast<u32>(rec[0])).arity;
                        for (u32 i = 0; i < ar; ++i)
                            gl.atom.objects.push_back(ObjectId{static_cast<u32>(rec[2 + i])});
                        conds[k].literals.push_back(std::move(gl));
                    }
                b.goal = search::any_of(*t->task, conds);
            }
            else if (o->goal_kind == 2)
            {
                b.goal.kind = search::GoalSpec::Kind::Custom;
                const uint64_t m = o->goal_mod, res = o->goal_res;
                b.goal.test = [m, res](StateView s) { return s.hash() % m == res; };
            }
            else if (o->goal_kind == 3)
            {
                // a custom test that no slot numbering changes: the number of true atoms is goal_res
                b.goal.kind = search::GoalSpec::Kind::Custom;
                const uint64_t k = o->goal_res;
                b.goal.test = [k](StateView s) { return s.count() == k; };
            }
            b.canonical_order = o->canonical_order != 0;
            b.stop_at_goal = o->stop_at_goal != 0;
            b.fingerprint = o->fingerprint != 0;
            b.layer_stats = true;
            b.layers.kind = static_cast<search::LayerOrdering::Kind>(o->layer_kind);
            b.layers.seed = o->layer_seed;
            if (o->max_next_layer_states)
                b.layers.max_next_layer_states = o->max_next_layer_states;
            if (o->beam_width)
                b.layers.beam_width = o->beam_width;
            b.layers.prefer_more_satisfied_goals = o->prefer_fewer == 0;
            b.layers.randomize_ties = o->randomize_ties != 0;
            if (o->scorer)
            {
                // the views' rows padded to a common width for the callback
                auto fn = o->scorer;
                void* user = o->scorer_user;
                b.layers.scorer = [fn, user](std::span<const StateView> states, std::span<f64> scores)
                {
                    u32 w = 1;
                    for (const StateView& v : states)
                        w = std::max(w, v.nw);
                    std::vector<u64> rows(states.size() * w, 0);
                    for (usize i = 0; i < states.size(); ++i)
                        std::copy(states[i].w, states[i].w + states[i].nw, rows.begin() + static_cast<std::ptrdiff_t>(i * w));
                    fn(user, rows.data(), states.size(), w, scores.data());
                };
            }
            EventLog log;
            if (o->record_events)
            {
                b.observer = &log;
                b.progress_interval = ~u64{0};
            }
            const auto t0 = std::chrono::steady_clock::now();
            const BrfsResult x = brfs(*t->task, b);
            g_events = std::move(log.ev);
            r->seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            r->states = x.states;
            r->expanded = x.expanded;
            r->generated = x.generated;
            r->goal_states = x.num_goal_states;
            r->fingerprint = x.fingerprint;
            r->layers = x.layers;
            r->status = static_cast<int32_t>(x.status);
            r->solved = x.solved;
            r->exhausted = x.exhausted;
            r->cost = x.cost;
            r->pruned = x.pruned;
            r->words = x.words;
            r->fluent_slots = x.fluent_slots;
            r->threads_used = x.threads_used;
            std::snprintf(r->store, sizeof(r->store), "%s", x.store.c_str());
            std::snprintf(r->message, sizeof(r->message), "%s", x.message.c_str());
            r->plan_len = static_cast<uint32_t>(x.plan.size());
            for (u32 i = 0; i < x.plan.size() && i < plan_cap; ++i)
            {
                const Action& a = x.plan[i];
                if (plan_schema)
                    plan_schema[i] = static_cast<int32_t>(a.schema.v);
                if (plan_binding)
                    for (u32 k = 0; k < binding_width; ++k)
                        plan_binding[static_cast<usize>(i) * binding_width + k] =
                            k < a.binding.size() ? static_cast<int32_t>(a.binding[k].v) : -1;
            }
            r->goal_words = 0;
            if (x.goal_state)
            {
                const StateView g = x.goal_state->view();
                r->goal_words = g.nw;
                for (u32 w = 0; w < g.nw && w < goal_cap && goal_state; ++w)
                    goal_state[w] = g.w[w];
            }
            for (u32 i = 0; i < x.layer_counts.size() && i < cap; ++i)
                for (u32 j = 0; j < 3; ++j)
                    layer_counts[i * 3 + j] = x.layer_counts[i][j];
            return static_cast<int>(x.layer_counts.size());
        },
        -1);
}


// Inserts rows [n, words] into the reference's FlatStateStore (single-threaded, grown at 70% load); unique = states
// stored. seconds: the inserts alone.
int mref_dedup_flat(const uint64_t* rows, uint64_t n, uint32_t words, uint64_t* unique, double* seconds)
{
    return guarded(
        [&]() -> int
        {
            FlatStateStore store(words, 16);
            const auto t0 = std::chrono::steady_clock::now();
            for (uint64_t i = 0; i < n; ++i)
                store.insert(rows + i * words, words);
            *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            *unique = store.size();
            return 0;
        },
        -1);
}

// Inserts rows [n, words] into the reference's ConcurrentStateStore on `threads` threads, in batches of `batch` rows
// (each thread a contiguous slice of the batch; the store's stop-the-world rehash between batches when it asks for
// one, and inside a batch a thread stops at the request until the batch ends and the rehash ran). unique = states
// stored; seconds: the inserts and rehashes.
int mref_dedup_concurrent(const uint64_t* rows, uint64_t n, uint32_t words, uint32_t threads, uint64_t batch,
                          uint64_t* unique, double* seconds)
{
    return guarded(
        [&]() -> int
        {
            Team team(threads);
            const u32 T = team.size();
            ConcurrentStateStore store(T);
            std::vector<uint64_t> next(T);
            std::atomic<uint64_t> stored{0};
            const auto t0 = std::chrono::steady_clock::now();
            for (uint64_t b0 = 0; b0 < n; b0 += batch)
            {
                const uint64_t b1 = std::min(n, b0 + batch);
                for (u32 t = 0; t < T; ++t)
                    next[t] = b0 + (b1 - b0) * t / T;
                for (;;)
                {
                    team.run(
                        [&](u32 t)
                        {
                            const uint64_t end = b0 + (b1 - b0) * (t + 1) / T;
                            uint64_t i = next[t], added = 0;
                            for (; i < end && !store.wants_rehash(); ++i)
                                added += store.insert(t, rows + i * words, words, i).second ? 1 : 0;
                            next[t] = i;
                            stored.fetch_add(added, std::memory_order_relaxed);
                        });
                    bool done = true;
                    for (u32 t = 0; t < T; ++t)
                        done = done && next[t] >= b0 + (b1 - b0) * (t + 1) / T;
                    if (store.wants_rehash())
                        store.rehash(team);
                    if (done)
                        break;
                }
            }
            *seconds = std::chrono::duration<double>(std::chrono::steady_clock::now() - t0).count();
            *unique = stored.load();
            return 0;
        },
        -1);
}


// ---- the reference pool's asynchronous API over a scripted sequence of calls (CpuEnvPool, rl/pool.hpp:114-172)

struct mref_pool
{
    std::unique_ptr<rl::CpuEnvPool> pool;
};

// A PoolBatch's arrays copied out (caller-owned, `cap` rows; null arrays are not written): env ids, states [rows, words]
// (zero padded), instances, counts, step counts, and for a step's batch the rewards, flags, final states and labels.
struct mref_pool_out
{
    uint64_t cap;
    uint32_t words, label_width;
    uint32_t* env_ids;
    uint64_t* states;
    int32_t* task_ids;
    int32_t* count;
    int32_t* steps;
    uint8_t* at_goal;
    uint8_t* terminated;
    uint8_t* goal;
    float* reward;
    uint8_t* truncated;
    uint8_t* invalid;
    uint64_t* final_states;
    int32_t* schema;
    int32_t* binding;
};

static int64_t copy_pool_batch(const rl::PoolBatch& b, mref_pool_out* o)
{
    if (b.rows > o->cap)
        throw std::invalid_argument("harness: pool batch of " + std::to_string(b.rows) + " rows, buffers hold " + std::to_string(o->cap));
    const u32 BW = b.row_words(), OW = o->words;
    for (u64 r = 0; r < b.rows; ++r)
    {
        if (o->env_ids)
            o->env_ids[r] = b.env_ids[r];
        if (o->task_ids)
            o->task_ids[r] = b.task_ids[r];
        if (o->count)
            o->count[r] = b.count[r];
        if (o->steps)
            o->steps[r] = b.steps[r];
        if (o->at_goal)
            o->at_goal[r] = b.at_goal[r];
        if (o->terminated)
            o->terminated[r] = b.terminated[r];
        if (o->goal)
            o->goal[r] = b.goal[r];
        for (u32 w = 0; w < OW && o->states; ++w)
            o->states[r * OW + w] = w < BW ? b.states[r * BW + w] : 0;
        if (!b.step)
            continue;
        if (o->reward)
            o->reward[r] = b.reward[r];
        if (o->truncated)
            o->truncated[r] = b.truncated[r];
        if (o->invalid)
            o->invalid[r] = b.invalid[r];
        if (o->schema)
            o->schema[r] = b.schema[r];
        for (u32 w = 0; w < OW && o->final_states; ++w)
            o->final_states[r * OW + w] = w < BW ? b.final_states[r * BW + w] : 0;
        for (u32 k = 0; k < o->label_width && o->binding; ++k)
            o->binding[r * o->label_width + k] = k < b.label_width ? b.binding[r * b.label_width + k] : -1;
    }
    return static_cast<int64_t>(b.rows);
}

mref_pool* mref_pool_create(mref_task* t, const mref_env_config* c, uint32_t num_envs, uint32_t threads, uint64_t first_env)
{
    return guarded(
        [&]() -> mref_pool*
        {
            rl::PoolOptions po;
            po.threads = threads;
            po.first_env = first_env;
            auto p = new mref_pool;
            p->pool = std::make_unique<rl::CpuEnvPool>(t->table, env_config(c), num_envs, po);
            return p;
        },
        nullptr);
}

void mref_pool_free(mref_pool* p) { delete p; }

// env_ids [n] (null: every env). Returns the rows of the reset's batch.
int64_t mref_pool_reset(mref_pool* p, const uint32_t* env_ids, uint64_t n, mref_pool_out* o)
{
    return guarded([&]() -> int64_t { return copy_pool_batch(p->pool->reset(env_ids, n, nullptr), o); }, -1);
}

// env_ids [n] (null: every env), actions [n] (null: the random policy). Returns the send's ticket.
int64_t mref_pool_send(mref_pool* p, const uint32_t* env_ids, uint64_t n, const int64_t* actions)
{
    return guarded(
        [&]() -> int64_t
        {
            rl::Actions a;
            a.v64 = actions;
            return static_cast<int64_t>(p->pool->send(env_ids, n, a, nullptr));
        },
        -1);
}

int64_t mref_pool_recv(mref_pool* p, uint64_t min_rows, mref_pool_out* o)
{
    return guarded([&]() -> int64_t { return copy_pool_batch(p->pool->recv(min_rows), o); }, -1);
}

int64_t mref_pool_recv_ticket(mref_pool* p, uint64_t ticket, mref_pool_out* o)
{
    return guarded([&]() -> int64_t { return copy_pool_batch(p->pool->recv_ticket(ticket), o); }, -1);
}

int64_t mref_pool_pending(mref_pool* p)
{
    return guarded([&]() -> int64_t { return static_cast<int64_t>(p->pool->pending()); }, -1);
}

}  // extern "C"
