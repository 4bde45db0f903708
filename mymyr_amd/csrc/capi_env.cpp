// C ABI of the device environment and the successor listing (include/mymyr_amd.h, "env" section). Argument checks
// follow the reference's check_env / check_step messages (src/mymyr/rl/env.cpp:102-135, 403-421).

#include "../../include/mymyr_amd.h"

#include "capi_internal.hpp"
#include "env.hpp"
#include "runtime.hpp"
#include "scan.hpp"
#include "state_set.hpp"

#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

using namespace mya;

/// One instance of an env's table: its task, tables and initial-state facts (host copies).
struct EnvInstance
{
    mya_task* task = nullptr;
    TaskDev T{};
    u32 init_count = 0;
    u32 init_goal = 0;
    u32 variant = 0;
};

struct mya_env
{
    std::vector<EnvInstance> inst;
    EnvCfg cfg{};
    u32 words = 1;        // the widest instance's words
    u32 label_width = 0;  // the largest schema arity
    u32 num_schemas = 0;  // the most schemas of any instance (columns of masks; the count cache has 2 more)
    InstDev* d_inst = nullptr;    // device [instances]
    TaskDev* d_tasks = nullptr;   // device [instances]
    u64* d_init = nullptr;        // device: per instance its goal masks (positive, then negative) over its words
    u32* d_init_cache = nullptr;  // device [instances, num_schemas + 2]: the initial states' count-cache rows
    u8* d_init_masks = nullptr;   // device [instances, max(1, num_schemas)]
    u32* d_status = nullptr;
    u32* h_status = nullptr;
    u64* d_seed = nullptr;        // device word: the RNG key of the random policy and of the sampler
    SamplerDev sampler{};          // the instance sampler (instances 0: off)
    u32* d_thresholds = nullptr;   // device [m - 1]
    i32* d_indices = nullptr;      // device [m]
    // grouped launches: per variant present, its block shape
    struct Launch
    {
        u32 variant;
        unsigned nw;
        size_t lds;
        u32 wave_words;
    };
    std::vector<Launch> launches;
    // the row groups of the last grouped call (device scratch, grown to the largest batch)
    u64 group_rows = 0;
    u32* d_hist = nullptr;   // [instances + 1]
    u32* d_starts = nullptr;  // [instances + 1]
    u32* d_chunks = nullptr;  // [instances + 1]
    u32* d_order = nullptr;   // [group_rows]
    u64 sampled_rows = 0;
    i32* d_sampled = nullptr;  // [sampled_rows]: the sampled next instances of a step
    std::mutex mutex;         // guards the scratch growth

    [[nodiscard]] u32 instances() const { return static_cast<u32>(inst.size()); }
    [[nodiscard]] const TaskDev& T0() const { return inst[0].T; }
    [[nodiscard]] u32 cache_width() const { return num_schemas + 2; }
};

namespace
{
void check_batch(const mya_env* e, const mya_env_batch* b)
{
    if (!b)
        throw std::invalid_argument("mymyr_amd: env: null batch");
    if (b->rows && !b->states)
        throw std::invalid_argument("mymyr: env: null state array");
    if (b->rows > 0x7FFFFFFFull)
        throw std::invalid_argument("mymyr: env: more than 2^31 - 1 environments in one batch");
    if (b->words < e->words)
        throw std::invalid_argument("mymyr: env: state rows of " + std::to_string(b->words) + " words; the " +
                                    (e->instances() > 1 ? "table" : "task") + " needs " + std::to_string(e->words) +
                                    " (its widest instance's words)");
    if ((b->goal_pos == nullptr) != (b->goal_neg == nullptr))
        throw std::invalid_argument("mymyr: env: per-env goals need both goal_pos and goal_neg");
    if (b->goal_pos)
        for (u32 i = 0; i < e->instances(); ++i)
            if (e->inst[i].T.goal_unsat)
                throw std::invalid_argument("mymyr: env: per-env goal masks cannot express the goal of instance " + std::to_string(i) +
                                            " (it is statically unsatisfiable); use the instances' goal tests (no goal masks)");
    if (b->visited)
    {
        const u32 H = b->visited_capacity;
        if (H < 2 || H > (1u << 20) || (H & (H - 1)))
            throw std::invalid_argument("mymyr: env: visited capacity must be a power of two in [2, 2^20]");
        if (b->rows && (!b->visited_count || !b->visited_status))
            throw std::invalid_argument("mymyr: env: visited tracking needs table, count and status arrays");
    }
    if (!b->task_ids && b->rows && e->instances() > 1)
        throw std::invalid_argument("mymyr: env: a batch over a table of " + std::to_string(e->instances()) +
                                    " instances needs task ids");
}

/// The batch's visited tables as the kernels take them (capacity 0: none).
VisitedDev visited_of(const mya_env_batch* b)
{
    if (!b->visited)
        return VisitedDev{};
    return VisitedDev{b->visited, b->visited_count, b->visited_status, b->visited_capacity, b->visited_status_per_row ? 1u : 0u};
}

/// Whether a call runs grouped by instance: over several instances (a one-instance batch runs in batch order, checking
/// its task ids on the way).
bool grouped(const mya_env* e) { return e->instances() > 1; }

/// The env's per-row scratch array `member` (of `have` rows), grown under the env's lock to `rows` (a call with a batch
/// no larger than before allocates nothing).
template<class X>
X* scratch_rows(mya_env* e, u64 rows, X* mya_env::*member, u64 mya_env::*have)
{
    std::lock_guard lock(e->mutex);
    if (rows > e->*have)
    {
        dev_free(e->*member);
        e->*member = nullptr;
        e->*have = 0;
        e->*member = dev_alloc<X>(rows, "env row scratch");
        e->*have = rows;
    }
    return e->*member;
}

/// Groups the batch's rows by instance into the env's scratch (grown under the env's lock; a call with a batch no
/// larger than before allocates nothing).
RowGroups group_rows(mya_env* e, const mya_env_batch* b, hipStream_t stream, u32* status = nullptr)
{
    scratch_rows(e, b->rows, &mya_env::d_order, &mya_env::group_rows);
    launch_group_rows(b->task_ids, b->rows, e->instances(), e->d_hist, e->d_order, e->d_starts, e->d_chunks, status ? status : e->d_status,
                      stream);
    return RowGroups{e->d_order, e->d_starts, e->d_chunks};
}

/// The table's domain check (TaskTable::domain_mismatch, src/mymyr/rl/task_table.cpp:75-100): empty if `t` has the
/// action schemas (names, arities) and predicates (names, arities, kinds) of `r` in the same order.
std::string domain_mismatch(const TaskText& r, const TaskText& t)
{
    if (t.schemas.size() != r.schemas.size())
        return std::to_string(t.schemas.size()) + " action schemas, instance 0 has " + std::to_string(r.schemas.size());
    for (size_t s = 0; s < t.schemas.size(); ++s)
        if (t.schemas[s].name != r.schemas[s].name || t.schemas[s].arity != r.schemas[s].arity)
            return "action schema " + std::to_string(s) + " is " + t.schemas[s].name + "/" + std::to_string(t.schemas[s].arity) +
                   ", instance 0 has " + r.schemas[s].name + "/" + std::to_string(r.schemas[s].arity);
    auto kind = [](char k) { return std::string(k == 'S' ? "static" : k == 'F' ? "fluent" : "derived"); };
    for (size_t d = 0; d < t.preds.size(); ++d)
        if (d >= r.preds.size() || r.preds[d].name != t.preds[d].name || r.preds[d].arity != t.preds[d].arity ||
            r.preds[d].kind != t.preds[d].kind)
            return "domain predicate " + std::to_string(d) + " is " + t.preds[d].name + "/" + std::to_string(t.preds[d].arity) + " (" +
                   kind(t.preds[d].kind) + "), instance 0 has " +
                   (d < r.preds.size() ? r.preds[d].name + "/" + std::to_string(r.preds[d].arity) + " (" + kind(r.preds[d].kind) + ")"
                                       : std::string("no more"));
    if (t.preds.size() != r.preds.size())
        return std::to_string(t.preds.size()) + " domain predicates, instance 0 has " + std::to_string(r.preds.size());
    return {};
}

/// A count over the batch's rows (refresh, goal): in batch order over one instance, else grouped by instance.
void run_count(mya_env* env, const mya_env_batch* batch, CountArgs& a, hipStream_t s)
{
    a.T = env->T0();
    a.tasks = env->d_tasks;
    a.inst = env->d_inst;
    a.instances = env->instances();
    a.states = batch->states;
    a.rows = batch->rows;
    a.words = batch->words;
    a.task_ids = batch->task_ids;
    a.goal_pos = batch->goal_pos;
    a.goal_neg = batch->goal_neg;
    a.status = env->d_status;
    a.cache_width = env->cache_width();
    a.mask_width = env->num_schemas;
    if (!grouped(env))
    {
        launch_env_count(a, s);
        return;
    }
    a.groups = group_rows(env, batch, s);
    if (env->instances() <= kPerInstanceLaunches)
        for (u32 k = 0; k < env->instances(); ++k)
        {
            a.T = env->inst[k].T;
            a.instance = k;
            launch_env_count(a, s);
        }
    else
        for (const mya_env::Launch& l : env->launches)
        {
            a.wave_words = l.wave_words;
            launch_env_count_grouped(a, l.variant, l.nw, l.lds, s);
        }
}

void free_env(mya_env* e)
{
    for (void* p : std::initializer_list<void*>{e->d_status, e->d_inst, e->d_tasks, e->d_init, e->d_init_cache, e->d_init_masks, e->d_hist,
                                                e->d_starts, e->d_chunks, e->d_order, e->d_thresholds, e->d_indices,
                                                e->d_sampled, e->d_seed})
        dev_free(p);
    if (e->h_status)
        (void)hipHostFree(e->h_status);
    delete e;
}
}  // namespace

namespace mya
{
/// Carves the scratch of an expansion of n rows from a block of at least expand_scratch_bytes(n) bytes (256-aligned).
ExpandScratch carve_expand_scratch(void* block, u64 n)
{
    unsigned char* p = static_cast<unsigned char*>(block);
    auto next = [&]<class T>(size_t count) {
        T* q = reinterpret_cast<T*>(p);
        p += scratch_bytes<T>(count);
        return q;
    };
    ExpandScratch x{};
    x.counts = next.operator()<u32>(n);
    x.noops = next.operator()<u32>(n);
    x.kept = next.operator()<u32>(n);
    x.pre = next.operator()<u64>(n + 1);
    x.fin = next.operator()<u64>(n + 1);
    x.scan = next.operator()<u64>(scan_scratch_words(n));
    x.words_status = next.operator()<u32>(2);
    return x;
}

/// The flat expansion of rows over instances `inst` (one: batch order; several: grouped by instance with `env`'s
/// scratch and the rows' task ids). `block` (device, at least expand_scratch_bytes(max(rows, 1)) bytes) holds the
/// expansion's scratch; the call synchronizes the stream before it returns, so the block is free again then.
void expand_rows(const std::vector<const TaskDev*>& inst, mya_env* env, const int32_t* task_ids, const uint64_t* states, uint64_t rows,
                 uint32_t words, const mya_expand_options* options, mya_expansion* out, hipStream_t stream, void* block, mya_task* lazy)
{
    {
        if (!options || !out || (rows && !states))
            throw std::invalid_argument("mymyr_amd: expand: null argument");
        if (!options->canonical_order)
            throw std::invalid_argument("mymyr_amd: expand: the device expansion takes canonical_order on");
        if (options->witness_pruning && inst.size() > 1)
            throw std::invalid_argument("mymyr_amd: expand: the device expansion over a task table takes witness_pruning off");
        TaskDev T = *inst[0];  // the widest instance's words and label width stand for the table in the checks
        for (const TaskDev* t : inst)
        {
            T.W = std::max(T.W, t->W);
            T.label_width = std::max(T.label_width, t->label_width);
        }
        constexpr u64 kMaxRows = (u64{1} << 31) - 1;
        if (rows > kMaxRows)
            throw std::invalid_argument("mymyr: expand: more than 2^31 - 1 states in one batch");
        // lazy slots: rows narrower than the task's current width hold no atom past them (src/mymyr/rl/expand.cpp:53)
        if (words < T.W && !lazy)
            throw std::invalid_argument("mymyr: expand: state rows of " + std::to_string(words) + " words; the task needs " +
                                        std::to_string(T.W));
        if (out->binding && out->label_width < T.label_width)
            throw std::invalid_argument("mymyr: expand: label width " + std::to_string(out->label_width) +
                                        " is below the largest schema arity " + std::to_string(T.label_width));
        if (out->capacity > kMaxRows)
            throw std::invalid_argument("mymyr: expand: capacity above 2^31 - 1 rows");
        if (out->succ && out->words == 0 && out->capacity)
            throw std::invalid_argument("mymyr: expand: successor rows of zero words");
        if (out->goal && !out->succ)
            throw std::invalid_argument("mymyr: expand: goal flags need the successor rows");
        if (options->drop_noops && out->capacity && !out->index)
            throw std::invalid_argument("mymyr: expand: drop_noops requires index");
        out->generated = out->total = 0;
        out->words_needed = 0;
        const u64 n = std::max<u64>(rows, 1);
        const ExpandScratch x = carve_expand_scratch(block, n);
        u32* const counts = x.counts;
        u32* const noops = x.noops;
        u32* const kept = x.kept;
        u64* const pre = x.pre;
        u64* const fin = x.fin;
        u64* const scratch = x.scan;
        u32* const words_status = x.words_status;
        launch_fill_u32(words_status, 2, 0, stream);
        ExpandArgs a{};
        a.T = *inst[0];
        a.witness = options->witness_pruning && a.T.witness ? 1 : 0;
        if (inst.size() > 1)
        {
            mya_env_batch b{};
            b.states = const_cast<uint64_t*>(states);
            b.rows = rows;
            b.words = words;
            b.task_ids = const_cast<int32_t*>(task_ids);
            a.groups = group_rows(env, &b, stream, words_status + 1);
        }
        // one launch over the batch, or one per instance over its group
        auto launch = [&](ExpandArgs& x) {
            if (!x.groups.order)
            {
                launch_expand(x, stream);
                return;
            }
            for (u32 k = 0; k < inst.size(); ++k)
            {
                x.T = *inst[k];
                x.instance = k;
                launch_expand(x, stream);
            }
        };
        a.states = states;
        a.rows = rows;
        a.words = words;
        a.drop_noops = options->drop_noops ? 1 : 0;
        a.out_words = out->words;
        a.label_width = out->label_width;
        a.counts = counts;
        a.noops = noops;
        a.words_needed = words_status;
        a.status = words_status + 1;
        a.pass = 0;
        launch(a);
        launch_exclusive_scan(counts, pre, rows, scratch, pre + rows, stream);
        if (a.drop_noops)
        {
            launch_kept_counts(counts, noops, rows, kept, stream);
            launch_exclusive_scan(kept, fin, rows, scratch, fin + rows, stream);
        }
        u64 totals[2] = {0, 0};
        u32 st[2] = {0, 0};
        hip_check(hipMemcpyAsync(&totals[0], pre + rows, sizeof(u64), hipMemcpyDeviceToHost, stream), "expand total");
        if (a.drop_noops)
            hip_check(hipMemcpyAsync(&totals[1], fin + rows, sizeof(u64), hipMemcpyDeviceToHost, stream), "expand total");
        hip_check(hipMemcpyAsync(st, words_status, sizeof(st), hipMemcpyDeviceToHost, stream), "expand status");
        hip_check(hipStreamSynchronize(stream), "expand");
        if (options->validate && (st[1] & kStatusWideRow))
            throw std::invalid_argument("mymyr: expand: a state has atoms past the task's slots");
        if (st[1] & kStatusTaskId)
            throw std::invalid_argument("mymyr: expand: a task id is outside the table's " + std::to_string(inst.size()) + " instances");
        if (st[1] & ~kStatusWideRow)
            throw std::runtime_error("mymyr_amd: expand: device status " + std::to_string(st[1]));
        const u64 generated = totals[0];
        if (generated > kMaxRows)
            throw std::invalid_argument("mymyr: expand: more than 2^31 - 1 successors in one batch");
        // an overflow with drop_noops reports the counts before dropping
        const bool dropping = a.drop_noops && generated <= out->capacity;
        const u64* offs = dropping ? fin : pre;
        out->generated = generated;
        out->total = dropping ? totals[1] : generated;
        if (out->offsets)
            launch_offsets_i32(offs, rows + 1, out->offsets, stream);
        const bool rows_out = out->succ || out->parent || out->schema || out->binding || out->goal || out->succ_hash || out->noop ||
                              out->index;
        if ((rows_out && out->capacity) || (out->succ && out->words < T.W))
        {
            a.pass = 1;
            a.drop_noops = dropping ? 1 : 0;
            a.offsets = offs;
            a.capacity = out->capacity;
            a.succ = out->succ;
            a.parent = out->parent;
            a.schema = out->schema;
            a.binding = out->binding;
            a.goal = out->goal;
            a.succ_hash = out->succ_hash;
            a.noop = out->noop;
            a.index = out->index;
            launch(a);
        }
        hip_check(hipMemcpyAsync(st, words_status, sizeof(st), hipMemcpyDeviceToHost, stream), "expand status");
        hip_check(hipStreamSynchronize(stream), "expand");
        // lazy slots: successors that added atoms without a slot are written again once those atoms are interned
        // (ascending canonical id; a row past `words` then counts in words_needed)
        while (lazy && (st[1] & kStatusNoSlot))
        {
            if (!resolve_missing(lazy, stream))
                throw std::logic_error("mymyr_amd: expand: an added atom without a slot was not recorded");
            a.T = *device_task(lazy).thost;
            launch_fill_u32(words_status, 2, 0, stream);
            launch(a);
            hip_check(hipMemcpyAsync(st, words_status, sizeof(st), hipMemcpyDeviceToHost, stream), "expand status");
            hip_check(hipStreamSynchronize(stream), "expand");
        }
        if (st[1] & ~kStatusWideRow)
            throw std::runtime_error("mymyr_amd: expand: device status " + std::to_string(st[1]));
        out->words_needed = st[0];
    }
}
}  // namespace mya

namespace
{
/// An env over `count` instances; one_domain: a task table (TaskTable::create's domain check), else a suite of several
/// domains (TaskSuite::group: global ids in the tasks' order, each domain's labels its own).
void create_env(mya_task* const* tasks, uint32_t count, const mya_env_config* config, mya_env** out, bool one_domain)
{
    {
        if (!tasks || !config || !out)
            throw std::invalid_argument("mymyr_amd: env_create: null argument");
        if (count == 0)
            throw std::invalid_argument("mymyr: TaskTable: no instances");
        if (count > kMaxInstances)
            throw std::invalid_argument("mymyr_amd: env: the device env takes at most " + std::to_string(kMaxInstances) + " instances");
        for (u32 i = 0; i < count; ++i)
            if (!tasks[i])
                throw std::invalid_argument("mymyr: TaskTable: instance " + std::to_string(i) + " is null");
            else if (lazy_task(tasks[i]))
                // the reference's table refusal (src/mymyr/rl/task_table.cpp:120-123)
                throw std::invalid_argument("mymyr: TaskTable: instance " + std::to_string(i) +
                                            " has lazy atom slots, numbered in the order searches meet its atoms; the rows of a table "
                                            "need a fixed slot layout (atoms 'auto', 'reachable' or 'dense')");
        for (u32 i = 1; one_domain && i < count; ++i)
        {
            const std::string why = domain_mismatch(tasks[0]->compiled->text, tasks[i]->compiled->text);
            if (!why.empty())
                throw std::invalid_argument("mymyr: TaskTable: instance " + std::to_string(i) + " is not of the domain of instance 0: " + why);
        }
        if (!config->canonical_order || config->witness_pruning)
            throw std::invalid_argument("mymyr_amd: env: the device step takes canonical_order on and witness_pruning off");
        if (config->dead_end != 0 && config->dead_end != 1)
            throw std::invalid_argument("mymyr_amd: env: dead_end must be 0 (no_successors) or 1 (none)");
        std::unique_ptr<mya_env, void (*)(mya_env*)> e(new mya_env, free_env);
        e->cfg.max_steps = config->max_steps;
        e->cfg.step_reward = config->step_reward;
        e->cfg.goal_reward = config->goal_reward;
        e->cfg.dead_end_reward = config->dead_end_reward;
        e->cfg.dead_end_none = config->dead_end == 1 ? 1 : 0;
        e->cfg.dead_end_terminal = config->dead_end_terminal;
        e->cfg.autoreset = config->autoreset;
        e->inst.resize(count);
        for (u32 i = 0; i < count; ++i)
        {
            EnvInstance& in = e->inst[i];
            in.task = tasks[i];
            in.T = *device_task(tasks[i]).thost;
            in.variant = env_variant(in.T);
            e->words = std::max(e->words, in.T.W);
            e->label_width = std::max(e->label_width, in.T.label_width);
            e->num_schemas = std::max(e->num_schemas, in.T.num_schemas);
        }
        const u32 S = e->num_schemas, cw = e->cache_width();
        e->d_status = dev_alloc<u32>(1, "env status");
        e->d_seed = dev_alloc<u64>(1, "env seed");
        hip_check(hipMemcpy(e->d_seed, &config->seed, sizeof(u64), hipMemcpyHostToDevice), "env seed");
        hip_check(hipHostMalloc(reinterpret_cast<void**>(&e->h_status), sizeof(u32), hipHostMallocDefault), "pinned status");
        hip_check(hipMemset(e->d_status, 0, sizeof(u32)), "env status");
        // per instance: the goal as masks over its words; then the initial states' counts, goal flags, masks and
        // count-cache rows (one count launch per instance)
        std::vector<size_t> goal_at(count);
        std::vector<u64> gm;
        for (u32 i = 0; i < count; ++i)
        {
            const u32 W = e->inst[i].T.W;
            goal_at[i] = gm.size();
            gm.resize(gm.size() + 2 * static_cast<size_t>(W), 0);
            for (u32 sl : tasks[i]->compiled->goal_pos)
                gm[goal_at[i] + (sl >> 6)] |= u64{1} << (sl & 63);
            for (u32 sl : tasks[i]->compiled->goal_neg)
                gm[goal_at[i] + W + (sl >> 6)] |= u64{1} << (sl & 63);
        }
        e->d_init = dev_alloc<u64>(gm.size(), "goal masks");
        hip_check(hipMemcpy(e->d_init, gm.data(), gm.size() * sizeof(u64), hipMemcpyHostToDevice), "goal masks");
        e->d_init_masks = dev_alloc<u8>(static_cast<size_t>(count) * std::max<u32>(1, S), "initial masks");
        e->d_init_cache = dev_alloc<u32>(static_cast<size_t>(count) * cw, "initial count caches");
        std::vector<i32> hc(count);
        std::vector<u8> hg(count);
        {
            i32* cnt = dev_alloc<i32>(count, "initial counts");
            u8* gl = dev_alloc<u8>(count, "initial goals");
            for (u32 i = 0; i < count; ++i)
            {
                const TaskDev& T = e->inst[i].T;
                launch_env_count(T, T.initial, 1, T.W, cnt + i, gl + i, e->d_init_masks + static_cast<size_t>(i) * std::max<u32>(1, S),
                                 e->d_init_cache + static_cast<size_t>(i) * cw, nullptr, nullptr, nullptr, nullptr, i, S);
            }
            hip_check(hipMemcpy(hc.data(), cnt, count * sizeof(i32), hipMemcpyDeviceToHost), "initial counts");
            hip_check(hipMemcpy(hg.data(), gl, count * sizeof(u8), hipMemcpyDeviceToHost), "initial goals");
            // the synchronous copies above have drained the null stream: the blocks are free in its order
            dev_free_async(cnt, nullptr);
            dev_free_async(gl, nullptr);
        }
        std::vector<InstDev> hi(count);
        std::vector<TaskDev> ht(count);
        for (u32 i = 0; i < count; ++i)
        {
            EnvInstance& in = e->inst[i];
            in.init_count = static_cast<u32>(hc[i]);
            in.init_goal = hg[i];
            InstDev& d = hi[i];
            d.initial = in.T.initial;
            d.init_cache = e->d_init_cache + static_cast<size_t>(i) * cw;
            d.init_masks = e->d_init_masks + static_cast<size_t>(i) * std::max<u32>(1, S);
            d.goal_pos = e->d_init + goal_at[i];
            d.goal_neg = e->d_init + goal_at[i] + in.T.W;
            d.W = in.T.W;
            d.init_count = in.init_count;
            d.init_goal = in.init_goal;
            d.fluent_slots = in.T.fluent_slots;
            d.variant = in.variant;
            d.init_hash = hash_state(tasks[i]->compiled->initial.data(), in.T.W);
            ht[i] = in.T;
        }
        e->d_inst = dev_alloc<InstDev>(count, "env instances");
        hip_check(hipMemcpy(e->d_inst, hi.data(), count * sizeof(InstDev), hipMemcpyHostToDevice), "env instances");
        e->d_tasks = dev_alloc<TaskDev>(count, "env instance tables");
        hip_check(hipMemcpy(e->d_tasks, ht.data(), count * sizeof(TaskDev), hipMemcpyHostToDevice), "env instance tables");
        if (count > 1)
        {
            for (u32 v = 0; v < 4; ++v)
            {
                std::vector<const TaskDev*> of;
                for (const EnvInstance& in : e->inst)
                    if (in.variant == v)
                        of.push_back(&in.T);
                if (of.empty())
                    continue;
                mya_env::Launch l{v, 0, 0, 0};
                l.nw = grouped_shape(of.data(), static_cast<u32>(of.size()), &l.lds, &l.wave_words);
                e->launches.push_back(l);
            }
            e->d_hist = dev_alloc<u32>(count + 1, "env group counters");
            e->d_starts = dev_alloc<u32>(count + 1, "env group starts");
            e->d_chunks = dev_alloc<u32>(count + 1, "env group chunks");
        }
        *out = e.release();
    }
}
}  // namespace

extern "C" {


int mya_env_create_table(mya_task* const* tasks, uint32_t count, const mya_env_config* config, mya_env** out)
{
    return guarded([&] { create_env(tasks, count, config, out, true); });
}

int mya_env_create_suite(mya_task* const* tasks, uint32_t count, const mya_env_config* config, mya_env** out)
{
    return guarded([&] { create_env(tasks, count, config, out, false); });
}

int mya_env_create(mya_task* task, const mya_env_config* config, mya_env** out)
{
    if (!task)
        return guarded([] { throw std::invalid_argument("mymyr_amd: env_create: null argument"); });
    return mya_env_create_table(&task, 1, config, out);
}

void mya_env_free(mya_env* env)
{
    if (env)
        free_env(env);
}

int mya_env_set_sampling(mya_env* env, uint32_t instances, const uint32_t* thresholds, const int32_t* indices, uint32_t m)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        if (instances == 0)
        {
            env->sampler = SamplerDev{};
            return;
        }
        // check_sampling (src/mymyr/rl/env.cpp:137-153)
        if (instances != env->instances())
            throw std::invalid_argument("mymyr: env: a sampler over " + std::to_string(instances) + " instances for " +
                                        std::to_string(env->instances()));
        if (m && (!thresholds || !indices))
            throw std::invalid_argument("mymyr: env: a weighted sampler needs one threshold fewer than indices");
        for (u32 k = 1; k + 1 < m; ++k)
            if (thresholds[k] < thresholds[k - 1])
                throw std::invalid_argument("mymyr: env: the sampler's thresholds are not ascending");
        for (u32 k = 0; k < m; ++k)
            if (indices[k] < 0 || static_cast<u32>(indices[k]) >= instances)
                throw std::invalid_argument("mymyr: env: the sampler's instance " + std::to_string(indices[k]) + " is outside the " +
                                            std::to_string(instances) + " instances");
        dev_free(env->d_thresholds);
        dev_free(env->d_indices);
        env->d_thresholds = nullptr;
        env->d_indices = nullptr;
        env->sampler = SamplerDev{};
        if (m)
        {
            env->d_thresholds = dev_alloc<u32>(std::max<u32>(1, m - 1), "sampler thresholds");
            env->d_indices = dev_alloc<i32>(m, "sampler indices");
            if (m > 1)
                hip_check(hipMemcpy(env->d_thresholds, thresholds, (m - 1) * sizeof(u32), hipMemcpyHostToDevice), "sampler thresholds");
            hip_check(hipMemcpy(env->d_indices, indices, m * sizeof(i32), hipMemcpyHostToDevice), "sampler indices");
        }
        env->sampler = SamplerDev{instances, m, env->d_thresholds, env->d_indices};
    });
}

int mya_env_initial_count(const mya_env* env, uint32_t instance, uint32_t* count, uint8_t* goal)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        if (instance >= env->instances())
            throw std::invalid_argument("mymyr: env: instance " + std::to_string(instance) + " is outside the table's " +
                                        std::to_string(env->instances()) + " instances");
        if (count)
            *count = env->inst[instance].init_count;
        if (goal)
            *goal = static_cast<uint8_t>(env->inst[instance].init_goal);
    });
}

int mya_env_reset(mya_env* env, const mya_env_batch* batch, const uint8_t* mask, int32_t* count, int keep_goals, int sample,
                  void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        check_batch(env, batch);
        if (sample && !env->sampler.instances)
            throw std::invalid_argument("mymyr: env: a sampling reset needs an instance sampler");
        if (sample && batch->rows && !batch->reset_counts)
            throw std::invalid_argument("mymyr: env: a sampling reset needs the reset counters");
        const auto s = static_cast<hipStream_t>(stream);
        launch_env_reset_draw(env->sampler, env->d_seed, batch->first_env, batch->rows, mask, sample != 0, batch->task_ids, batch->reset_counts,
                              batch->sampling_seeds, batch->env_ids, s);
        launch_env_reset(env->d_inst, env->instances(), batch->states, batch->rows, batch->words, mask, batch->task_ids, batch->steps,
                         batch->at_goal, count, batch->counts, env->cache_width(), env->d_status, s);
        if (batch->goal_pos)
            launch_env_reset_goals(env->d_inst, env->instances(), batch->rows, batch->words, mask, batch->task_ids, batch->goal_pos,
                                   batch->goal_neg, keep_goals != 0, batch->at_goal, env->d_status, s);
        launch_visited_restart(visited_of(batch), env->d_inst, env->instances(), batch->states, batch->rows, batch->words, mask,
                               batch->task_ids, false, s);
    });
}

namespace
{
/// The step of mya_env_step (actions: index actions, null: the random policy) and of mya_env_step_labels (labels).
void env_step(mya_env* env, const mya_env_batch* batch, const mya_step_outputs* out, const int64_t* actions, const int32_t* label_schema,
              const int32_t* label_binding, uint32_t label_stride, const int32_t* next_task_ids, void* stream)
{
    {
        if (!env || !out)
            throw std::invalid_argument("mymyr_amd: env: null argument");
        check_batch(env, batch);
        if (batch->rows && !batch->at_goal)
            throw std::invalid_argument("mymyr_amd: env: the device step needs the at_goal array");
        if (!actions && !label_schema && batch->rows && !batch->draws)
            throw std::invalid_argument("mymyr: env: the random policy needs the draw counters");
        if (env->cfg.max_steps && batch->rows && !batch->steps)
            throw std::invalid_argument("mymyr: env: truncation (max_steps) needs the step counters");
        if (next_task_ids && batch->rows && !batch->task_ids && env->cfg.autoreset)
            throw std::invalid_argument("mymyr_amd: env: next_task_ids needs the batch's task_ids (an autoreset writes the new instance)");
        if (out->binding && out->label_width < env->label_width)
            throw std::invalid_argument("mymyr: env: label width " + std::to_string(out->label_width) + " is below the largest schema arity " +
                                        std::to_string(env->label_width));
        const u32 fw = out->final_words ? out->final_words : batch->words;
        if (out->final_states && fw < env->words)
            throw std::invalid_argument("mymyr: env: final state rows of " + std::to_string(fw) + " words; the widest instance has " +
                                        std::to_string(env->words));
        if (out->atoms && out->max_atoms == 0)
            throw std::invalid_argument("mymyr_amd: env: atoms output needs max_atoms > 0");
        EnvArgs a{};
        a.T = env->T0();
        a.tasks = env->d_tasks;
        a.inst = env->d_inst;
        a.instances = env->instances();
        a.cfg = env->cfg;
        a.states = batch->states;
        a.rows = batch->rows;
        a.words = batch->words;
        a.task_ids = batch->task_ids;
        a.next_task_ids = next_task_ids;
        a.seed = env->d_seed;
        a.seeds = batch->seeds;
        a.env_ids = batch->env_ids;
        a.reset_counts = batch->reset_counts;
        a.steps = batch->steps;
        a.draws = batch->draws;
        a.at_goal = batch->at_goal;
        a.first_env = batch->first_env;
        a.actions = actions;
        a.label_schema = label_schema;
        a.label_binding = label_binding;
        a.label_stride = label_stride;
        a.reward = out->reward;
        a.terminated = out->terminated;
        a.truncated = out->truncated;
        a.count = out->count;
        a.final_states = out->final_states;
        a.final_words = fw;
        a.schema = out->schema;
        a.binding = out->binding;
        a.label_width = out->label_width;
        a.invalid = out->invalid;
        a.goal = out->goal;
        a.atoms = out->atoms;
        a.max_atoms = out->max_atoms;
        a.masks = out->masks;
        a.counts = batch->counts;
        a.cache_width = env->cache_width();
        a.mask_width = env->num_schemas;
        a.goal_pos = batch->goal_pos;
        a.goal_neg = batch->goal_neg;
        a.visited = visited_of(batch);
        a.revisited = out->revisited;
        a.status = env->d_status;
        const auto s = static_cast<hipStream_t>(stream);
        // without next_task_ids, rows restart in their next sampled instances when the env has a sampler and the batch
        // reset counters (drawn before the step, from the counters' values before its autoresets advance them)
        if (!next_task_ids && batch->reset_counts && env->sampler.instances && env->cfg.autoreset && batch->rows)
        {
            a.next_task_ids = scratch_rows(env, batch->rows, &mya_env::d_sampled, &mya_env::sampled_rows);
            launch_env_sample_next(env->sampler, env->d_seed, batch->first_env, batch->rows, batch->reset_counts, batch->sampling_seeds,
                                   batch->env_ids, const_cast<i32*>(a.next_task_ids), s);
        }
        if (!grouped(env))
        {
            // the batch-order step runs every row as instance 0: given ids are only checked
            launch_check_ids(batch->task_ids, batch->rows, 1, env->d_status, s);
            launch_check_ids(next_task_ids, batch->rows, 1, env->d_status, s);
            launch_env_step(a, s);
            return;
        }
        a.groups = group_rows(env, batch, s);
        if (env->instances() <= kPerInstanceLaunches)
            for (u32 k = 0; k < env->instances(); ++k)
            {
                a.T = env->inst[k].T;
                a.instance = k;
                launch_env_step(a, s);
            }
        else
            for (const mya_env::Launch& l : env->launches)
            {
                a.wave_words = l.wave_words;
                launch_env_step_grouped(a, l.variant, l.nw, l.lds, s);
            }
    }
}
}  // namespace

int mya_env_step(mya_env* env, const mya_env_batch* batch, const mya_step_outputs* out, const int64_t* actions,
                 const int32_t* next_task_ids, void* stream)
{
    return guarded([&] { env_step(env, batch, out, actions, nullptr, nullptr, 0, next_task_ids, stream); });
}

int mya_env_step_labels(mya_env* env, const mya_env_batch* batch, const mya_step_outputs* out, const int32_t* schema,
                        const int32_t* binding, uint32_t binding_stride, const int32_t* next_task_ids, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        if (batch && batch->rows && (!schema || (!binding && env->label_width)))
            throw std::invalid_argument("mymyr: label actions require schema and binding arrays");
        if (binding && binding_stride < env->label_width)
            throw std::invalid_argument("mymyr: label binding rows of " + std::to_string(binding_stride) + " columns; the largest schema arity is " +
                                        std::to_string(env->label_width));
        env_step(env, batch, out, nullptr, schema, binding, binding_stride, next_task_ids, stream);
    });
}

int mya_env_refresh(mya_env* env, const mya_env_batch* batch, int32_t* count, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        check_batch(env, batch);
        CountArgs a{};
        a.count = count;
        a.goal = batch->at_goal;
        a.cache = batch->counts;
        run_count(env, batch, a, static_cast<hipStream_t>(stream));
    });
}

int mya_env_reserve(mya_env* env, uint64_t rows)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        if (rows > 0x7FFFFFFFull)
            throw std::invalid_argument("mymyr: env: more than 2^31 - 1 environments in one batch");
        if (rows == 0)
            return;
        scratch_rows(env, rows, &mya_env::d_sampled, &mya_env::sampled_rows);
        if (grouped(env))
            scratch_rows(env, rows, &mya_env::d_order, &mya_env::group_rows);
        for (const EnvInstance& in : env->inst)
            prepare_env_launches(in.T);
        for (const mya_env::Launch& l : env->launches)
            prepare_grouped_launches(l.variant, l.lds);
    });
}

int mya_env_clear_visited(mya_env* env, const mya_env_batch* batch, const uint8_t* mask, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        check_batch(env, batch);
        if (env->instances() > 1 && batch->task_ids)
            launch_check_ids(batch->task_ids, batch->rows, env->instances(), env->d_status, static_cast<hipStream_t>(stream));
        launch_visited_restart(visited_of(batch), env->d_inst, env->instances(), batch->states, batch->rows, batch->words, mask,
                               batch->task_ids, true, static_cast<hipStream_t>(stream));
    });
}

int mya_env_set_seed(mya_env* env, uint64_t seed, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        launch_set_word(env->d_seed, seed, static_cast<hipStream_t>(stream));
    });
}

int mya_env_random_actions(mya_env* env, const mya_env_batch* batch, const int32_t* count, uint32_t max_actions, int64_t* out, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        check_batch(env, batch);
        if (batch->rows && (!batch->draws || !count || !out))
            throw std::invalid_argument("mymyr_amd: env: random_actions needs the draw counters, the counts and an output array");
        launch_env_random_actions(env->d_seed, batch->seeds, batch->env_ids, batch->first_env, batch->draws, count, batch->rows,
                                  max_actions ? max_actions : 0xFFFFFFFFu, out, static_cast<hipStream_t>(stream));
    });
}

int mya_env_goal(mya_env* env, const mya_env_batch* batch, uint8_t* goal, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        check_batch(env, batch);
        if (batch->rows && !goal)
            throw std::invalid_argument("mymyr: env: goal query needs an output array");
        CountArgs a{};
        a.goal = goal;
        run_count(env, batch, a, static_cast<hipStream_t>(stream));
    });
}

int mya_env_check(mya_env* env)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        hip_check(hipMemcpy(env->h_status, env->d_status, sizeof(u32), hipMemcpyDeviceToHost), "env status");
        const u32 s = *env->h_status;
        if (s)
        {
            hip_check(hipMemset(env->d_status, 0, sizeof(u32)), "env status");
            std::string m = "mymyr_amd: env: device status";
            if (s & kStatusCapacity)
                m += " capacity";
            if (s & kStatusNoSlot)
                m += " add-effect-without-slot";
            if (s & kStatusPickFailed)
                m += " pick-failed";
            if (s & kStatusGoalMask)
                m = "mymyr: env: goal masks set fluent slots the task does not have; supply goals for the task's slots";
            if (s & kStatusTaskId)
                m = "mymyr: env: a task id is outside the table's " + std::to_string(env->instances()) +
                    " instances (a reset put its row in instance 0; a step left its row unstepped or kept an autoresetting row's instance)";
            throw std::runtime_error(m);
        }
    });
}

int mya_encode_atoms(mya_env* env, const uint64_t* states, uint64_t rows, uint32_t words, int32_t* out, uint32_t max_atoms, void* stream)
{
    return guarded([&] {
        if (!env || (rows && (!states || !out)))
            throw std::invalid_argument("mymyr_amd: encode_atoms: null argument");
        if (words < env->words)
            throw std::invalid_argument("mymyr_amd: encode_atoms: rows narrower than the widest instance");
        launch_encode_atoms(states, rows, words, env->words, out, max_atoms, env->d_status, static_cast<hipStream_t>(stream));
    });
}

int mya_schema_masks(mya_env* env, const uint64_t* states, uint64_t rows, uint32_t words, uint8_t* masks, void* stream)
{
    return guarded([&] {
        if (!env || (rows && (!states || !masks)))
            throw std::invalid_argument("mymyr_amd: schema_masks: null argument");
        if (words < env->T0().W)
            throw std::invalid_argument("mymyr_amd: schema_masks: rows narrower than the task");
        launch_env_count(env->T0(), states, rows, words, nullptr, nullptr, masks, nullptr, static_cast<hipStream_t>(stream));
    });
}

int mya_successors(mya_task* task, const uint64_t* states, uint64_t rows, uint32_t words, int32_t cap, int32_t* count, int32_t* schema,
                   int32_t* binding, uint64_t* succ, void* stream)
{
    return guarded([&] {
        if (!task || (rows && (!states || !count)))
            throw std::invalid_argument("mymyr_amd: successors: null argument");
        if (cap < 0)
            throw std::invalid_argument("mymyr_amd: successors: negative cap");
        std::unique_lock<std::mutex> lazy_lock;
        if (lazy_task(task))
            lazy_lock = std::unique_lock<std::mutex>(task->lazy_mutex);
        const DeviceTask& d = device_task(task);
        if (words < d.thost->W && !lazy_task(task))
            throw std::invalid_argument("mymyr_amd: successors: rows of " + std::to_string(words) + " words; the task needs " +
                                        std::to_string(d.thost->W));
        const hipStream_t s = static_cast<hipStream_t>(stream);
        ScratchLease lease(scratch_bytes<u32>(1), "successors status");
        u32* st = lease.take<u32>(1);
        u32 hs = 0;
        for (;;)
        {
            launch_fill_u32(st, 1, 0, s);
            launch_successors(*d.thost, states, rows, words, static_cast<u32>(cap), count, schema, binding, succ, st, s);
            hip_check(hipMemcpyAsync(&hs, st, sizeof(u32), hipMemcpyDeviceToHost, s), "status");
            hip_check(hipStreamSynchronize(s), "successors");
            // lazy slots: the listing again once the added atoms without a slot are interned
            if (!(lazy_task(task) && (hs & kStatusNoSlot) && succ))
                break;
            if (!resolve_missing(task, s))
                throw std::logic_error("mymyr_amd: successors: an added atom without a slot was not recorded");
        }
        if (hs & kStatusWideRow)
            throw std::invalid_argument("mymyr: successors: a successor has atoms past the rows' " + std::to_string(words) +
                                        " words (the task's lazy slots now need " + std::to_string(d.thost->W) + ")");
        if (hs)
            throw std::runtime_error("mymyr_amd: successors: device status " + std::to_string(hs));
    });
}

int mya_expand(mya_task* task, const uint64_t* states, uint64_t rows, uint32_t words, const mya_expand_options* options,
               mya_expansion* out, void* stream)
{
    return guarded([&] {
        if (!task)
            throw std::invalid_argument("mymyr_amd: expand: null argument");
        std::unique_lock<std::mutex> lazy_lock;
        if (lazy_task(task))
            lazy_lock = std::unique_lock<std::mutex>(task->lazy_mutex);
        const TaskDev* T = device_task(task).thost.get();
        ScratchLease lease(expand_scratch_bytes(std::max<u64>(rows, 1)), "expand scratch");
        expand_rows({T}, nullptr, nullptr, states, rows, words, options, out, static_cast<hipStream_t>(stream), lease.base(),
                    lazy_task(task) ? task : nullptr);
    });
}

int mya_env_expand(mya_env* env, const uint64_t* states, const int32_t* task_ids, uint64_t rows, uint32_t words,
                   const mya_expand_options* options, mya_expansion* out, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: expand: null env");
        if (!task_ids && rows && env->instances() > 1)
            throw std::invalid_argument("mymyr: expand: a batch over a table of " + std::to_string(env->instances()) +
                                        " instances needs task ids");
        std::vector<const TaskDev*> inst;
        for (const EnvInstance& in : env->inst)
            inst.push_back(&in.T);
        ScratchLease lease(expand_scratch_bytes(std::max<u64>(rows, 1)), "expand scratch");
        expand_rows(inst, env, task_ids, states, rows, words, options, out, static_cast<hipStream_t>(stream), lease.base());
    });
}

int mya_pad(const mya_expansion* flat, uint64_t rows, mya_padded_expansion* out, void* stream)
{
    return guarded([&] {
        if (!flat || !out)
            throw std::invalid_argument("mymyr_amd: pad: null argument");
        if (!flat->offsets)
            throw std::invalid_argument("mymyr: pad: the flat expansion has no offsets");
        if (out->succ && flat->succ && out->words < flat->words)
            throw std::invalid_argument("mymyr: pad: padded rows narrower than the flat rows");
        if (out->binding && flat->binding && out->label_width < flat->label_width)
            throw std::invalid_argument("mymyr: pad: padded label width below the flat label width");
        constexpr u64 kMaxRows = (u64{1} << 31) - 1;
        if (rows > kMaxRows || flat->capacity > kMaxRows)
            throw std::invalid_argument("mymyr_amd: pad: more than 2^31 - 1 states or flat rows");
        const bool flat_overflow = flat->generated > flat->capacity || flat->total > flat->capacity || flat->words_needed > flat->words;
        ScratchLease lease(scratch_bytes<u32>(1), "pad overflow");
        u32* d_over = lease.take<u32>(1);
        const hipStream_t s = static_cast<hipStream_t>(stream);
        launch_fill_u32(d_over, 1, 0, s);
        PadArgs a{};
        a.rows = rows;
        a.capacity = flat->capacity;
        a.offsets = flat->offsets;
        a.succ = flat->succ;
        a.flat_words = flat->words;
        a.flat_label_width = flat->label_width;
        a.schema = flat->schema;
        a.binding = flat->binding;
        a.goal = flat->goal;
        a.succ_hash = flat->succ_hash;
        a.noop = flat->noop;
        a.index = flat->index;
        a.k = out->k;
        a.words = out->words;
        a.label_width = out->label_width;
        a.out_index = out->index;
        a.mask = out->mask;
        a.count = out->count;
        a.out_succ = out->succ;
        a.out_schema = out->schema;
        a.out_binding = out->binding;
        a.out_goal = out->goal;
        a.out_succ_hash = out->succ_hash;
        a.out_noop = out->noop;
        a.canonical = out->canonical;
        a.overflow = d_over;
        launch_pad(a, s);
        u32 h = 0;
        hip_check(hipMemcpyAsync(&h, d_over, sizeof(h), hipMemcpyDeviceToHost, s), "pad overflow");
        hip_check(hipStreamSynchronize(s), "pad");
        out->overflow = flat_overflow || h ? 1 : 0;
    });
}

int mya_visited_mask(const uint64_t* table, const int32_t* count, uint64_t table_rows, uint32_t capacity, const uint64_t* succ_hash,
                     const int32_t* parent, const int32_t* rows, uint64_t parents, uint64_t size, uint8_t* out, void* stream)
{
    return guarded([&] {
        if (capacity < 2 || capacity > (1u << 20) || (capacity & (capacity - 1)))
            throw std::invalid_argument("mymyr: visited capacity must be a power of two in [2, 2^20]");
        if (size && (!succ_hash || !parent || !out || (table_rows && (!table || !count))))
            throw std::invalid_argument("mymyr: visited_mask requires table, count, succ_hash, parent and out arrays");
        if (!rows)
            parents = table_rows;
        launch_visited_mask(table, count, table_rows, capacity, succ_hash, parent, rows, parents, size, out,
                            static_cast<hipStream_t>(stream));
    });
}

int mya_label_actions(const int32_t* offsets, const int32_t* schema, const int32_t* binding, uint32_t label_width, uint64_t rows,
                      const int32_t* label_schema, const int32_t* label_binding, uint32_t stride, int64_t* actions, void* stream)
{
    return guarded([&] {
        if (stride < label_width)
            throw std::invalid_argument("mymyr: env: label stride " + std::to_string(stride) + " is below the label width " +
                                        std::to_string(label_width));
        if (rows && (!offsets || !label_schema || !actions || (label_width && !label_binding)))
            throw std::invalid_argument("mymyr: env: label mode requires explicit labels");
        launch_label_actions(offsets, schema, binding, label_width, rows, label_schema, label_binding, stride, actions,
                             static_cast<hipStream_t>(stream));
    });
}

}  // extern "C"
