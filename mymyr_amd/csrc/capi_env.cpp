// C ABI of the device environment and the successor listing (include/mymyr_amd.h, "env" section). Argument checks
// follow the reference's check_env / check_step messages (src/mymyr/rl/env.cpp:102-135, 403-421).

#include "../../include/mymyr_amd.h"

#include "capi_internal.hpp"
#include "env.hpp"
#include "runtime.hpp"
#include "scan.hpp"
#include "state_set.hpp"

#include <cstring>
#include <vector>

using namespace mya;

struct mya_env
{
    mya_task* task = nullptr;
    TaskDev T{};                // host copy of the pointer table
    EnvCfg cfg{};
    u32 init_count = 0;
    u32 init_goal = 0;
    u8* init_masks = nullptr;  // device [num_schemas]
    u32* init_cache = nullptr; // device [num_schemas + 2]: the initial state's count-cache row
    u64* goal_masks = nullptr; // device [2, W]: the task's goal as masks (positive, then negative)
    u32* d_status = nullptr;
    u32* h_status = nullptr;
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
    if (b->words < e->T.W)
        throw std::invalid_argument("mymyr: env: state rows of " + std::to_string(b->words) + " words; the task needs " +
                                    std::to_string(e->T.W) + " (its widest instance's words)");
    if ((b->goal_pos == nullptr) != (b->goal_neg == nullptr))
        throw std::invalid_argument("mymyr: env: per-env goals need both goal_pos and goal_neg");
    if (b->goal_pos && e->T.goal_unsat)
        throw std::invalid_argument("mymyr: env: per-env goal masks cannot express the goal of instance 0 (it is statically "
                                    "unsatisfiable); use the instances' goal tests (no goal masks)");
}
}  // namespace

extern "C" {

int mya_env_create(mya_task* task, const mya_env_config* config, mya_env** out)
{
    return guarded([&] {
        if (!task || !config || !out)
            throw std::invalid_argument("mymyr_amd: env_create: null argument");
        if (!config->canonical_order || config->witness_pruning)
            throw std::invalid_argument("mymyr_amd: env: the device step takes canonical_order on and witness_pruning off");
        if (config->dead_end != 0 && config->dead_end != 1)
            throw std::invalid_argument("mymyr_amd: env: dead_end must be 0 (no_successors) or 1 (none)");
        auto e = std::make_unique<mya_env>();
        e->task = task;
        const DeviceTask& d = device_task(task);
        e->T = *d.thost;
        e->cfg.seed = config->seed;
        e->cfg.max_steps = config->max_steps;
        e->cfg.step_reward = config->step_reward;
        e->cfg.goal_reward = config->goal_reward;
        e->cfg.dead_end_reward = config->dead_end_reward;
        e->cfg.dead_end_none = config->dead_end == 1 ? 1 : 0;
        e->cfg.dead_end_terminal = config->dead_end_terminal;
        e->cfg.autoreset = config->autoreset;
        e->d_status = dev_alloc<u32>(1, "env status");
        hip_check(hipHostMalloc(reinterpret_cast<void**>(&e->h_status), sizeof(u32), hipHostMallocDefault), "pinned status");
        hip_check(hipMemset(e->d_status, 0, sizeof(u32)), "env status");
        // the initial state's successor count and goal flag
        const u32 W = e->T.W;
        u64* row = dev_alloc<u64>(W, "initial row");
        i32* cnt = dev_alloc<i32>(1, "initial count");
        u8* gl = dev_alloc<u8>(1, "initial goal");
        hip_check(hipMemcpy(row, task->compiled->initial.data(), W * sizeof(u64), hipMemcpyHostToDevice), "initial row");
        e->init_masks = dev_alloc<u8>(std::max<u32>(1, e->T.num_schemas), "initial masks");
        e->init_cache = dev_alloc<u32>(cache_width(e->T), "initial count cache");
        {
            // the task's goal as masks over its words
            std::vector<u64> gm(2 * static_cast<size_t>(W), 0);
            for (u32 sl : task->compiled->goal_pos)
                gm[sl >> 6] |= u64{1} << (sl & 63);
            for (u32 sl : task->compiled->goal_neg)
                gm[W + (sl >> 6)] |= u64{1} << (sl & 63);
            e->goal_masks = dev_alloc<u64>(gm.size(), "goal masks");
            hip_check(hipMemcpy(e->goal_masks, gm.data(), gm.size() * sizeof(u64), hipMemcpyHostToDevice), "goal masks");
        }
        launch_env_count(e->T, row, 1, W, cnt, gl, e->init_masks, e->init_cache, nullptr);
        i32 hc = 0;
        u8 hg = 0;
        hip_check(hipMemcpy(&hc, cnt, sizeof(i32), hipMemcpyDeviceToHost), "initial count");
        hip_check(hipMemcpy(&hg, gl, sizeof(u8), hipMemcpyDeviceToHost), "initial goal");
        dev_free(row);
        dev_free(cnt);
        dev_free(gl);
        e->init_count = static_cast<u32>(hc);
        e->init_goal = hg;
        *out = e.release();
    });
}

void mya_env_free(mya_env* env)
{
    if (!env)
        return;
    dev_free(env->d_status);
    dev_free(env->init_masks);
    dev_free(env->init_cache);
    dev_free(env->goal_masks);
    if (env->h_status)
        (void)hipHostFree(env->h_status);
    delete env;
}

int mya_env_initial_count(const mya_env* env, uint32_t* count, uint8_t* goal)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        if (count)
            *count = env->init_count;
        if (goal)
            *goal = static_cast<uint8_t>(env->init_goal);
    });
}

int mya_env_reset(mya_env* env, const mya_env_batch* batch, const uint8_t* mask, int32_t* count, int keep_goals, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        check_batch(env, batch);
        launch_env_reset(env->T, batch->states, batch->rows, batch->words, mask, batch->steps, batch->at_goal, count, batch->counts,
                         env->init_cache, env->init_count, env->init_goal, static_cast<hipStream_t>(stream));
        if (batch->goal_pos)
            launch_env_reset_goals(env->T, batch->rows, batch->words, mask, batch->goal_pos, batch->goal_neg, env->goal_masks,
                                   env->goal_masks + env->T.W, keep_goals != 0, batch->at_goal, env->d_status,
                                   static_cast<hipStream_t>(stream));
    });
}

int mya_env_step(mya_env* env, const mya_env_batch* batch, const mya_step_outputs* out, const int64_t* actions, void* stream)
{
    return guarded([&] {
        if (!env || !out)
            throw std::invalid_argument("mymyr_amd: env: null argument");
        check_batch(env, batch);
        if (batch->rows && !batch->at_goal)
            throw std::invalid_argument("mymyr_amd: env: the device step needs the at_goal array");
        if (!actions && batch->rows && !batch->draws)
            throw std::invalid_argument("mymyr: env: the random policy needs the draw counters");
        if (env->cfg.max_steps && batch->rows && !batch->steps)
            throw std::invalid_argument("mymyr: env: truncation (max_steps) needs the step counters");
        if (out->binding && out->label_width < env->T.label_width)
            throw std::invalid_argument("mymyr: env: label width " + std::to_string(out->label_width) + " is below the largest schema arity " +
                                        std::to_string(env->T.label_width));
        const u32 fw = out->final_words ? out->final_words : batch->words;
        if (out->final_states && fw < env->T.W)
            throw std::invalid_argument("mymyr: env: final state rows of " + std::to_string(fw) + " words; the task has " +
                                        std::to_string(env->T.W));
        EnvArgs a{};
        a.T = env->T;
        a.cfg = env->cfg;
        a.states = batch->states;
        a.rows = batch->rows;
        a.words = batch->words;
        a.steps = batch->steps;
        a.draws = batch->draws;
        a.at_goal = batch->at_goal;
        a.first_env = batch->first_env;
        a.actions = actions;
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
        a.init_masks = env->init_masks;
        a.counts = batch->counts;
        a.init_counts = env->init_cache;
        a.goal_pos = batch->goal_pos;
        a.goal_neg = batch->goal_neg;
        a.task_goal_pos = env->goal_masks;
        a.task_goal_neg = env->goal_masks + env->T.W;
        if (out->atoms && out->max_atoms == 0)
            throw std::invalid_argument("mymyr_amd: env: atoms output needs max_atoms > 0");
        a.init_count = env->init_count;
        a.init_goal = env->init_goal;
        a.status = env->d_status;
        launch_env_step(a, static_cast<hipStream_t>(stream));
    });
}

int mya_env_refresh(mya_env* env, const mya_env_batch* batch, int32_t* count, void* stream)
{
    return guarded([&] {
        if (!env)
            throw std::invalid_argument("mymyr_amd: env: null env");
        check_batch(env, batch);
        launch_env_count(env->T, batch->states, batch->rows, batch->words, count, batch->at_goal, nullptr, batch->counts,
                         static_cast<hipStream_t>(stream), batch->goal_pos, batch->goal_neg, env->d_status);
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
            throw std::runtime_error(m);
        }
    });
}

int mya_encode_atoms(mya_env* env, const uint64_t* states, uint64_t rows, uint32_t words, int32_t* out, uint32_t max_atoms, void* stream)
{
    return guarded([&] {
        if (!env || (rows && (!states || !out)))
            throw std::invalid_argument("mymyr_amd: encode_atoms: null argument");
        if (words < env->T.W)
            throw std::invalid_argument("mymyr_amd: encode_atoms: rows narrower than the task");
        launch_encode_atoms(states, rows, words, env->T.W, out, max_atoms, env->d_status, static_cast<hipStream_t>(stream));
    });
}

int mya_schema_masks(mya_env* env, const uint64_t* states, uint64_t rows, uint32_t words, uint8_t* masks, void* stream)
{
    return guarded([&] {
        if (!env || (rows && (!states || !masks)))
            throw std::invalid_argument("mymyr_amd: schema_masks: null argument");
        if (words < env->T.W)
            throw std::invalid_argument("mymyr_amd: schema_masks: rows narrower than the task");
        launch_env_count(env->T, states, rows, words, nullptr, nullptr, masks, nullptr, static_cast<hipStream_t>(stream));
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
        const DeviceTask& d = device_task(task);
        const TaskDev& T = *d.thost;
        if (words < T.W)
            throw std::invalid_argument("mymyr_amd: successors: rows of " + std::to_string(words) + " words; the task needs " +
                                        std::to_string(T.W));
        u32* st = dev_alloc<u32>(1, "status");
        hip_check(hipMemsetAsync(st, 0, sizeof(u32), static_cast<hipStream_t>(stream)), "status");
        launch_successors(T, states, rows, words, static_cast<u32>(cap), count, schema, binding, succ, st, static_cast<hipStream_t>(stream));
        u32 hs = 0;
        hip_check(hipMemcpyAsync(&hs, st, sizeof(u32), hipMemcpyDeviceToHost, static_cast<hipStream_t>(stream)), "status");
        hip_check(hipStreamSynchronize(static_cast<hipStream_t>(stream)), "successors");
        dev_free(st);
        if (hs)
            throw std::runtime_error("mymyr_amd: successors: device status " + std::to_string(hs));
    });
}

int mya_expand(mya_task* task, const uint64_t* states, uint64_t rows, uint32_t words, const mya_expand_options* options,
               mya_expansion* out, void* stream_)
{
    return guarded([&] {
        if (!task || !options || !out || (rows && !states))
            throw std::invalid_argument("mymyr_amd: expand: null argument");
        if (!options->canonical_order || options->witness_pruning)
            throw std::invalid_argument("mymyr_amd: expand: the device expansion takes canonical_order on and witness_pruning off");
        const DeviceTask& d = device_task(task);
        const TaskDev& T = *d.thost;
        constexpr u64 kMaxRows = (u64{1} << 31) - 1;
        if (rows > kMaxRows)
            throw std::invalid_argument("mymyr: expand: more than 2^31 - 1 states in one batch");
        if (words < T.W)
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
        const auto stream = static_cast<hipStream_t>(stream_);
        out->generated = out->total = 0;
        out->words_needed = 0;
        // scratch: per-row counts and no-op counts, offsets before and after dropping, scan scratch, status words
        const u64 n = std::max<u64>(rows, 1);
        u32* counts = dev_alloc<u32>(n, "expand counts");
        u32* noops = dev_alloc<u32>(n, "expand no-op counts");
        u32* kept = dev_alloc<u32>(n, "expand kept counts");
        u64* pre = dev_alloc<u64>(n + 1, "expand offsets");
        u64* fin = dev_alloc<u64>(n + 1, "expand kept offsets");
        u64* scratch = dev_alloc<u64>(scan_scratch_words(n), "expand scan scratch");
        u32* words_status = dev_alloc<u32>(2, "expand status");  // [0] words needed, [1] status
        struct Free
        {
            std::vector<void*> p;
            ~Free()
            {
                for (void* q : p)
                    dev_free(q);
            }
        } freeing{{counts, noops, kept, pre, fin, scratch, words_status}};
        launch_fill_u32(words_status, 2, 0, stream);
        ExpandArgs a{};
        a.T = T;
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
        launch_expand(a, stream);
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
            launch_expand(a, stream);
        }
        hip_check(hipMemcpyAsync(st, words_status, sizeof(st), hipMemcpyDeviceToHost, stream), "expand status");
        hip_check(hipStreamSynchronize(stream), "expand");
        if (st[1] & ~kStatusWideRow)
            throw std::runtime_error("mymyr_amd: expand: device status " + std::to_string(st[1]));
        out->words_needed = st[0];
    });
}

}  // extern "C"
