/* mymyr_amd: the MI355X-native state-expansion path of a lifted classical planner (applicable-action testing,
 * effect application on packed u64 bitset states, goal and reward evaluation, 64-bit state hashing and device
 * dedup), exposed as a C ABI: plain pointers and sizes, int status returns, no Python or torch types.
 *
 * Conventions
 *   - Every function returns 0 on success and a negative value on failure; mya_last_error() then holds the message
 *     (thread-local). Argument errors name the argument, as the reference's "mymyr: ..." exceptions do
 *     (src/mymyr/rl/env.cpp:102-135).
 *   - Pointers documented "device" are HIP device memory; "stream" is a hipStream_t (null: the default stream).
 *     Calls on a stream are asynchronous unless documented otherwise.
 *   - States are rows of `words` little-endian u64 words; slot i is bit i & 63 of word i >> 6 (the reference's state
 *     contract, include/mymyr/core/bitset.hpp:2-5).
 *   - Caller-owned output arrays that are null are not written (include/mymyr/rl/env.hpp:137).
 */
#ifndef MYMYR_AMD_H
#define MYMYR_AMD_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct mya_task mya_task;
typedef struct mya_env mya_env;
typedef struct mya_hashset mya_hashset;

/* ---------------------------------------------------------------------------------------------------------- misc */

/* The last error message of the calling thread ("" if none). */
const char* mya_last_error(void);

/* ABI version of this header (bumped on any signature change). */
#define MYA_ABI_VERSION 20
int mya_abi_version(void);

/* Device memory held by the library (replaces DeviceContext::usage(), include/mymyr/cuda/runtime.hpp:140-146, 183):
 * freed blocks are kept for reuse, so `reserved` (bytes taken from the driver: handed out, idle, or waiting for a
 * stream-ordered free) can exceed `used` (bytes handed out). `allocations` counts the device blocks the library has
 * handed out (from its cache or the driver), `driver_allocations` its hipMalloc calls; both only grow. */
typedef struct mya_memory_usage
{
    uint64_t reserved;
    uint64_t used;
    uint64_t reserved_high;
    uint64_t used_high;
    uint64_t allocations;
    uint64_t driver_allocations;
} mya_memory_usage;
int mya_memory_usage_get(mya_memory_usage* out);

/* ---------------------------------------------------------------------------------------------------------- tasks */

/* Atom slot modes (reference TaskOptions::Atoms, include/mymyr/task/task.hpp:88-104). Lazy slots
 * (include/mymyr/task/atom_index.hpp:19-22) start with the initial state's atoms, in its atom order; the device BrFS,
 * mya_expand, mya_expand_noalloc and mya_successors give the atoms their successors add without a slot the next
 * slots, in ascending canonical id, between device launches (include/mymyr/cuda/generator.hpp:20-24), so a lazy
 * task's words and fluent_slots grow with use. Such calls on one lazy task run one at a time. Environments and task
 * tables refuse lazy tasks, as the reference's TaskTable does (src/mymyr/rl/task_table.cpp:120-123). */
#define MYA_ATOMS_AUTO 0
#define MYA_ATOMS_REACHABLE 1
#define MYA_ATOMS_DENSE 2
#define MYA_ATOMS_LAZY 3

/* Loads a task from the reference's text format (replaces Task::from_text_file / Task::create over
 * read_task_text, include/mymyr/task/task.hpp:166-167, include/mymyr/formalism/text_format.hpp:23-24).
 * Host-only: compiles the canonical layout, atom slots, initial state, goal and the device tables. */
int mya_task_load_text(const char* text, size_t len, int atoms, mya_task** out);
int mya_task_load_file(const char* path, int atoms, mya_task** out);
void mya_task_free(mya_task* task);

typedef struct mya_task_info
{
    uint32_t words;         /* state words W (Task::words(), at least 1; lazy slots: the current width) */
    uint32_t fluent_slots;  /* atom slots (lazy slots: those assigned so far) */
    uint32_t atom_mode;     /* 0 reachable, 1 dense, 2 lazy (AtomMode) */
    uint32_t num_schemas;
    uint32_t label_width;   /* largest schema arity */
    uint32_t num_objects;
    uint32_t max_arity;     /* largest fluent predicate arity */
    uint32_t goal_unsat;    /* no state is a goal under the current slots */
    uint64_t dense_fluent;  /* size of the typed-dense canonical fluent space */
    uint64_t reachable_fluent; /* relaxed-reachable fluent atoms (0 when not computed: dense option; under auto the count
                                * stops once it fills the dense layout's words, which decides the mode) */
    uint32_t view_words;    /* per-state device view size in u64 words */
    uint32_t reserved;
} mya_task_info;

int mya_task_info_get(const mya_task* task, mya_task_info* out);

/* Slot records: rec [fluent_slots, 1 + max(1, max_arity)] u32 = predicate then arguments (zero padded);
 * cid [fluent_slots] u64 canonical ids (AtomIndex::record / canonical, include/mymyr/task/atom_index.hpp:167-172).
 * Either may be null. Lazy slots: fluent_slots as mya_task_info_get last reported it, with no call that interns
 * between the two. */
int mya_task_slots(const mya_task* task, uint32_t* rec, uint64_t* cid);

/* The initial state, zero padded to `words` (>= the task's words). Host memory. */
int mya_task_initial(const mya_task* task, uint64_t* row, uint32_t words);

/* ---------------------------------------------------------------------------------------------------------- hashing */

/* hash_state of `n` rows of `words` words: the reference's public state hash over the trimmed words
 * (hash::state, include/mymyr/core/hash.hpp:56-60; device hash_rows, python/src/cuda_bindings.cpp:1289-1320).
 * rows, out: device. */
int mya_hash_rows(const uint64_t* rows, uint64_t n, uint32_t words, uint64_t* out, void* stream);

/* Host versions (C API hash_words, include/mymyr/ext.h:104). */
uint64_t mya_hash_words(const uint64_t* w, uint32_t n, uint64_t seed);
uint64_t mya_hash_state(const uint64_t* w, uint32_t n);

/* Philox-4x32-10 block of (seed; draw, env, purpose) and the random-policy index (include/mymyr/rl/rng.hpp:45-83),
 * host versions of the device code. */
void mya_philox(uint64_t seed, uint64_t env, uint64_t draw, uint32_t purpose, uint32_t out[4]);
uint32_t mya_successor_index(uint64_t seed, uint64_t env, uint64_t draw, uint32_t count);
/* The instance of env `env`'s draw number `reset_count` under `seed` (rl::rng::instance_draw,
 * include/mymyr/rl/rng.hpp:94-115): uniform over `instances` when m is 0, else indices[k] with k the number of the
 * m - 1 ascending thresholds at most the draw's 32 bits (host arrays). */
int32_t mya_instance_draw(uint64_t seed, uint64_t env, uint32_t reset_count, uint32_t instances, const uint32_t* thresholds,
                          const int32_t* indices, uint32_t m);

/* ---------------------------------------------------------------------------------------------------------- state set */

/* A device-resident open-addressing set of rows of `words` words with capacity ceil(max_states / max_load) slots
 * (replaces the state_set launchers, include/mymyr/cuda/state_set.hpp:52-91). batch: the most rows one insert
 * processes at once (larger inserts are split). */
int mya_hashset_create(uint64_t max_states, uint32_t words, double max_load, uint64_t batch, mya_hashset** out);
void mya_hashset_free(mya_hashset* set);

/* Inserts n rows (device). ids (device, optional) receives each row's state id (the first-inserted equal row's id:
 * smallest batch index wins within a batch, new ids in row order; -1 for a row whose state did not fit); is_new
 * (device, optional) 1 for rows that added a state. With new_count (host) the call synchronizes the stream, returns
 * the number of new states and fails if the set overflowed; without it the insert is asynchronous and an overflow is
 * reported by the next mya_hashset_size. A set that overflowed must be cleared. */
int mya_hashset_insert(mya_hashset* set, const uint64_t* rows, uint64_t n, int64_t* ids, uint8_t* is_new,
                       uint64_t* new_count, void* stream);
/* The number of stored states; waits for the set's last insert and fails if an insert overflowed the set. */
int mya_hashset_size(mya_hashset* set, uint64_t* size);
/* Device pointer to the stored rows [size, words] in id order. */
int mya_hashset_rows(const mya_hashset* set, const uint64_t** rows);
int mya_hashset_clear(mya_hashset* set, void* stream);

/* No reference counterpart: the synthetic input of the dedup workload. Rows [start, start + count) of the seeded
 * stream in which row i > 0 is, with probability dup, an exact copy of an earlier row, else fresh words
 * mix64(seed + (16 i + k + 1) * 0x9E3779B97F4A7C15). out [count, words]: device. Async on the stream. */
int mya_dedup_rows(uint64_t start, uint64_t count, uint32_t words, uint64_t seed, double dup, uint64_t* out, void* stream);

/* No reference counterpart: the random-access rates the state set's probes are bound by, for measurement. n operations
 * of one kind (0 load, 1 compare-and-swap, 2 atomic min, 3 store; the atomics' old values are used, as the probes use
 * them) on 8-byte words at seeded random addresses of table [words] (device; words a power of two), 4 independent
 * operations per thread in flight over MYA_RANDOM_OPS_THREADS threads, whose folded load and atomic results go to
 * sink [MYA_RANDOM_OPS_THREADS] (device). Async on the stream. */
#define MYA_RANDOM_OPS_THREADS 1048576u
int mya_random_ops(uint64_t* table, uint64_t words, uint64_t n, int kind, uint64_t seed, uint64_t* sink, void* stream);

/* ---------------------------------------------------------------------------------------------------------- env */

/* EnvConfig (include/mymyr/rl/env.hpp:76-92), index action space. dead_end: 0 no_successors, 1 none.
 * canonical_order must be 1 and witness_pruning 0 (the reference env defaults; the device step implements those). */
typedef struct mya_env_config
{
    uint64_t seed;
    uint32_t max_steps;
    float step_reward;
    float goal_reward;
    float dead_end_reward;
    int32_t dead_end;
    int32_t dead_end_terminal;
    int32_t autoreset;
    int32_t canonical_order;
    int32_t witness_pruning;
    int32_t reserved;
} mya_env_config;

/* EnvBatch (include/mymyr/rl/env.hpp:96-135), device pointers: states [rows, words] (required), steps i32 [rows],
 * draws u64 [rows] (required for the random policy), at_goal u8 [rows] (required, as for the reference device env). */
typedef struct mya_env_batch
{
    uint64_t* states;
    uint64_t rows;
    uint32_t words;
    uint32_t reserved;
    int32_t* steps;
    uint64_t* draws;
    uint8_t* at_goal;
    uint64_t first_env;
    /* The count cache (the reference device env's EnvBatch::counts, include/mymyr/rl/env.hpp:106-110), optional:
     * [rows, S + 2] uint32 with S the most schemas of any instance of the env, each row's per-schema successor counts
     * of its current state (0 past its instance's schemas), then a 64-bit fingerprint of that state and its
     * instance (low word first). reset, refresh and step keep it current, and a step takes the
     * counts of a row from it instead of counting the row's successors when the fingerprint matches the row's state
     * (a state written directly is counted again; refresh brings at_goal up to date for it). Null: every step counts. */
    uint32_t* counts;
    /* Per-env goal masks (EnvBatch::goal_pos / goal_neg, include/mymyr/rl/env.hpp:103-104), optional, both or neither:
     * [rows, words] each. A row's goal is (s & goal_pos) == goal_pos and (s & goal_neg) == 0 (mask_goal,
     * src/mymyr/rl/env.cpp:55-61). reset writes the task's goal into them unless keep_goals; an autoreset writes it. */
    uint64_t* goal_pos;
    uint64_t* goal_neg;
    /* Each row's instance (EnvBatch::task_ids, include/mymyr/rl/env.hpp:102), device int32 [rows], optional: null puts
     * every row in instance 0 (required over several instances). reset puts a row in the instance its entry names; an
     * autoreset writes the instance the row restarts in. A row's words past its instance's are padding: a step
     * neither reads nor writes them, and a reset zeroes the words it may have dirtied (TaskSuite::initial_row,
     * src/mymyr/rl/task_suite.cpp:130-138). */
    int32_t* task_ids;
    /* Per-row RNG keys and env ids of the random policy (EnvBatch::seeds / env_ids, include/mymyr/rl/env.hpp:114-115),
     * device, optional: null uses the config's seed and first_env + row. */
    const uint64_t* seeds;
    const uint32_t* env_ids;
    /* The instance sampler's per-row counters and keys (EnvBatch::reset_counts / sampling_seeds, rl/env.hpp:116-120),
     * device, optional: a row's next sampled instance is the draw of (its sampling key or the config's seed, its env
     * id, reset_counts[row]); every reset and autoreset of the row advances its counter, sampled or not. Null
     * reset_counts: no counting and no sampling. */
    uint32_t* reset_counts;
    const uint64_t* sampling_seeds;
    /* Visited tables (EnvBatch::visited, include/mymyr/rl/env.hpp:126-130; rl/visited.hpp), device, optional (null
     * visited: none): visited [rows, visited_capacity] u64 keys by linear probing (the reference's layout, word for
     * word), visited_count [rows], visited_status [1] (or [rows] with visited_status_per_row) with sticky bit 0 for an
     * overflowed row. visited_capacity is a power of two in [2, 2^20]. reset restarts a reset row's table with its
     * initial state's key; a step inserts the reached state's key (unless the episode is over without autoreset) and
     * an autoreset restarts the table. */
    uint64_t* visited;
    int32_t* visited_count;
    int32_t* visited_status;
    uint32_t visited_capacity;
    int32_t visited_status_per_row;
} mya_env_batch;

/* StepOutputs (include/mymyr/rl/env.hpp:138-152), device pointers, null = not written. binding [rows, label_width];
 * final_states [rows, final_words] (final_words 0: the batch's words).
 * atoms [rows, max_atoms] int32 and masks [rows, num_schemas] uint8 encode the observed state after the step (and
 * the autoreset): its true-atom slots ascending, -1 padded (State::slots, include/mymyr/state/state.hpp:96-101), and
 * the schemas with an applicable binding (rl::schema_masks, include/mymyr/rl/masks.hpp:9-11). */
typedef struct mya_step_outputs
{
    float* reward;
    uint8_t* terminated;
    uint8_t* truncated;
    int32_t* count;
    uint64_t* final_states;
    int32_t* schema;
    int32_t* binding;
    uint32_t label_width;
    uint32_t final_words;
    uint8_t* invalid;
    uint8_t* goal;
    int32_t* atoms;
    uint8_t* masks;
    uint32_t max_atoms;
    uint32_t reserved;
    /* [rows]: the reached state's key was in the row's visited table before the step (StepOutputs::revisited) */
    uint8_t* revisited;
} mya_step_outputs;

/* A device environment over one task (replaces cuda::DeviceEnv, include/mymyr/cuda/env.hpp:89, and
 * rl::HostEnv, include/mymyr/rl/env.hpp:181). Uploads the task and counts the initial state's successors. The same
 * as mya_env_create_table over a table of one instance. */
int mya_env_create(mya_task* task, const mya_env_config* config, mya_env** out);
/* A device environment over a task table: `count` instances of one domain (TaskTable::create,
 * include/mymyr/rl/task_table.hpp:69-75), at most 65,536. Fails with the reference's message ("mymyr: TaskTable:
 * instance i is not of the domain of instance 0: ...", src/mymyr/rl/task_table.cpp:75-100) unless every instance has
 * instance 0's action schemas (names, arities) and predicates (names, arities, kinds) in the same order. A batch's rows
 * are at least the widest instance's words; the label width is the largest schema arity. The env keeps the tasks'
 * device images alive by reference: free the env before the tasks. */
int mya_env_create_table(mya_task* const* tasks, uint32_t count, const mya_env_config* config, mya_env** out);
/* A device environment over a task suite: instances of several domains (TaskSuite::group,
 * include/mymyr/rl/task_suite.hpp:1-30, 64): global task ids in the tasks' order, labels in each instance's own
 * domain's schema ids and objects, rows the widest instance's words, the label width the largest arity; the count
 * cache and schema masks have the most schemas of any instance (a narrower domain's columns past its own stay 0).
 * No domain check; otherwise as mya_env_create_table. */
int mya_env_create_suite(mya_task* const* tasks, uint32_t count, const mya_env_config* config, mya_env** out);
void mya_env_free(mya_env* env);
/* The env's instance sampler (EnvConfig::sampling, include/mymyr/rl/env.hpp:89-91; rl/sampling.hpp): `instances`
 * 0 turns it off, else it must be the table's instance count; m = 0 draws uniformly, else thresholds [m - 1]
 * (ascending) and indices [m] (instances) are mymyr.rl.InstanceSampler's arrays (host memory, copied). Autoresets
 * without next_task_ids, and resets with `sample`, of batches with reset counters draw from it. Errors follow
 * check_sampling (src/mymyr/rl/env.cpp:137-153). Not while a step of the env is in flight on another stream. */
int mya_env_set_sampling(mya_env* env, uint32_t instances, const uint32_t* thresholds, const int32_t* indices, uint32_t m);
/* The initial state's successor count and goal flag of an instance (DeviceEnv::initial_count,
 * include/mymyr/cuda/env.hpp:161-162). */
int mya_env_initial_count(const mya_env* env, uint32_t instance, uint32_t* count, uint8_t* goal);
/* HostEnv::reset (env.cpp:179-205, 223-255): rows with mask[i] != 0 (device, optional) to the initial state of their
 * instance (batch->task_ids, or with `sample` the rows' next sampled instances, written there; an id outside the
 * table resets the row into instance 0, writes 0 there and sets the sticky status, as DeviceEnv::reset,
 * include/mymyr/cuda/env.hpp:163-168), steps 0, at_goal and count (device, optional) of that initial state; draws
 * kept, reset counters advanced. With per-env goal masks, the instance's goal is written into them unless keep_goals,
 * in which case the given masks stay, at_goal is their test on the initial state, and masks that set fluent slots the
 * instance does not have set the sticky status (mya_env_check). Async on the stream. */
int mya_env_reset(mya_env* env, const mya_env_batch* batch, const uint8_t* mask, int32_t* count, int keep_goals, int sample,
                  void* stream);
/* HostEnv::step (env.cpp:530-548 / step_row_impl 351-528): actions (device, int64 [rows], optional: the random policy
 * when null); next_task_ids (device, int32 [rows], optional: the instance an autoresetting row restarts in; null: its
 * next sampled instance when the env has a sampler and the batch reset counters, else its own). Async on the stream;
 * device-side failures set the sticky status that mya_env_check reports: among them a task id outside the table in
 * batch->task_ids (over several instances the row is not stepped; a one-instance env steps every row as instance 0)
 * or in next_task_ids (an autoresetting row keeps its instance; DeviceEnv::step, include/mymyr/cuda/env.hpp:180-184).
 * Over several instances the rows are grouped by instance on the device first (a counting sort of task_ids into
 * env-owned scratch, allocated on the first call with a larger batch). */
int mya_env_step(mya_env* env, const mya_env_batch* batch, const mya_step_outputs* out, const int64_t* actions,
                 const int32_t* next_task_ids, void* stream);
/* The label-mode step (DeviceEnv::step(EnvBatch&, const StepOutputs&, rl::Labels, next_task_ids),
 * include/mymyr/cuda/env.hpp:185-188; rl::HostEnv's Labels step, src/mymyr/rl/env.cpp:376-426): row i's action is the
 * label (schema[i], binding[i * binding_stride + k] for k below the schema's arity; device int32 arrays), applied where
 * it is applicable in the row's state; elsewhere the row does not move and out->invalid is set (a row with no
 * applicable action is stuck first). out->count is the reached state's full successor count (the caller clamps it to
 * 0/1 for ActionSpace::Label). No host synchronization: capturable into a HIP graph like mya_env_step. Async. */
int mya_env_step_labels(mya_env* env, const mya_env_batch* batch, const mya_step_outputs* out, const int32_t* schema,
                        const int32_t* binding, uint32_t binding_stride, const int32_t* next_task_ids, void* stream);
/* Sizes the env's scratch for batches of up to `rows` rows and sets its kernels' LDS limits now (the reference device
 * env's reserve), so that later calls with such batches allocate nothing and make no runtime call besides kernel
 * launches, as HIP graph capture of them requires. */
int mya_env_reserve(mya_env* env, uint64_t rows);
/* New RNG key of the random policy and of the sampler (BatchedEnv.set_seed, python/mymyr/rl/torch/_batched.py:549-556),
 * written to the env's device word in stream order: steps enqueued before it draw with the old key, steps and graph
 * replays after it with the new one. The caller restarts the draw and reset counters if it wants fresh streams. */
int mya_env_set_seed(mya_env* env, uint64_t seed, void* stream);
/* The random policy's next choices without a step (DeviceEnv::random_actions, include/mymyr/cuda/env.hpp:189-192):
 * out[i] (device int64 [rows]) = the successor index a step would draw now for row i (batch->draws, the row's key and
 * env id), among the first max_actions successors (0: no limit), 0 where count[i] (device int32 [rows]) is 0. Async. */
int mya_env_random_actions(mya_env* env, const mya_env_batch* batch, const int32_t* count, uint32_t max_actions, int64_t* out,
                           void* stream);
/* Whether each row's current state is a goal of its instance (HostEnv::goal, src/mymyr/rl/env.cpp:272-281): the
 * per-env masks' test when the batch has them, else the instance's goal test; goal (device uint8 [rows]). Async. */
int mya_env_goal(mya_env* env, const mya_env_batch* batch, uint8_t* goal, void* stream);
/* HostEnv::clear_visited (include/mymyr/rl/env.hpp:210-211): the visited tables of the rows with mask[i] != 0 (device,
 * optional: all rows) hold their current states' keys only; the overflow status is kept. Async on the stream. */
int mya_env_clear_visited(mya_env* env, const mya_env_batch* batch, const uint8_t* mask, void* stream);
/* Reads and clears the sticky device status (synchronizes the env's status copy); -1 with a message if a step failed. */
int mya_env_check(mya_env* env);
/* Recomputes at_goal and the count cache (when the batch has one) of every row from its state and instance, after the
 * caller wrote states, task ids or goal masks directly (DeviceEnv::refresh, include/mymyr/cuda/env.hpp:170-174);
 * count (device, optional) receives the successor counts. Async on the stream. */
int mya_env_refresh(mya_env* env, const mya_env_batch* batch, int32_t* count, void* stream);

/* The true-atom slots of rows, ascending, -1 padded to max_atoms (State::slots, include/mymyr/state/state.hpp:96-101);
 * states [rows, words], out [rows, max_atoms] int32: device. Async on the stream; more atoms than max_atoms set the
 * env's sticky status (mya_env_check). */
int mya_encode_atoms(mya_env* env, const uint64_t* states, uint64_t rows, uint32_t words, int32_t* out, uint32_t max_atoms,
                     void* stream);
/* Per row and schema, whether some binding is applicable (rl::schema_masks, include/mymyr/rl/masks.hpp:9-11);
 * masks [rows, num_schemas] uint8, device; the rows are states of instance 0. Async on the stream. */
int mya_schema_masks(mya_env* env, const uint64_t* states, uint64_t rows, uint32_t words, uint8_t* masks, void* stream);

/* Successors of rows in canonical order, witness pruning off (Successors::generate, successors.hpp:154-248):
 * count [rows] i32; schema [rows, cap] i32; binding [rows, cap, label_width] i32 (-1 padded); succ [rows, cap, words]
 * u64. Device pointers (each optional but count). Entries past cap are counted, not written. Synchronous. */
int mya_successors(mya_task* task, const uint64_t* states, uint64_t rows, uint32_t words, int32_t cap, int32_t* count,
                   int32_t* schema, int32_t* binding, uint64_t* succ, void* stream);

/* rl::expand over one task (include/mymyr/rl/expand.hpp:1-130, ExpandOptions and Expansion): the flat CSR
 * expansion of rows [rows, words] (device). Device arrays of the expansion (each optional, null: not written):
 * succ [capacity, words] successor rows, parent / schema / index [capacity] int32, binding [capacity, label_width]
 * int32 (-1 past the schema's arity), goal / noop [capacity] uint8, succ_hash [capacity] uint64 (hash_state of the
 * successor), offsets [rows + 1] int32 (successors of row i are [offsets[i], offsets[i+1])). Rows past the capacity are
 * counted, not written: generated (all successors) > capacity is the overflow. With drop_noops the no-op successors of
 * a row are removed unless all of its successors are no-ops (then all are kept), index gives each kept row's position
 * in its row's full order, and an overflow reports the counts before dropping (offsets[rows] == total == generated).
 * Successors in canonical order, with witness pruning when asked. Synchronous: generated, total and words_needed are set on
 * return. */
typedef struct mya_expand_options
{
    int32_t canonical_order; /* must be 1 */
    int32_t witness_pruning; /* 1: one successor per effect-relevant binding (ExpandOptions::witness_pruning); 0 over a task table */
    int32_t validate;        /* reject rows with atoms past the task's slots */
    int32_t drop_noops;
} mya_expand_options;

typedef struct mya_expansion
{
    uint64_t capacity;
    uint32_t words;       /* words of the succ rows */
    uint32_t label_width; /* columns of binding (at least the largest schema arity) */
    uint64_t* succ;
    int32_t* parent;
    int32_t* schema;
    int32_t* binding;
    uint8_t* goal;        /* needs succ */
    int32_t* offsets;
    uint64_t* succ_hash;
    uint8_t* noop;
    int32_t* index;       /* required with drop_noops when capacity > 0 */
    uint64_t generated;   /* out: successors before dropping */
    uint64_t total;       /* out: kept successors */
    uint32_t words_needed; /* out: widest trimmed successor that did not fit `words` (0 if all fit) */
    uint32_t reserved;
} mya_expansion;

int mya_expand(mya_task* task, const uint64_t* states, uint64_t rows, uint32_t words, const mya_expand_options* options,
               mya_expansion* out, void* stream);
/* rl::expand over the env's task table (include/mymyr/rl/expand.hpp:1-130: a batch over a TaskTable): row i is a state
 * of instance task_ids[i] (device int32 [rows]; null only over a table of one instance), rows are at least the
 * widest instance's words, and the successors of row i are states of its instance, labelled with its objects. The
 * rows are grouped by instance on the device with the env's scratch. Same outputs, options and errors as mya_expand,
 * plus an error for a task id outside the table. Synchronous. */
int mya_env_expand(mya_env* env, const uint64_t* states, const int32_t* task_ids, uint64_t rows, uint32_t words,
                   const mya_expand_options* options, mya_expansion* out, void* stream);

/* No counterpart in the reference: for callers that cannot allocate device memory (code in tight serving loops,
 * harnesses that forbid hipMalloc). mya_expand over at most MYA_EXPAND_NOALLOC_MAX_ROWS rows with the same arguments,
 * outputs and errors, and no device allocation or free: the expansion's scratch (about 7 MiB) is a static device array
 * that each device the library runs on holds until the process ends. The task must already have its device image on
 * the current device (any earlier call with the task that reaches the device, e.g. mya_expand of 0 rows, uploads it).
 * The calls of one process share its one array per device and run one at a time (a process-wide lock; each process
 * that loads the library holds its own copies). Synchronous on `stream`, as mya_expand. */
#define MYA_EXPAND_NOALLOC_MAX_ROWS 262144u
int mya_expand_noalloc(mya_task* task, const uint64_t* states, uint64_t rows, uint32_t words, const mya_expand_options* options,
                       mya_expansion* out, void* stream);

/* PaddedExpansion (include/mymyr/rl/expand.hpp:162-181) without numeric and derived words: the [rows, k] view of a flat
 * expansion. Device arrays; a null array is not written. index [rows, k] (flat row, -1 padding), mask [rows, k],
 * count [rows] (the true successor counts, which may exceed k), succ [rows, k, words] (zero padding), schema (-1),
 * binding [rows, k, label_width] (-1), goal (0), succ_hash (0), noop (0), canonical (the flat index, -1). */
typedef struct mya_padded_expansion
{
    uint32_t k;
    uint32_t words;       /* at least the flat expansion's words when succ is written from flat succ rows */
    uint32_t label_width; /* at least the flat label width when binding is written from a flat binding */
    uint32_t reserved;
    int32_t* index;
    uint8_t* mask;
    int32_t* count;
    uint64_t* succ;
    int32_t* schema;
    int32_t* binding;
    uint8_t* goal;
    uint64_t* succ_hash;
    uint8_t* noop;
    int32_t* canonical;
    int32_t overflow;     /* out: a count above k, a successor past the flat capacity, or the flat expansion's overflow */
    int32_t reserved2;
} mya_padded_expansion;

/* rl::pad (include/mymyr/rl/expand.hpp:183-186, src/mymyr/rl/expand.cpp:799-873): scatters the flat expansion of `rows`
 * states (device arrays of `flat` as mya_expand wrote them; offsets [rows + 1] required; capacity, generated, total,
 * words_needed as returned) into `out`. An array of `out` whose flat source is null is filled with its padding.
 * Synchronous: out->overflow is set on return. */
int mya_pad(const mya_expansion* flat, uint64_t rows, mya_padded_expansion* out, void* stream);

/* rl::visited_mask (include/mymyr/rl/visited.hpp:63-74; the device launch of include/mymyr/cuda/rl_ops.hpp:53-58, the
 * torch op mymyr::visited_mask of python/mymyr/rl/torch/_ops.py:464-486): out[j] = whether succ_hash[j] is in the
 * visited table of row parent[j], or of rows[parent[j]] when `rows` ([parents] entries) is given (without it parents
 * = table_rows). table [table_rows, capacity] and count [table_rows] as an env's visited tables hold them; capacity a
 * power of two in [2, 2^20]. -1 is padding; a parent or mapped row outside [-1, parents) or [-1, table_rows) reads as
 * not visited. Device arrays; asynchronous on `stream`. */
int mya_visited_mask(const uint64_t* table, const int32_t* count, uint64_t table_rows, uint32_t capacity, const uint64_t* succ_hash,
                     const int32_t* parent, const int32_t* rows, uint64_t parents, uint64_t size, uint8_t* out, void* stream);

/* The index form of label actions (HostEnv::step with Labels, src/mymyr/rl/env.cpp:376-426): actions[i] = the position
 * of row i's label (label_schema [rows], label_binding [rows, stride], stride >= label_width; columns past the
 * schema's arity are ignored) in the row's successors of a flat expansion in canonical order (offsets [rows + 1],
 * schema, binding [., label_width] as mya_env_expand writes them without drop_noops), or -1 when the label is not
 * applicable. An env step with these actions is the reference's label step, its counts clamped to 0/1. Device arrays;
 * asynchronous on `stream`. */
int mya_label_actions(const int32_t* offsets, const int32_t* schema, const int32_t* binding, uint32_t label_width, uint64_t rows,
                      const int32_t* label_schema, const int32_t* label_binding, uint32_t stride, int64_t* actions, void* stream);

/* ---------------------------------------------------------------------------------------------------------- BrFS */

/* Options of brfs(Task, BrfsOptions) (include/mymyr/search/brfs.hpp:62-101) that the device search takes. */
typedef struct mya_brfs_options
{
    uint32_t max_depth;      /* expand only states of depth < max_depth (UINT32_MAX: unbounded) */
    int32_t witness_pruning; /* reference default 1 */
    uint64_t max_states;     /* stop (OutOfStates) once this many states are stored (UINT64_MAX: unbounded) */
    uint64_t max_expanded;   /* stop before the expansion that would exceed this many (UINT64_MAX: unbounded) */
    int32_t stop_at_goal;    /* reference default 1 */
    int32_t fingerprint;     /* compute BrfsResult::fingerprint */
    uint64_t chunk;          /* candidates per device batch (0: automatic) */
    uint64_t memory_states;  /* state capacity when max_states is unbounded (0: 2^26) */
    int32_t timings;         /* time each kernel class with HIP events (mya_brfs_result.kernel_ms) */
    int32_t reserved;
    /* BrfsOptions::start and blocked_states (brfs.hpp:82-83): host rows of `words` words (the task's row words,
     * mya_task_info.words). start (null: the task's initial state) replaces the initial state; the blocked_count
     * rows are never stored: a successor equal to one of them counts as generated and pruned (the start state is
     * exempt: it is stored even if blocked). */
    const uint64_t* start;
    const uint64_t* blocked;
    uint64_t blocked_count;
    uint32_t words;
    /* BrfsOptions::max_seconds and cancel (brfs.hpp:97-98): with timed != 0 the search stops with status 3
     * (OutOfTime) once max_seconds of wall time have passed (max_seconds <= 0: before the first expansion); cancel
     * (null: none) is a flag that another thread sets nonzero to stop the search with status 4 (Cancelled). Both are
     * checked between device batches (the reference checks every 8 expansions), so a stopped search's counts stop at
     * a batch boundary. */
    int32_t timed;
    double max_seconds;
    const volatile int32_t* cancel;
    /* BrfsOptions::goal (brfs.hpp:87-91) as GoalSpec::AnyOf of ground conditions (include/mymyr/search/control.hpp:93-118,
     * search::any_of, include/mymyr/search/goal.hpp:35): with goal_kind 1 a state is a goal iff one of goal_count
     * conditions holds in it (goal_kind 0: the task's goal). Condition k's literals are the records
     * [goal_offsets[k], goal_offsets[k + 1]) of goal_literals, MYA_GOAL_LITERAL_INTS int32 each: predicate, positive
     * (0 or 1), the number of objects, then the objects. As the reference resolves them (src/mymyr/search/goal.cpp:14-60):
     * a static literal is decided against the task's static facts (a false one leaves its condition out), a fluent atom
     * outside its predicate's domains or without a slot makes a positive literal's condition impossible (left out) and
     * a negative literal true (dropped). Host arrays. An invalid literal (predicate, object count or object out of
     * range) is an error. */
    int32_t goal_kind;
    uint32_t goal_count;
    const uint32_t* goal_offsets;
    const int32_t* goal_literals;
    /* BrfsOptions::observer and progress_interval (brfs.hpp:99-100; the events of search::SearchObserver,
     * include/mymyr/search/control.hpp:157-186): null for none. progress_interval 0 means the reference's default,
     * 2^16 expansions. */
    const struct mya_search_observer* observer;
    uint64_t progress_interval;
    /* BrfsOptions::layers (search::LayerOrdering, include/mymyr/search/layer_ordering.hpp:63-113). layer_kind: 0 queue
     * (the plain BrFS), 1 in order, 2 reverse, 3 randomized (SplitMix64 of layer_seed), 4 goal count (by the task goal's
     * satisfied literals, most first unless prefer_fewer_satisfied_goals), 5 scored (layer_scorer: scores[i] of the
     * layer's host rows [n, words], lower first; NaN is an error). With an ordered kind each next layer is reordered
     * before it is expanded (state ids follow the expansion order; the start layer keeps its order). max_next_layer_states
     * (0: no limit) cuts a layer's generation once the next layer holds that many states, dropping the rest of the
     * layer; beam_width (0: no beam) keeps the first beam_width states of each ordered layer, the others stay stored
     * and are never expanded; randomize_ties breaks equal scores by SplitMix64 tokens drawn in generation order. The
     * reference's checks apply (check_layers, layer_ordering.hpp:117-134); beam_novelty is accepted as 0 (all tested)
     * or 1 (survivors only, the same in a BrFS), relaxed survivors-only (2) is refused. */
    int32_t layer_kind;
    int32_t prefer_fewer_satisfied_goals;
    uint64_t layer_seed;
    uint32_t max_next_layer_states;
    uint32_t beam_width;
    int32_t randomize_ties;
    int32_t beam_novelty;
    void (*layer_scorer)(void* user, const uint64_t* rows, uint64_t n, uint32_t words, double* scores);
    void* layer_scorer_user;
    /* BrfsOptions::goal as GoalSpec::Custom (include/mymyr/search/control.hpp:99-121): goal_test(user, rows, n, words,
     * out) sets out[i] to 1 when host row i ([n, words], the task's slot layout) is a goal state and to 0 otherwise;
     * a nonzero return stops the search with an error. It decides instead of the task's goal and of goal_kind (which
     * must be 0). The ground search calls it on each batch of parents it counts, the lifted one on each layer before
     * expanding it; a state is tested before its expansion, as the reference tests a state popped for expansion
     * (src/mymyr/search/brfs.cpp:332-339). Null: none. */
    int32_t (*goal_test)(void* user, const uint64_t* rows, uint64_t n, uint32_t words, uint8_t* out);
    void* goal_test_user;
} mya_brfs_options;
#define MYA_GOAL_LITERAL_INTS 9

/* search::SearchStatistics (include/mymyr/search/control.hpp:129-139): the counts of a layer (on_pass), of the search
 * so far (on_progress) or of the whole search (on_end, with pruned); seconds of wall time since the search (on_pass:
 * the layer) started. memory_bytes is 0 in events, as in the reference. */
typedef struct mya_search_statistics
{
    uint64_t expanded;
    uint64_t generated;
    uint64_t states;
    uint64_t pruned;
    double seconds;
    uint64_t memory_bytes;
} mya_search_statistics;

/* The events of search::SearchObserver (include/mymyr/search/control.hpp:157-186), each on the thread that called
 * mya_brfs; a null function is skipped. on_start: the start state's row (`words` words); on_pass: the end of BrFS layer
 * `layer` (0 first) with that layer's counts; on_progress: before a device batch once `progress_interval` more states
 * were expanded (the reference asks every progress_interval expansions; the device search asks at its batch
 * boundaries), returning 0 stops the search with status 4 (Cancelled); on_solution: the plan (schemas[i],
 * bindings[i * label_width ..], -1 padded) and its cost; on_end: the final status and statistics.
 * on_expand (state `id` expanded), on_generate (a transition of `parent` by the action (schema, binding[arity]) to
 * `child`, UINT64_MAX when the successor got no id (a blocked state), with the successor's row and whether the
 * transition entered it) and on_prune (a blocked successor, after its on_generate) come in the reference's order,
 * state by state and successor by successor, but a device batch at a time once the batch is confirmed: with any of
 * them set, the search brings each batch's parents, transitions and successor rows to the host (slower; for
 * analysis and tests). on_transition is not sent by a BrFS, as in the reference. */
typedef struct mya_search_observer
{
    void* user;
    void (*on_start)(void* user, const uint64_t* state, uint32_t words);
    void (*on_pass)(void* user, uint32_t layer, const mya_search_statistics* pass);
    int32_t (*on_progress)(void* user, const mya_search_statistics* so_far);
    void (*on_solution)(void* user, const int32_t* schemas, const int32_t* bindings, uint32_t length, uint32_t label_width,
                        double cost);
    void (*on_end)(void* user, int32_t status, const mya_search_statistics* total);
    void (*on_expand)(void* user, uint64_t id, const uint64_t* state, uint32_t words);
    void (*on_generate)(void* user, uint64_t parent, int32_t schema, const int32_t* binding, uint32_t arity, uint64_t child,
                        const uint64_t* state, uint32_t words, int32_t is_new);
    void (*on_prune)(void* user, uint64_t parent, int32_t schema, const int32_t* binding, uint32_t arity, const uint64_t* state,
                     uint32_t words);
} mya_search_observer;

/* BrfsResult fields (include/mymyr/search/brfs.hpp:103-138). status: the reference's SearchStatus codes
 * (0 solved, 1 exhausted, 2 out of states, 3 out of time, 4 cancelled, 5 failed, 6 unsolvable). */
typedef struct mya_brfs_result
{
    int32_t status;
    int32_t solved;
    int32_t exhausted;
    uint32_t layers;
    uint64_t states;
    uint64_t expanded;
    uint64_t generated;
    uint64_t goal_states;
    uint64_t fingerprint;
    int64_t first_goal; /* id of the first goal state tested (-1: none) */
    double search_s;    /* wall time of the whole call */
    double device_s;    /* wall time from the start state's insert to the end of the search */
    /* per kernel class (0 count, 1 emit, 2 insert, 3 unused, 4 rank, 5 compact, 6 other, 7 unused): summed HIP-event
     * durations (with options.timings), algorithmic bytes and launches */
    double kernel_ms[8];
    uint64_t kernel_bytes[8];
    uint64_t kernel_launches[8];
    uint64_t pruned;       /* successors not stored because they are blocked states */
    uint64_t memory_bytes; /* device bytes of the search's buffers (state set, arena, nodes, chunk and layer arrays) */
    uint32_t words;        /* the task's state words at the end (BrfsResult::words; lazy slots: after interning) */
    uint32_t fluent_slots; /* assigned fluent atom slots at the end (BrfsResult::fluent_slots) */
    uint32_t threads_used; /* host threads the search ran on (BrfsResult::threads_used): 1, the calling thread */
    uint32_t reserved2;
    char store[16];        /* the store (BrfsResult::store): "device" (the device state set), "none" when nothing was searched */
    char message[256];     /* why the search stopped early or ran otherwise than asked (BrfsResult::message); "" if neither */
} mya_brfs_result;

/* The plan of a solved search: BrfsResult::plan, cost and goal_state (include/mymyr/search/brfs.hpp:118-131), the
 * actions from the start state to the first goal state tested, rebuilt from per-state node records (the first
 * discovery of each state: its parent and action, src/mymyr/search/brfs.cpp:235-268). Host arrays, caller-owned;
 * null arrays are not written. */
typedef struct mya_brfs_plan
{
    int32_t* schema;       /* [cap] the actions' schemas */
    int32_t* binding;      /* [cap, label_width] their objects, -1 past a schema's arity */
    uint32_t cap;          /* actions the arrays hold */
    uint32_t label_width;  /* columns of binding */
    uint64_t* goal_state;  /* [goal_cap] the goal state's words */
    uint32_t goal_cap;
    uint32_t length;       /* out: actions of the plan (0 unless solved; those past cap are not written) */
    uint32_t goal_words;   /* out: words of the goal state (0 unless solved) */
    uint32_t reserved;
    double cost;           /* out: the plan's cost (unit action costs: its length); 0 unless solved */
} mya_brfs_plan;

/* Layer-synchronous BrFS on the current device (replaces brfs(), include/mymyr/search/brfs.hpp:140, and
 * cuda::brfs, include/mymyr/cuda/brfs.hpp:89-123). layer_counts [cap, 3] (host, optional) receives
 * {expanded, generated, new} per expanded layer; plan (optional) receives the plan of a solved search. Returns the
 * number of layers, or -1. Synchronous. */
int mya_brfs(mya_task* task, const mya_brfs_options* options, mya_brfs_result* result, uint64_t* layer_counts,
             uint32_t cap, mya_brfs_plan* plan);

/* ---------------------------------------------------------------------------------------------------------- DLPack */

/* Device arrays handed to other frameworks without a copy (replaces the reference's DLArray export,
 * python/src/arrays.cpp:100-235, and its stream handoff, python/src/dlpack.hpp:1-94). The structs below have the
 * layout of DLPack 1.x's DLDevice, DLDataType, DLTensor, DLManagedTensor (legacy) and DLManagedTensorVersioned,
 * under this library's names so that the header can sit beside a caller's own dlpack.h. */
#define MYA_DL_ROCM 10 /* kDLROCM */
#define MYA_DL_INT 0
#define MYA_DL_UINT 1
#define MYA_DL_FLOAT 2
#define MYA_DL_BOOL 6
#define MYA_DL_FLAG_READ_ONLY 1u /* DLPACK_FLAG_BITMASK_READ_ONLY */
#define MYA_DL_MAJOR 1
#define MYA_DL_MINOR 0
/* Consumer streams follow the DLPack convention for ROCm: -1 no synchronization, 0 the default stream, any other
 * value a hipStream_t. */
#define MYA_DL_STREAM_NONE (-1)

typedef struct
{
    int32_t device_type;
    int32_t device_id;
} mya_dl_device;

typedef struct
{
    uint8_t code;
    uint8_t bits;
    uint16_t lanes;
} mya_dl_dtype;

typedef struct
{
    void* data;
    mya_dl_device device;
    int32_t ndim;
    mya_dl_dtype dtype;
    int64_t* shape;
    int64_t* strides; /* in elements */
    uint64_t byte_offset;
} mya_dl_tensor;

typedef struct mya_dl_managed
{
    mya_dl_tensor dl_tensor;
    void* manager_ctx;
    void (*deleter)(struct mya_dl_managed* self);
} mya_dl_managed;

typedef struct
{
    uint32_t major;
    uint32_t minor;
} mya_dl_version;

typedef struct mya_dl_managed_versioned
{
    mya_dl_version version;
    void* manager_ctx;
    void (*deleter)(struct mya_dl_managed_versioned* self);
    uint64_t flags;
    mya_dl_tensor dl_tensor;
} mya_dl_managed_versioned;

/* Device memory owned by the library, reference-counted (the reference's DLArray blocks, python/src/arrays.cpp): the
 * creator holds one reference and every exported tensor another; the memory is freed when the last is dropped.
 * Contents start undefined. Allocated on the current device. */
typedef struct mya_buffer mya_buffer;
int mya_buffer_create(uint64_t bytes, mya_buffer** out);
void* mya_buffer_data(const mya_buffer* buffer);
uint64_t mya_buffer_bytes(const mya_buffer* buffer);
/* Drops the caller's reference. */
void mya_buffer_release(mya_buffer* buffer);

/* Exports a view of a buffer: element type (code, bits), ndim (0..8) extents `shape` and element strides `strides`
 * (null: row-major), starting byte_offset bytes into the buffer (aligned to the element size; folded into the data
 * pointer). Every element of the view must lie inside the buffer; strides must be non-negative. flags: 0 or
 * MYA_DL_FLAG_READ_ONLY (versioned only). Work on producer_stream (a hipStream_t) is made to precede later work on
 * consumer_stream (see MYA_DL_STREAM_NONE). *out receives a mya_dl_managed_versioned* (versioned != 0) or a
 * mya_dl_managed*, which holds a reference to the buffer until its deleter is called. */
int mya_buffer_export(mya_buffer* buffer, uint64_t byte_offset, uint8_t code, uint8_t bits, int32_t ndim,
                      const int64_t* shape, const int64_t* strides, uint64_t flags, void* producer_stream,
                      int64_t consumer_stream, int versioned, void** out);

/* Exports the stored rows of a state set as a uint64 [size, words] tensor (waits for the set's last insert, like
 * mya_hashset_size). The tensor holds a reference to the set: it stays valid after mya_hashset_free until its deleter
 * runs; a later mya_hashset_clear makes its contents undefined. */
int mya_hashset_export_rows(mya_hashset* set, uint64_t flags, int64_t consumer_stream, int versioned, void** out);

/* For Python hosts: a PyCapsule destructor for capsules named "dltensor" or "dltensor_versioned" that hold a tensor
 * exported above. It calls the tensor's deleter unless a consumer has taken the tensor (renamed the capsule), as the
 * DLPack Python protocol specifies. It finds the CPython API in the running process and does nothing outside one. */
void mya_dlpack_capsule_destructor(void* capsule);

#ifdef __cplusplus
}
#endif
#endif
