#pragma once
// Device-resident open-addressing state set: rows of W u64 words in an arena (ids in insertion order), one u64 table
// entry per slot = (tag32 << 32) | code, code = id + 1 (settled) or kPending | epoch | candidate (a candidate of a
// batch: pending while that batch is inserted, then standing for the id the batch's epoch maps it to).
//
// A batch insert keeps the reference's id rule (include/mymyr/cuda/state_set.hpp:2-18, the CPU stores'
// first-discovery ids: src/mymyr/search/brfs.cpp:1657-1780): among equal candidates of one batch the smallest
// candidate index wins (64-bit atomicMin on the pending entry), and new ids follow candidate order (an exclusive scan
// of the winner flags). The probe hash (set_hash) is the public state hash (hash_state) for rows of at most 8 words
// and an order-free sum of mixed words above (set_hash_wide); slot = fastrange of its low 32 bits over the capacity,
// tag = its high 32 bits, linear probing.
//
// A batch is three steps on one stream: probe (group of lanes per row: hash, probe, CAS or atomicMin, loser flags),
// the winner list (a scan of the flags: winner w gets id = the set's size + w, recorded as winner bits and a first id
// per 64 candidates in the batch's epoch of id_map), and compaction over the winners (rows into the arena; the entries keep their epoch codes). The set's size lives on the device in two words used alternately (the scan of a batch
// writes next = current + winners), so batches need no host synchronization; the host copy is refreshed by the
// calls that synchronize.

#include "state_set_device.hpp"

#include <hip/hip_runtime.h>

namespace mya
{
struct StateSet
{
    StateSetView v{};
    u64 max_states = 0;
    u64 size = 0;       // host copy of the size (exact after a synchronizing call)
    u64 batch_cap = 0;
    u64* cand_slot = nullptr;  // [batch_cap] probe result per candidate (state_set_device.hpp encodings)
    u8* flags = nullptr;       // [batch_cap] winner flag bytes, 1 at rest
    u32* list = nullptr;       // [batch_cap] the winners' candidate indices in order (winner w gets id size + w)
    u64* scan_scratch = nullptr;
    u64* d_size = nullptr;     // [2] the size, alternating per batch
    u32* d_status = nullptr;   // sticky kStatus* bits
    u64* h_pinned = nullptr;   // [4] size before, size after, status of the last insert
    int cur = 0;               // d_size[cur] is the current size
    hipStream_t last = nullptr;
    WinnerBlock* id_map = nullptr;  // [epochs, winner_blocks(batch_cap)] winner ids per epoch (v.id_map)
    u64* id_limit = nullptr;        // [epochs] the epochs' cut ids (v.id_limit)
    u32 epochs = 0;            // epochs in rotation (at most kMaxEpochs)
    u64 batches = 0;           // epochs taken since the last clear or settling pass
};

/// Allocates a set for up to max_states rows of `words` words at the given maximum load: capacity =
/// (max_states + pending) / load, where `pending` bounds the candidates a batch may hold as pending entries beyond
/// max_states (a driver that cuts a batch at max_states after probing it).
void state_set_create(StateSet& s, u64 max_states, u32 words, double max_load, u64 batch_cap, hipStream_t stream,
                      u64 pending = 0);
/// Frees the set's device memory: with a stream, in that stream's order (the blocks are reused only after the work
/// queued on it so far, which must include every use of the set); without one, after the device has finished all work.
void state_set_destroy(StateSet& s, hipStream_t stream = nullptr);
/// Clears the set (size 0) without freeing.
void state_set_clear(StateSet& s, hipStream_t stream);

/// Starts a batch: takes the next free epoch into s.v.epoch (when all are taken, one pass over the table settles every
/// candidate-coded entry to id + 1 first). Drivers with their own probe kernels call it before each batch's probe.
void state_set_begin_batch(StateSet& s, hipStream_t stream);

/// Inserts rows [n, W] (device), in batches of at most batch_cap rows, asynchronously on the stream. Optional outputs:
/// ids [n] (i64 id of each row's state; -1 for a row past the capacity), is_new [n]. With new_count (host) the call
/// synchronizes and returns the number of new states, throwing on a full set or table. Without it, a capacity
/// overflow is reported by the next synchronizing call (state_set_sync); the set must then be cleared.
void state_set_insert(StateSet& s, const u64* rows, u64 n, i64* ids, u8* is_new, u64* new_count, hipStream_t stream);

/// Waits for the set's last insert and refreshes s.size; throws if a batch overflowed the set or its table.
void state_set_sync(StateSet& s);

/// Device words of the current and the next size, for drivers that run their own probe and compaction kernels: the
/// scan of a batch reads the current size and writes the next; state_set_flip then makes the next current.
inline u64* state_set_size_now(StateSet& s) { return s.d_size + s.cur; }
inline u64* state_set_size_next(StateSet& s) { return s.d_size + (s.cur ^ 1); }
inline void state_set_flip(StateSet& s) { s.cur ^= 1; }

/// The winners of a batch of n candidates in order into s.list (losers' flags reset), their ids into the batch's
/// epoch of id_map, is_new[j] (optional) the flags, and next size = size + winners.
void state_set_rank(StateSet& s, u64 n, hipStream_t stream, u8* is_new = nullptr);

/// A cut inside the last ranked batch whose search goes on (a BrFS layer cut by max_next_layer_states): only the
/// batch's winners below `size` are stored, so the set's size becomes `size` and the table entries of the others
/// (pending codes of the batch's epoch) stand for no state from now on (the epoch's ids from `size` on are cut).
void state_set_cut(StateSet& s, u64 size, hipStream_t stream);

/// The probe of a batch begun with state_set_begin_batch over candidate rows [m, words] (device) that the caller produced:
/// a stored equal row drops a candidate, equal candidates keep the smallest index, the others take pending entries
/// (the losers' flags are cleared). state_set_rank and the caller's compaction follow. With `blocked`, a candidate equal
/// to a blocked state is dropped first (flag cleared, blocked->hit[j] = 1; every other candidate's hit byte is 0).
void state_set_probe(StateSet& s, const u64* rows, u64 m, hipStream_t stream, const BlockedView* blocked = nullptr,
                     u64* cand_slot = nullptr);

/// After a batch's rank and compaction: ids[j] = the id of candidate j's state (its own as a winner, the equal one's
/// otherwise; -1 when it got none: blocked, or past a cut), from the probe results cand_slot [n] (blocked candidates'
/// entries are not read by callers).
void state_set_resolve_ids(StateSet& s, const u64* cand_slot, u64 n, i64* ids, hipStream_t stream);

/// hash_state of every row (a group of lanes per row).
void launch_hash_rows(const u64* rows, u64 n, u32 words, u64* out, hipStream_t stream);

/// Fills n u32 words with v.
void launch_fill_u32(u32* p, u64 n, u32 v, hipStream_t stream);

/// Threads of launch_random_ops (its sink's length).
constexpr u64 kRandomOpsThreads = u64{1} << 20;
/// n random 8-byte operations (0 load, 1 CAS, 2 atomicMin, 3 store) on table [words] (a power of two), results into
/// sink [kRandomOpsThreads]: the random-access rates of the probes' memory operations.
void launch_random_ops(u64* table, u64 words, u64 n, int kind, u64 seed, u64* sink, hipStream_t stream);

/// Rows [start, start + count) of the seeded dedup stream (the dedup workload's synthetic input).
void launch_dedup_rows(u64 start, u64 count, u32 words, u64 seed, double dup, u64* out, hipStream_t stream);
}  // namespace mya
