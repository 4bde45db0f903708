#pragma once
// Device-resident open-addressing state set: rows of W u64 words in an arena (ids in insertion order), one u64 table
// entry per slot = (tag32 << 32) | code, code = id + 1 (settled) or kPending | candidate (pending within a batch).
//
// A batch insert keeps the reference's id rule (include/mymyr/cuda/state_set.hpp:2-18, the CPU stores'
// first-discovery ids: src/mymyr/search/brfs.cpp:1657-1780): among equal candidates of one batch the smallest
// candidate index wins (64-bit atomicMin on the pending entry), and new ids follow candidate order (an exclusive scan
// of the winner flags). The probe hash is the public state hash (hash_state); slot = fastrange of its low 32 bits over
// the capacity, tag = its high 32 bits, linear probing.

#include "device_common.hpp"

namespace mya
{
constexpr u32 kPending = 0x80000000u;

/// Slot of a state hash: fastrange of its low 32 bits over the capacity (the tag is the high 32 bits).
__host__ __device__ inline u64 slot_of_hash(u64 h, u64 cap) { return ((h & 0xFFFFFFFFull) * cap) >> 32; }

struct StateSetView
{
    u64* table;
    u64 capacity;
    u64* arena;   // [max_states, W]
    u64* hashes;  // [max_states]
    u32 words;
};

struct StateSet
{
    StateSetView v{};
    u64 max_states = 0;
    u64 size = 0;  // host copy, updated by insert
    // batch scratch
    u64 batch_cap = 0;
    u64* cand_slot = nullptr;  // [batch_cap]
    u32* flags = nullptr;      // [batch_cap]
    u64* offsets = nullptr;    // [batch_cap]
    u64* hashes_tmp = nullptr; // [batch_cap]
    u64* scan_scratch = nullptr;
    u64* d_total = nullptr;    // [2]: new count, spare
    u32* d_status = nullptr;
    u64* h_pinned = nullptr;   // pinned host word for the new count
};

/// Allocates a set for up to max_states rows of `words` words at the given maximum load: capacity =
/// (max_states + pending) / load, where `pending` bounds the candidates a batch may hold as pending entries beyond
/// max_states (a driver that cuts a batch at max_states after probing it).
void state_set_create(StateSet& s, u64 max_states, u32 words, double max_load, u64 batch_cap, hipStream_t stream,
                      u64 pending = 0);
void state_set_destroy(StateSet& s);
/// Clears the set (size 0) without freeing.
void state_set_clear(StateSet& s, hipStream_t stream);

/// Inserts rows [n, W] (device). hashes: the rows' state hashes (device, optional: computed when null). Optional
/// outputs: ids [n] (i64 id of each row's state), is_new [n]. new_count: host out (synchronizes the stream).
/// Throws on capacity overflow (the set is left with the rows it had).
void state_set_insert(StateSet& s, const u64* rows, const u64* hashes, u64 n, i64* ids, u8* is_new, u64* new_count,
                      hipStream_t stream);

/// Launch pieces of an insert for drivers that keep the batch on the device (BrFS): probe (after which winners are
/// those whose entry holds their candidate), flags + scan, and compaction at base id `base`. Candidate rows and
/// hashes stay readable until compaction ends. With `mask` (device, optional) the probe takes only the candidates j
/// with mask[j] != 0; the others are neither inserted nor winners (their rows and hashes are not read).
void state_set_probe(StateSet& s, const u64* rows, const u64* hashes, u64 n, hipStream_t stream, const u8* mask = nullptr);
void state_set_rank(StateSet& s, u64 n, hipStream_t stream);  // d_total[0] = winners
void state_set_compact(StateSet& s, const u64* rows, const u64* hashes, u64 n, u64 base, u64 limit, i64* ids, u8* is_new,
                       hipStream_t stream);

/// hash_state of every row (thread per row).
void launch_hash_rows(const u64* rows, u64 n, u32 words, u64* out, hipStream_t stream);

/// Rows [start, start + count) of the seeded dedup stream (the dedup workload's synthetic input).
void launch_dedup_rows(u64 start, u64 count, u32 words, u64 seed, double dup, u64* out, hipStream_t stream);
}  // namespace mya
