#pragma once
// Device building blocks of the state set, shared by the generic batch insert (rows in a buffer) and the BrFS insert
// (rows recomputed from (parent, action) records): a row is handled by a group of G lanes, lane q of the group holding
// the word pairs p = k * G + q (k < K) of the row as (word 2p, word 2p + 1). A random row access is then one
// coalesced request of the whole group, and the group's lanes follow one control path (every branch depends on
// group-uniform values only).
//
// The table hash of rows of at most 8 words is the public hash_state (include/mymyr/core/hash.hpp:38-60) over the
// trimmed words, chained over the pairs in order with the pair broadcast from its lane (wider rows: set_hash_wide);
// the table probe keeps the reference's id rule (include/mymyr/cuda/state_set.hpp:2-18): among equal candidates the
// smallest candidate index wins (64-bit atomicMin on the pending entry), new ids follow candidate order.
//
// Entries are never rewritten after the probe: a batch's pending entries keep the candidate code of their winner, and
// the batch's epoch (one of up to 64, 6 bits of the code) maps candidate indices to ids through its winner blocks,
// written by the winner list. When every epoch is taken, one streaming pass settles all entries to id + 1. This trades
// the random 8-byte rewrite of every new state's entry (a read-modify-write of a memory line) for a 16-byte winner-block
// read on the probes that compare against a recent state.
//
// Winner flags need no second pass over the table: every candidate starts at flag 1 (the winner list of the previous
// batch resets the zeros), and only zeros are written during the probe: a candidate equal to a stored state, a candidate
// that finds a smaller equal one already pending (no atomic: a pending entry only decreases), and the larger index of
// every atomicMin exchange between two pending candidates. Every candidate but the smallest of its content is zeroed
// by one of these, so the flags that stay 1 are exactly the winners. Atomics (about 3x slower than random reads) are
// thus spent only on new contents (one CAS) and on the rarer case of a smaller index arriving after a larger one. Rows of
// other candidates are never read back from memory written in the same kernel (a row source recomputes them), so no
// release fence is needed between a row write and the entry that publishes it.

#include "device_common.hpp"
#include "scan.hpp"

namespace mya
{
constexpr u32 kPending = 0x80000000u;  // a candidate-coded entry: epoch and candidate index instead of id + 1
constexpr u32 kJBits = 25;             // candidate index bits of a candidate-coded entry (batches of at most 2^25)
constexpr u32 kJMask = (1u << kJBits) - 1;
constexpr u32 kEpochMask = (1u << (31 - kJBits)) - 1;
constexpr u32 kMaxEpochs = kEpochMask + 1;
constexpr u64 kMaxBatch = u64{1} << kJBits;
constexpr u32 kNoSlot = 0xFFFFFFFFu;
constexpr u64 kProbeFailed = ~u64{0};

/// The entry code of candidate j of the batch of the given epoch.
__host__ __device__ inline u32 cand_code(u32 epoch, u64 j) { return kPending | (epoch << kJBits) | static_cast<u32>(j); }
__host__ __device__ inline u32 code_epoch(u32 code) { return (code >> kJBits) & kEpochMask; }

/// Slot of a state hash: fastrange of its low 32 bits over the capacity (the tag is the high 32 bits).
__host__ __device__ inline u64 slot_of_hash(u64 h, u64 cap) { return ((h & 0xFFFFFFFFull) * cap) >> 32; }

struct StateSetView
{
    u64* table;
    u64 capacity;
    u64* arena;         // [max_rows, words]
    u32 words;
    u32 epoch;          // the epoch of the batch being inserted
    const WinnerBlock* id_map;  // [epochs, id_stride]: the ids of each epoch's batch winners (written by the winner list)
    u64 id_stride;              // winner blocks per epoch
    const u64* id_limit;        // [epochs]: ids at or past an epoch's limit were cut (they stand for no stored state)
    u64 max_rows;       // rows of the arena: ids at or past it were never stored
};

/// The id candidate j of epoch e's batch (a winner) took, or kCutId past the epoch's cut.
constexpr u64 kCutId = 0x7FFFFFFEu;  // past every arena (sets hold fewer than 2^31 - 2 states): matches nothing
__host__ __device__ inline u64 epoch_winner_id(const WinnerBlock* id_map, u64 stride, const u64* id_limit, u32 e, u32 j)
{
    const u64 id = winner_id(id_map[e * stride + (j >> 6)], j);
    return id < id_limit[e] ? id : kCutId;
}

/// The id a committed entry code stands for: id + 1 for settled codes, the epoch's winner id for candidate codes.
__device__ __forceinline__ u64 committed_id(const StateSetView& s, u32 code)
{
    return (code & kPending) ? epoch_winner_id(s.id_map, s.id_stride, s.id_limit, code_epoch(code), code & kJMask)
                             : static_cast<u64>(code) - 1;
}

/// cand_slot encodings written by the probe: (tag << 32) | slot for a candidate that holds or held a pending entry;
/// (id << 32) | kNoSlot for a candidate equal to the stored state `id`; kProbeFailed when the table was full.
__host__ __device__ inline bool cand_is_stored(u64 cs) { return static_cast<u32>(cs) == kNoSlot; }

template<int G, int K>
struct Slice
{
    u64 lo[K], hi[K];  // pair k * G + q: words 2p (lo) and 2p + 1 (hi)
};

/// Rows above kLongRowWords words (K = 0) stay in memory: the slice is the row's address, and the group's lanes stride
/// over its word pairs wherever the row is compared, hashed or copied (lane q: pairs q, q + G, ...).
constexpr u32 kLongRowWords = 2048;
template<int G>
struct Slice<G, 0>
{
    const u64* row;
    u32 W;
};

/// Lane q's words of a row of W words (zeros past W).
template<int G, int K>
__device__ __forceinline__ void load_row(const u64* __restrict__ row, u32 W, u32 q, Slice<G, K>& s)
{
    if constexpr (K == 0)
    {
        s.row = row;
        s.W = W;
    }
    else
    {
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            const u32 w = 2 * (k * G + q);
            if (w + 1 < W && (W & 1) == 0)
            {
                const ulonglong2 v = *reinterpret_cast<const ulonglong2*>(row + w);
                s.lo[k] = v.x;
                s.hi[k] = v.y;
            }
            else
            {
                s.lo[k] = w < W ? row[w] : 0;
                s.hi[k] = w + 1 < W ? row[w + 1] : 0;
            }
        }
    }
}

template<int G, int K>
__device__ __forceinline__ void store_row(u64* __restrict__ row, u32 W, u32 q, const Slice<G, K>& s)
{
    if constexpr (K == 0)
    {
        // W (even for these widths: multiples of 64 words) copied pair by pair across the group
        for (u32 w = 2 * q; w + 1 < W; w += 2 * G)
            *reinterpret_cast<ulonglong2*>(row + w) = *reinterpret_cast<const ulonglong2*>(s.row + w);
        if ((W & 1) && q == 0)
            row[W - 1] = s.row[W - 1];
    }
    else
    {
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            const u32 w = 2 * (k * G + q);
            if (w + 1 < W && (W & 1) == 0)
                *reinterpret_cast<ulonglong2*>(row + w) = ulonglong2{s.lo[k], s.hi[k]};
            else
            {
                if (w < W)
                    row[w] = s.lo[k];
                if (w + 1 < W)
                    row[w + 1] = s.hi[k];
            }
        }
    }
}

/// Value of lane `src` of the group (all lanes of the wave must execute this).
template<int G>
__device__ __forceinline__ u64 group_bcast(u64 v, u32 gbase, u32 src)
{
    if constexpr (G == 1)
        return v;
    else
        return __shfl(v, static_cast<int>(gbase + src), kWave);
}

template<int G>
__device__ __forceinline__ u32 group_max(u32 v)
{
#pragma unroll
    for (int d = 1; d < G; d <<= 1)
        v = max(v, static_cast<u32>(__shfl_xor(static_cast<int>(v), d, kWave)));
    return v;
}

/// Whether every lane of the group has `ok` (group-uniform result).
template<int G>
__device__ __forceinline__ bool group_all(bool ok, u32 gbase)
{
    if constexpr (G == 1)
        return ok;
    else
    {
        const u64 bad = __ballot(!ok);
        const u64 mask = G == 64 ? ~u64{0} : (((u64{1} << G) - 1) << gbase);
        return (bad & mask) == 0;
    }
}

template<int G, int K>
__device__ __forceinline__ bool group_equal(const Slice<G, K>& a, const Slice<G, K>& b, u32 gbase)
{
    bool eq = true;
    if constexpr (K == 0)
    {
        const u32 q = lane_id() - gbase;
        for (u32 w = 2 * q; w < a.W && eq; w += 2 * G)
            eq = a.row[w] == b.row[w] && (w + 1 >= a.W || a.row[w + 1] == b.row[w + 1]);
    }
    else
    {
#pragma unroll
        for (int k = 0; k < K; ++k)
            eq = eq && a.lo[k] == b.lo[k] && a.hi[k] == b.hi[k];
    }
    return group_all<G>(eq, gbase);
}

/// hash_state of the group's row (group-uniform).
template<int G, int K>
__device__ __forceinline__ u64 group_hash(const Slice<G, K>& s, u32 q, u32 gbase)
{
    if constexpr (K == 0)
    {
        // the serial chain of hash_state over the trimmed words, on the group's first lane
        u64 h = 0;
        if (q == 0)
            h = hash_state(s.row, s.W);
        return group_bcast<G>(h, gbase, 0);
    }
    else
    {
        u32 top = 0;  // 1 + index of the lane's highest nonzero word
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            const u32 w = 2 * (k * G + q);
            if (s.hi[k])
                top = w + 2;
            else if (s.lo[k])
                top = w + 1;
        }
        const u32 n = group_max<G>(top);
        u64 h = kHashSeed ^ (static_cast<u64>(n) * kHashP1);
#pragma unroll
        for (int k = 0; k < K; ++k)
#pragma unroll
            for (int r = 0; r < G; ++r)
            {
                const u32 p = k * G + r;
                const u64 a = group_bcast<G>(s.lo[k], gbase, r);
                const u64 b = group_bcast<G>(s.hi[k], gbase, r);
                if (2 * p < n)
                    h = mulfold(h ^ a ^ kHashP1, b ^ kHashP2);
            }
        return mix64(h);
    }
}

/// Rows wider than this many words are placed in the table by set_hash_wide instead of hash_state.
constexpr u32 kWideHashWords = 8;

/// The table hash of rows wider than kWideHashWords words: mix64 of the seed xor the sum over the row's nonzero words w
/// of mix64(word + (w + 1) * phi). A row's table slot and tag only place it (ids follow candidate order, and the public
/// state hash has its own kernels), so wide rows take this order-free sum, which the lanes of a group add up in
/// parallel, instead of hash_state's chain of one dependent multiply-fold per word pair with a cross-lane broadcast
/// each. Trailing zero words add nothing, as in hash_state.
MYA_HD inline u64 set_hash_wide(const u64* w, u32 n)
{
    u64 acc = 0;
    for (u32 i = 0; i < n; ++i)
        if (w[i])
            acc += mix64(w[i] + static_cast<u64>(i + 1) * 0x9E3779B97F4A7C15ull);
    return mix64(acc ^ kHashSeed);
}

/// The table hash of a row of `words` words (host side of group_set_hash).
MYA_HD inline u64 set_hash(const u64* w, u32 words) { return words > kWideHashWords ? set_hash_wide(w, words) : hash_state(w, words); }

template<int G>
__device__ __forceinline__ u64 group_sum64(u64 v)
{
#pragma unroll
    for (int d = 1; d < G; d <<= 1)
        v += __shfl_xor(v, d, kWave);
    return v;
}

/// set_hash of the group's row (group-uniform): set_hash_wide for the groups of rows above 8 words (the lanes' sums
/// added across the group), hash_state below.
template<int G, int K>
__device__ __forceinline__ u64 group_set_hash(const Slice<G, K>& s, u32 q, u32 gbase)
{
    if constexpr (K == 0)
    {
        // set_hash_wide with the lanes striding over the row's words
        u64 acc = 0;
        for (u32 w = q; w < s.W; w += G)
            if (const u64 v = s.row[w])
                acc += mix64(v + static_cast<u64>(w + 1) * 0x9E3779B97F4A7C15ull);
        return mix64(group_sum64<G>(acc) ^ kHashSeed);
    }
    else if constexpr (G * K * 2 > kWideHashWords)
    {
        u64 acc = 0;
#pragma unroll
        for (int k = 0; k < K; ++k)
        {
            const u64 w = 2 * static_cast<u64>(k * G + q);
            if (s.lo[k])
                acc += mix64(s.lo[k] + (w + 1) * 0x9E3779B97F4A7C15ull);
            if (s.hi[k])
                acc += mix64(s.hi[k] + (w + 2) * 0x9E3779B97F4A7C15ull);
        }
        return mix64(group_sum64<G>(acc) ^ kHashSeed);
    }
    else
        return group_hash<G, K>(s, q, gbase);
}

__device__ __forceinline__ u64 load_entry(const u64* e) { return __hip_atomic_load(e, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT); }

struct ProbeResult
{
    u64 cand_slot;  // the cand_slot encoding of the candidate
    bool lose;      // the candidate is not the winner of its content (its flag must be cleared)
};

/// Probes the table for the group's row `me` (candidate j, hash h) and inserts it as pending if no equal row is there.
/// Src::load(c, q, out) gives lane q's words of candidate c. Returns the candidate's own outputs, which the caller
/// stores once the wave has reconverged (one coalesced store per wave instead of one per divergent path); the only
/// store made here is the flag of another candidate that this one displaces from a pending entry.
template<int G, int K, class Src>
__device__ __forceinline__ ProbeResult probe_insert(const StateSetView& s, const Src& src, u64 j, const Slice<G, K>& me, u64 h,
                                                    u32 q, u32 gbase, u8* __restrict__ flags, u32* __restrict__ status)
{
    const u64 tag = h >> 32;
    const u64 mine = (tag << 32) | cand_code(s.epoch, j);
    // groups of 4 lanes or more load 4 consecutive entries per round (lane q: slot + q) and examine them in probe order,
    // so a probe that crosses occupied entries waits for one load per 4 of them; smaller groups load one at a time (their
    // probes are decided at the first entry often enough that more loads cost more)
    if constexpr (G < 4)
    {
        u64 slot = slot_of_hash(h, s.capacity);
        for (u64 probes = 0; probes < s.capacity; ++probes)
        {
            u64 e = q == 0 ? load_entry(s.table + slot) : 0;
            e = group_bcast<G>(e, gbase, 0);
            if (e == 0)
            {
                u64 old = 0;
                if (q == 0)
                    old = atomicCAS(reinterpret_cast<unsigned long long*>(s.table + slot), 0ull, static_cast<unsigned long long>(mine));
                old = group_bcast<G>(old, gbase, 0);
                if (old == 0)
                    return {(tag << 32) | slot, false};
                e = old;
            }
            if ((e >> 32) == tag)
            {
                // a pending entry holds a candidate of this batch (its row comes from the row source); any other entry a
                // stored state (its row is in the arena; an id past the arena was cut by a capacity overflow and matches
                // nothing)
                const u32 code = static_cast<u32>(e);
                const bool pending = (code & kPending) && code_epoch(code) == s.epoch;
                const u64 id = pending ? 0 : committed_id(s, code);
                Slice<G, K> o;
                if (pending)
                    src.load(code & kJMask, q, o);
                else if (id < s.max_rows)
                    load_row<G, K>(s.arena + id * s.words, s.words, q, o);
                if ((pending || id < s.max_rows) && group_equal<G, K>(me, o, gbase))
                {
                    if (!pending)
                        return {(id << 32) | kNoSlot, true};
                    // a smaller candidate holding the entry already makes this one lose without an atomic (a pending
                    // entry only ever decreases, so a stale read shows a value at least as large as the current one)
                    if ((code & kJMask) < j)
                        return {(tag << 32) | slot, true};
                    u64 old = 0;
                    if (q == 0)
                        old = atomicMin(reinterpret_cast<unsigned long long*>(s.table + slot), static_cast<unsigned long long>(mine));
                    old = group_bcast<G>(old, gbase, 0);
                    const u64 other = static_cast<u32>(old) & kJMask;
                    if (other > j && q == 0)
                        flags[other] = 0;
                    return {(tag << 32) | slot, other < j};
                }
            }
            slot = slot + 1 == s.capacity ? 0 : slot + 1;
        }
    }
    else
    {
        constexpr int P = 4;
        u64 base = slot_of_hash(h, s.capacity);
        for (u64 probes = 0; probes < s.capacity; probes += P)
        {
            u64 mine_e = 0;
            if (q < P)
            {
                const u64 sq = base + q >= s.capacity ? base + q - s.capacity : base + q;
                mine_e = load_entry(s.table + sq);
            }
    #pragma unroll
            for (int r = 0; r < P; ++r)
            {
                const u64 slot = base + r >= s.capacity ? base + r - s.capacity : base + r;
                u64 e = group_bcast<G>(mine_e, gbase, r);
                if (e == 0)
                {
                    u64 old = 0;
                    if (q == 0)
                        old = atomicCAS(reinterpret_cast<unsigned long long*>(s.table + slot), 0ull, static_cast<unsigned long long>(mine));
                    old = group_bcast<G>(old, gbase, 0);
                    if (old == 0)
                        return {(tag << 32) | slot, false};
                    e = old;
                }
                if ((e >> 32) == tag)
                {
                    // a pending entry holds a candidate of this batch (its row comes from the row source); any other entry
                    // a stored state (its row is in the arena; an id past the arena was cut by a capacity overflow and
                    // matches nothing)
                    const u32 code = static_cast<u32>(e);
                    const bool pending = (code & kPending) && code_epoch(code) == s.epoch;
                    const u64 id = pending ? 0 : committed_id(s, code);
                    Slice<G, K> o;
                    if (pending)
                        src.load(code & kJMask, q, o);
                    else if (id < s.max_rows)
                        load_row<G, K>(s.arena + id * s.words, s.words, q, o);
                    if ((pending || id < s.max_rows) && group_equal<G, K>(me, o, gbase))
                    {
                        if (!pending)
                            return {(id << 32) | kNoSlot, true};
                        // a smaller candidate holding the entry already makes this one lose without an atomic (a pending
                        // entry only ever decreases, so a stale read shows a value at least as large as the current one)
                        if ((code & kJMask) < j)
                            return {(tag << 32) | slot, true};
                        u64 old = 0;
                        if (q == 0)
                            old = atomicMin(reinterpret_cast<unsigned long long*>(s.table + slot), static_cast<unsigned long long>(mine));
                        old = group_bcast<G>(old, gbase, 0);
                        const u64 other = static_cast<u32>(old) & kJMask;
                        if (other > j && q == 0)
                            flags[other] = 0;
                        return {(tag << 32) | slot, other < j};
                    }
                }
            }
            base = base + P >= s.capacity ? base + P - s.capacity : base + P;
        }
    }
    if (q == 0)
        atomicOr(status, kStatusTableFull);
    return {kProbeFailed, true};
}

/// States a search never stores (the reference's BlockedSet, src/mymyr/search/iw_detail.hpp:95-105, compared by
/// content): rows [count, words] and a linear-probing table of (hash tag << 32) | (row index + 1) entries over
/// `capacity` slots (at most half of them taken, so every probe ends at an empty slot), slot and tag as the state
/// set's. hit [batch] receives per candidate whether it was blocked. capacity 0: nothing is blocked.
struct BlockedView
{
    const u64* table;
    u64 capacity;
    const u64* rows;
    u32 words;
    u8* hit;
};

/// Whether the group's row `me` (hash h) is a blocked state (group-uniform).
template<int G, int K>
__device__ __forceinline__ bool group_blocked(const BlockedView& b, const Slice<G, K>& me, u64 h, u32 q, u32 gbase)
{
    const u64 tag = h >> 32;
    u64 slot = slot_of_hash(h, b.capacity);
    for (u64 probes = 0; probes < b.capacity; ++probes)
    {
        u64 e = q == 0 ? b.table[slot] : 0;
        e = group_bcast<G>(e, gbase, 0);
        if (e == 0)
            return false;
        if ((e >> 32) == tag)
        {
            Slice<G, K> o;
            load_row<G, K>(b.rows + (static_cast<u64>(static_cast<u32>(e)) - 1) * b.words, b.words, q, o);
            if (group_equal<G, K>(me, o, gbase))
                return true;
        }
        slot = slot + 1 == b.capacity ? 0 : slot + 1;
    }
    return false;
}

/// Winner w of the batch (candidate j = list[w], id = id0 + w): below `limit` its row into the arena; at or past it,
/// kStatusCapacity (and is_new[j] = 0). The winner's table entry keeps its candidate code: the batch's epoch maps it to
/// the id (its winner block), so no entry is rewritten.
template<int G, int K, class Src>
__device__ __forceinline__ void compact_winner(const StateSetView& s, const Src& src, u64 w, u32 q, const u32* __restrict__ list,
                                               u64 id0, u64 limit, u8* __restrict__ is_new, u32* __restrict__ status)
{
    const u64 j = list[w];
    const u64 id = id0 + w;
    if (id >= limit)
    {
        if (q == 0)
        {
            atomicOr(status, kStatusCapacity);
            if (is_new)
                is_new[j] = 0;
        }
        return;
    }
    Slice<G, K> r;
    src.load(j, q, r);
    store_row<G, K>(s.arena + id * s.words, s.words, q, r);
}
}  // namespace mya
