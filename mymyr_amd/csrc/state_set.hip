// Device state set (state_set.hpp): the batch insert of rows held in a buffer, row hashing, the dedup stream.

#include "runtime.hpp"
#include "state_set.hpp"

#include <algorithm>
#include <cmath>

namespace mya
{
namespace
{
constexpr int kBlock = 256;

/// Rows of a device buffer as the row source of the probe and the compaction.
struct BufferRows
{
    const u64* rows;
    u32 W;
    template<int G, int K>
    __device__ __forceinline__ void load(u64 c, u32 q, Slice<G, K>& o) const
    {
        load_row<G, K>(rows + c * W, W, q, o);
    }
};

/// The group of this lane: (candidate, lane in group, first lane of the group in the wave).
template<int G>
__device__ __forceinline__ void group_of(u64& j, u32& q, u32& gbase)
{
    const u64 t = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    const u32 lane = lane_id();
    j = t / G;
    q = lane % G;
    gbase = lane - q;
}

template<int G, int K>
__global__ __launch_bounds__(kBlock) void k_hash_rows(const u64* __restrict__ rows, u64 n, u32 words, u64* __restrict__ out)
{
    u64 j;
    u32 q, gbase;
    group_of<G>(j, q, gbase);
    if (j >= n)
        return;
    Slice<G, K> r;
    load_row<G, K>(rows + j * words, words, q, r);
    const u64 h = group_hash<G, K>(r, q, gbase);
    if (q == 0)
        out[j] = h;
}

template<int G, int K>
__global__ __launch_bounds__(kBlock) void k_insert(StateSetView s, const u64* __restrict__ rows, u64 n, u64* __restrict__ cand_slot,
                                                  u8* __restrict__ flags, u32* __restrict__ status, BlockedView blocked)
{
    u64 j;
    u32 q, gbase;
    group_of<G>(j, q, gbase);
    if (j >= n)
        return;
    const BufferRows src{rows, s.words};
    Slice<G, K> me;
    src.load(j, q, me);
    const u64 h = group_set_hash<G, K>(me, q, gbase);
    if (blocked.capacity)
    {
        // a blocked candidate is dropped before the table is probed (it takes no entry and no id)
        const bool hit = group_blocked<G, K>(blocked, me, h, q, gbase);
        if (q == 0)
        {
            blocked.hit[j] = hit ? 1 : 0;
            if (hit)
                flags[j] = 0;
        }
        if (hit)
            return;
    }
    const ProbeResult r = probe_insert<G, K>(s, src, j, me, h, q, gbase, flags, status);
    if (q == 0)
    {
        if (cand_slot)
            cand_slot[j] = r.cand_slot;
        if (r.lose)
            flags[j] = 0;
    }
}

// Compaction over the batch's winners (their count: size_next - size_now, read on the device).
template<int G, int K>
__global__ __launch_bounds__(kBlock) void k_compact(StateSetView s, const u64* __restrict__ rows, const u32* __restrict__ list,
                                                   const u64* __restrict__ size_now,
                                                   const u64* __restrict__ size_next, u64 limit, u8* __restrict__ is_new,
                                                   u32* __restrict__ status)
{
    u64 w;
    u32 q, gbase;
    group_of<G>(w, q, gbase);
    const u64 id0 = *size_now;
    if (w >= *size_next - id0)
        return;
    compact_winner<G, K>(s, BufferRows{rows, s.words}, w, q, list, id0, limit, is_new, status);
}

__global__ __launch_bounds__(kBlock) void k_resolve_ids(StateSetView s, const u64* __restrict__ cand_slot, u64 n, i64* __restrict__ ids)
{
    const u64 j = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= n)
        return;
    const u64 cs = cand_slot[j];
    i64 id = -1;
    if (cs == kProbeFailed)
        id = -1;
    else if (cand_is_stored(cs))
        id = static_cast<i64>(cs >> 32);
    else
    {
        const u64 c = committed_id(s, static_cast<u32>(s.table[static_cast<u32>(cs)]));
        id = c < s.max_rows ? static_cast<i64>(c) : -1;
    }
    ids[j] = id;
}

// Settles every candidate-coded entry to id + 1 (two entries per thread per step).
__global__ __launch_bounds__(kBlock) void k_settle(u64* __restrict__ table, u64 capacity, const WinnerBlock* __restrict__ id_map, u64 stride,
                                                  const u64* __restrict__ id_limit)
{
    const u64 pairs = capacity / 2;
    for (u64 i = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x; i < pairs; i += static_cast<u64>(gridDim.x) * kBlock)
    {
        const ulonglong2 v = reinterpret_cast<const ulonglong2*>(table)[i];
        u64 e[2] = {v.x, v.y};
        bool dirty = false;
        for (int k = 0; k < 2; ++k)
        {
            const u32 code = static_cast<u32>(e[k]);
            if (code & kPending)
            {
                e[k] = (e[k] & 0xFFFFFFFF00000000ull) | (epoch_winner_id(id_map, stride, id_limit, code_epoch(code), code & kJMask) + 1u);
                dirty = true;
            }
        }
        if (dirty)
            reinterpret_cast<ulonglong2*>(table)[i] = ulonglong2{e[0], e[1]};
    }
}

/// A cut batch keeps the winners below the set's new size: ids from `size` on stand for kCutId (an id past every arena, so
/// their entries match nothing, also once settled: code id + 1 keeps the pending bit clear).
__global__ void k_cut_words(u64* __restrict__ size_now, u64* __restrict__ limit, u64 size)
{
    *size_now = size;
    *limit = size;
}

__global__ __launch_bounds__(kBlock) void k_fill_u32(u32* __restrict__ p, u64 n, u32 v)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x; i < n; i += static_cast<u64>(gridDim.x) * kBlock)
        p[i] = v;
}

__global__ void k_set_words(u64* p, u64 a, u64 b, u32* status)
{
    p[0] = a;
    p[1] = b;
    *status = 0;
}

// The dedup stream: row i is, with probability `dup` (i > 0), an exact copy of row src(i) < i, else fresh words
// mix64(seed + (16 i + k + 1) * gamma). Counter-based, so any range of rows is generated independently.
constexpr u64 kGamma = 0x9E3779B97F4A7C15ULL;
constexpr u64 kDupKey = 0xD1B54A32D192ED03ULL;
constexpr u64 kSrcKey = 0x8CB92BA72F3D8DD7ULL;

__global__ __launch_bounds__(kBlock) void k_dedup_rows(u64 start, u64 count, u32 words, u64 seed, u64 thr, u64* __restrict__ out)
{
    const u64 t = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    const u64 j = t / words;
    const u32 k = static_cast<u32>(t - j * words);
    if (j >= count)
        return;
    u64 cur = start + j;
    while (cur > 0 && (mix64((seed ^ kDupKey) ^ (cur * kGamma)) >> 32) < thr)
        cur = ((mix64((seed ^ kSrcKey) ^ (cur * kGamma)) & 0xFFFFFFFFull) * cur) >> 32;
    out[t] = mix64(seed + (cur * 16 + k + 1) * kGamma);
}

/// n random 8-byte operations of kind kKind (0 load, 1 CAS, 2 atomicMin, 3 store) on table[mix64(seed + i * gamma) & mask],
/// four independent ones per thread in flight; the loads' and atomics' results fold into sink[thread].
template<int kKind>
__global__ __launch_bounds__(kBlock) void k_random_ops(u64* __restrict__ table, u64 mask, u64 n, u64 seed, u64* __restrict__ sink)
{
    constexpr int kIn = 4;
    const u64 t = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    const u64 threads = static_cast<u64>(gridDim.x) * kBlock;
    u64 acc = 0;
    for (u64 i0 = t * kIn; i0 < n; i0 += threads * kIn)
    {
        u64 a[kIn];
#pragma unroll
        for (int k = 0; k < kIn; ++k)
            a[k] = mix64(seed + (i0 + k) * kGamma) & mask;
#pragma unroll
        for (int k = 0; k < kIn; ++k)
        {
            if (i0 + k >= n)
                break;
            unsigned long long* p = reinterpret_cast<unsigned long long*>(table + a[k]);
            if constexpr (kKind == 0)
                acc ^= *p;
            else if constexpr (kKind == 1)
                acc ^= atomicCAS(p, 0ull, static_cast<unsigned long long>(a[k] | 1));
            else if constexpr (kKind == 2)
                acc ^= atomicMin(p, static_cast<unsigned long long>(~a[k]));
            else
                *p = i0 + k;
        }
    }
    if constexpr (kKind != 3)
        sink[t] = acc;
}

/// Calls f.template operator()<G, K>() for the lane-group shape of rows of W words.
template<class F>
void with_shape(u32 W, F&& f)
{
    if (W <= 2)
        f.template operator()<1, 1>();
    else if (W <= 4)
        f.template operator()<2, 1>();
    else if (W <= 8)
        f.template operator()<4, 1>();
    else if (W <= 16)
        f.template operator()<4, 2>();  // four lanes of two pairs: faster than eight of one on 16-word rows
    else if (W <= 32)
        f.template operator()<16, 1>();
    else if (W <= 128)
        f.template operator()<64, 1>();
    else if (W <= 256)
        f.template operator()<64, 2>();
    else if (W <= 512)
        f.template operator()<64, 4>();
    else if (W <= 1024)
        f.template operator()<64, 8>();
    else if (W <= kLongRowWords)
        f.template operator()<64, 16>();
    else
        f.template operator()<64, 0>();  // long rows: compared, hashed and copied from memory by a 64-lane group
}

/// The lane-group shape of the compaction: the probe's, except that rows of 9-16 words are copied by eight lanes of
/// one word pair (their probe takes four lanes of two).
template<class F>
void with_copy_shape(u32 W, F&& f)
{
    if (W > 8 && W <= 16)
        f.template operator()<8, 1>();
    else
        with_shape(W, f);
}

template<int G>
unsigned group_blocks(u64 n)
{
    return blocks_for(n * G, kBlock);
}
}  // namespace

void launch_fill_u32(u32* p, u64 n, u32 v, hipStream_t stream)
{
    if (n == 0)
        return;
    hipLaunchKernelGGL(k_fill_u32, dim3(std::min<u64>(blocks_for(n, kBlock), 8192)), dim3(kBlock), 0, stream, p, n, v);
    launch_check("fill");
}

void launch_random_ops(u64* table, u64 words, u64 n, int kind, u64 seed, u64* sink, hipStream_t stream)
{
    const dim3 grid(kRandomOpsThreads / kBlock), block(kBlock);
    const u64 mask = words - 1;
    if (kind == 0)
        hipLaunchKernelGGL(k_random_ops<0>, grid, block, 0, stream, table, mask, n, seed, sink);
    else if (kind == 1)
        hipLaunchKernelGGL(k_random_ops<1>, grid, block, 0, stream, table, mask, n, seed, sink);
    else if (kind == 2)
        hipLaunchKernelGGL(k_random_ops<2>, grid, block, 0, stream, table, mask, n, seed, sink);
    else
        hipLaunchKernelGGL(k_random_ops<3>, grid, block, 0, stream, table, mask, n, seed, sink);
    launch_check("random ops");
}

void launch_dedup_rows(u64 start, u64 count, u32 words, u64 seed, double dup, u64* out, hipStream_t stream)
{
    if (count == 0)
        return;
    const u64 thr = static_cast<u64>(dup * 4294967296.0);
    hipLaunchKernelGGL(k_dedup_rows, dim3(blocks_for(count * words, kBlock)), dim3(kBlock), 0, stream, start, count, words, seed, thr, out);
    launch_check("dedup rows");
}

void launch_hash_rows(const u64* rows, u64 n, u32 words, u64* out, hipStream_t stream)
{
    if (n == 0)
        return;
    with_shape(words, [&]<int G, int K>() {
        hipLaunchKernelGGL((k_hash_rows<G, K>), dim3(group_blocks<G>(n)), dim3(kBlock), 0, stream, rows, n, words, out);
    });
    launch_check("hash_rows");
}

void state_set_create(StateSet& s, u64 max_states, u32 words, double max_load, u64 batch_cap, hipStream_t stream, u64 pending)
{
    if (words == 0)
        throw std::invalid_argument("mymyr_amd: state set rows need at least one word");
    if (!(max_load > 0.0 && max_load <= 0.95))
        throw std::invalid_argument("mymyr_amd: state set load must be in (0, 0.95]");
    if (max_states >= (u64{1} << 31) - 1)
        throw std::invalid_argument("mymyr_amd: state set holds at most 2^31 - 2 states");
    if (batch_cap >= (u64{1} << 31))
        throw std::invalid_argument("mymyr_amd: state set batches hold fewer than 2^31 rows");
    // an even capacity of at least 64 slots (the epoch settling streams the table two entries at a time)
    u64 cap = std::max<u64>(64, static_cast<u64>(std::ceil(static_cast<double>(max_states + pending) / max_load)));
    cap += cap & 1;
    if (cap >= (u64{1} << 32) - 1)
        throw std::invalid_argument("mymyr_amd: state set table capacity above 2^32 - 2 slots");
    s.v.words = words;
    s.v.capacity = cap;
    s.max_states = max_states;
    s.batch_cap = std::clamp<u64>(batch_cap, 1, kMaxBatch);
    // epochs in rotation: as many as fit 512 MiB of id maps (the 2^25-candidate batches of the BrFS: 64), at least 4
    const u64 blocks = winner_blocks(s.batch_cap);
    s.epochs = static_cast<u32>(std::clamp<u64>((u64{1} << 29) / (blocks * sizeof(WinnerBlock)), 4, kMaxEpochs));
    s.id_map = dev_alloc<WinnerBlock>(s.epochs * blocks, "state set epoch ids");
    s.id_limit = dev_alloc<u64>(s.epochs, "state set epoch cuts");
    s.v.id_map = s.id_map;
    s.v.id_limit = s.id_limit;
    s.v.id_stride = blocks;
    s.v.max_rows = max_states;
    s.v.table = dev_alloc<u64>(cap, "state set table");
    s.v.arena = dev_alloc<u64>(max_states * words, "state set arena");
    s.cand_slot = dev_alloc<u64>(s.batch_cap, "state set batch slots");
    s.flags = dev_alloc<u8>((s.batch_cap + 15) / 16 * 16, "state set batch flags");
    s.list = dev_alloc<u32>(s.batch_cap, "state set batch winners");
    s.scan_scratch = dev_alloc<u64>(scan_scratch_words(s.batch_cap), "state set scan scratch");
    s.d_size = dev_alloc<u64>(2, "state set size");
    s.d_status = dev_alloc<u32>(1, "state set status");
    s.h_pinned = static_cast<u64*>(pinned_acquire(sizeof(u64) * 4));
    launch_fill_u32(reinterpret_cast<u32*>(s.flags), (s.batch_cap + 15) / 16 * 4, 0x01010101u, stream);  // flag bytes 1
    state_set_clear(s, stream);
}

void state_set_destroy(StateSet& s, hipStream_t stream)
{
    for (void* p : {static_cast<void*>(s.v.table), static_cast<void*>(s.v.arena), static_cast<void*>(s.cand_slot),
                    static_cast<void*>(s.flags), static_cast<void*>(s.list), static_cast<void*>(s.scan_scratch),
                    static_cast<void*>(s.d_size), static_cast<void*>(s.d_status), static_cast<void*>(s.id_map),
                    static_cast<void*>(s.id_limit)})
    {
        if (stream)
            dev_free_async(p, stream);
        else
            dev_free(p);
    }
    if (s.h_pinned)
    {
        // the pinned words are reused by the next set only after this one's last copies into them have landed
        if (stream)
            (void)hipStreamSynchronize(stream);
        pinned_release(s.h_pinned);
    }
    s = StateSet{};
}

void state_set_clear(StateSet& s, hipStream_t stream)
{
    // a fill kernel rather than a memset node, so that a captured clear replays correctly
    launch_fill_u32(reinterpret_cast<u32*>(s.v.table), s.v.capacity * 2, 0u, stream);
    hipLaunchKernelGGL(k_set_words, dim3(1), dim3(1), 0, stream, s.d_size, u64{0}, u64{0}, s.d_status);
    launch_check("clear state set");
    s.cur = 0;
    s.size = 0;
    s.batches = 0;
    s.v.epoch = 0;
    s.last = stream;
}

void state_set_begin_batch(StateSet& s, hipStream_t stream)
{
    if (s.batches == s.epochs)
    {
        // every epoch is taken: one streaming pass settles all candidate-coded entries, and the rotation restarts
        hipLaunchKernelGGL(k_settle, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(s.v.capacity / 2, kBlock), 8192))), dim3(kBlock),
                           0, stream, s.v.table, s.v.capacity, s.id_map, s.v.id_stride, s.id_limit);
        launch_check("state set settle");
        s.batches = 0;
    }
    s.v.epoch = static_cast<u32>(s.batches++);
}

void state_set_rank(StateSet& s, u64 n, hipStream_t stream, u8* is_new)
{
    launch_winner_list(s.flags, n, s.scan_scratch, state_set_size_next(s), state_set_size_now(s), s.list,
                       s.id_map + static_cast<u64>(s.v.epoch) * s.v.id_stride, s.id_limit + s.v.epoch, is_new, stream);
    launch_check("state set rank");
}

void state_set_resolve_ids(StateSet& s, const u64* cand_slot, u64 n, i64* ids, hipStream_t stream)
{
    if (n == 0)
        return;
    hipLaunchKernelGGL(k_resolve_ids, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, stream, s.v, cand_slot, n, ids);
    launch_check("state set ids");
}

void state_set_cut(StateSet& s, u64 size, hipStream_t stream)
{
    hipLaunchKernelGGL(k_cut_words, dim3(1), dim3(1), 0, stream, state_set_size_now(s), s.id_limit + s.v.epoch, size);
    launch_check("state set cut");
    s.size = size;
}

void state_set_probe(StateSet& s, const u64* rows, u64 m, hipStream_t stream, const BlockedView* blocked, u64* cand_slot)
{
    if (m == 0)
        return;
    const BlockedView bl = blocked ? *blocked : BlockedView{};
    with_shape(s.v.words, [&]<int G, int K>() {
        hipLaunchKernelGGL((k_insert<G, K>), dim3(group_blocks<G>(m)), dim3(kBlock), 0, stream, s.v, rows, m, cand_slot, s.flags,
                           s.d_status, bl);
    });
    launch_check("state set probe");
    s.last = stream;
}

void state_set_sync(StateSet& s)
{
    // the size and status words are read here only (an asynchronous insert copies nothing back)
    hip_check(hipMemcpyAsync(s.h_pinned + 1, state_set_size_now(s), sizeof(u64), hipMemcpyDeviceToHost, s.last), "read size");
    hip_check(hipMemcpyAsync(s.h_pinned + 2, s.d_status, sizeof(u32), hipMemcpyDeviceToHost, s.last), "read status");
    hip_check(hipStreamSynchronize(s.last), "state set");
    const u32 status = static_cast<u32>(s.h_pinned[2]);
    const u64 after = s.h_pinned[1];
    s.size = std::min(after, s.max_states);
    if (status & kStatusTableFull)
        throw std::length_error("mymyr_amd: state set table full");
    if (status & kStatusCapacity)
        throw std::length_error("mymyr_amd: state set full (" + std::to_string(s.max_states) + " states; the inserts needed " +
                                std::to_string(after) + ")");
}

void state_set_insert(StateSet& s, const u64* rows, u64 n, i64* ids, u8* is_new, u64* new_count, hipStream_t stream)
{
    const u32 W = s.v.words;
    if (new_count)
        hip_check(hipMemcpyAsync(s.h_pinned, state_set_size_now(s), sizeof(u64), hipMemcpyDeviceToHost, stream), "read size");
    with_shape(W, [&]<int G, int K>() {
        for (u64 done = 0; done < n;)
        {
            const u64 m = std::min(n - done, s.batch_cap);
            const u64* r = rows + done * W;
            state_set_begin_batch(s, stream);
            // the probe results are kept only for the ids
            hipLaunchKernelGGL((k_insert<G, K>), dim3(group_blocks<G>(m)), dim3(kBlock), 0, stream, s.v, r, m, ids ? s.cand_slot : nullptr,
                               s.flags, s.d_status, BlockedView{});
            launch_check("state set probe");
            state_set_rank(s, m, stream, is_new ? is_new + done : nullptr);
            with_copy_shape(W, [&]<int G2, int K2>() {
                hipLaunchKernelGGL((k_compact<G2, K2>), dim3(group_blocks<G2>(m)), dim3(kBlock), 0, stream, s.v, r, s.list,
                                   state_set_size_now(s), state_set_size_next(s), s.max_states, is_new ? is_new + done : nullptr,
                                   s.d_status);
            });
            launch_check("state set compact");
            if (ids)
            {
                hipLaunchKernelGGL(k_resolve_ids, dim3(blocks_for(m, kBlock)), dim3(kBlock), 0, stream, s.v, s.cand_slot, m, ids + done);
                launch_check("state set ids");
            }
            state_set_flip(s);
            done += m;
        }
    });
    s.last = stream;
    if (new_count)
    {
        state_set_sync(s);
        *new_count = s.h_pinned[1] - s.h_pinned[0];
    }
}
}  // namespace mya
