// Device state set (state_set.hpp): row hashing, CAS probing with a min-candidate winner, ranking, compaction.

#include "runtime.hpp"
#include "scan.hpp"
#include "state_set.hpp"

#include <algorithm>
#include <cmath>

namespace mya
{
namespace
{
constexpr u64 kDupSettled = u64{1} << 63;
constexpr u64 kProbeFailed = ~u64{0};
constexpr u64 kProbeSkipped = ~u64{0} - 1;  // a candidate outside the probe mask
constexpr int kBlock = 256;


__device__ __forceinline__ bool rows_equal(const u64* __restrict__ a, const u64* __restrict__ b, u32 w)
{
    for (u32 i = 0; i < w; ++i)
        if (a[i] != b[i])
            return false;
    return true;
}

__global__ __launch_bounds__(kBlock) void k_hash_rows(const u64* __restrict__ rows, u64 n, u32 words, u64* __restrict__ out)
{
    const u64 i = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    if (i >= n)
        return;
    out[i] = hash_state(rows + i * words, words);
}

__global__ __launch_bounds__(kBlock) void k_probe(StateSetView s, const u64* __restrict__ rows, const u64* __restrict__ hashes,
                                                 const u8* __restrict__ mask, u64 n, u64* __restrict__ cand_slot,
                                                 u32* __restrict__ status)
{
    const u64 j = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= n)
        return;
    if (mask && !mask[j])
    {
        cand_slot[j] = kProbeSkipped;
        return;
    }
    const u64 h = hashes[j];
    const u64 tag = h >> 32;
    const u32 W = s.words;
    const u64* row = rows + j * W;
    u64 slot = slot_of_hash(h, s.capacity);
    for (u64 probes = 0; probes < s.capacity; ++probes)
    {
        u64 e = __hip_atomic_load(s.table + slot, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (e == 0)
        {
            const u64 mine = (tag << 32) | kPending | j;
            const u64 old = atomicCAS(reinterpret_cast<unsigned long long*>(s.table + slot), 0ull, static_cast<unsigned long long>(mine));
            if (old == 0)
            {
                cand_slot[j] = slot;
                return;
            }
            e = old;
        }
        if ((e >> 32) == tag)
        {
            const u32 code = static_cast<u32>(e);
            const bool pending = (code & kPending) != 0;
            const u64* other = pending ? rows + static_cast<u64>(code & ~kPending) * W : s.arena + static_cast<u64>(code - 1) * W;
            if (rows_equal(row, other, W))
            {
                if (pending)
                {
                    atomicMin(reinterpret_cast<unsigned long long*>(s.table + slot), static_cast<unsigned long long>((tag << 32) | kPending | j));
                    cand_slot[j] = slot;
                }
                else
                    cand_slot[j] = slot | kDupSettled;
                return;
            }
        }
        slot = slot + 1 == s.capacity ? 0 : slot + 1;
    }
    atomicOr(status, kStatusTableFull);
    cand_slot[j] = kProbeFailed;
}

__global__ __launch_bounds__(kBlock) void k_flags(StateSetView s, const u64* __restrict__ cand_slot, u64 n, u32* __restrict__ flags)
{
    const u64 j = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= n)
        return;
    const u64 cs = cand_slot[j];
    u32 win = 0;
    if (cs < kProbeSkipped && !(cs & kDupSettled))
        win = static_cast<u32>(s.table[cs]) == (kPending | static_cast<u32>(j)) ? 1u : 0u;
    flags[j] = win;
}

__global__ __launch_bounds__(kBlock) void k_compact(StateSetView s, const u64* __restrict__ rows, const u64* __restrict__ hashes,
                                                   const u64* __restrict__ cand_slot, const u32* __restrict__ flags,
                                                   const u64* __restrict__ offsets, u64 n, u64 base, u64 limit, u8* __restrict__ is_new)
{
    const u64 j = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= n)
        return;
    const bool win = flags[j] != 0;
    if (is_new)
        is_new[j] = 0;
    if (!win)
        return;
    const u64 id = base + offsets[j];
    if (id >= limit)
        return;
    const u32 W = s.words;
    const u64* src = rows + j * W;
    u64* dst = s.arena + id * W;
    for (u32 i = 0; i < W; ++i)
        dst[i] = src[i];
    const u64 h = hashes[j];
    s.hashes[id] = h;
    s.table[cand_slot[j]] = ((h >> 32) << 32) | static_cast<u32>(id + 1);
    if (is_new)
        is_new[j] = 1;
}

__global__ __launch_bounds__(kBlock) void k_resolve_ids(StateSetView s, const u64* __restrict__ cand_slot, u64 n, i64* __restrict__ ids)
{
    const u64 j = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= n)
        return;
    const u64 cs = cand_slot[j];
    if (cs >= kProbeSkipped)
    {
        ids[j] = -1;
        return;
    }
    const u32 code = static_cast<u32>(s.table[cs & ~kDupSettled]);
    ids[j] = (code & kPending) ? -1 : static_cast<i64>(code) - 1;
}
// The dedup stream: row i is, with probability `dup` (i > 0), an exact copy of row src(i) < i, else fresh words
// mix64(seed + (16 i + k + 1) * gamma). Counter-based, so any range of rows is generated independently.
constexpr u64 kGamma = 0x9E3779B97F4A7C15ULL;
constexpr u64 kDupKey = 0xD1B54A32D192ED03ULL;
constexpr u64 kSrcKey = 0x8CB92BA72F3D8DD7ULL;

__global__ __launch_bounds__(kBlock) void k_dedup_rows(u64 start, u64 count, u32 words, u64 seed, u64 thr, u64* __restrict__ out)
{
    const u64 j = static_cast<u64>(blockIdx.x) * kBlock + threadIdx.x;
    if (j >= count)
        return;
    u64 cur = start + j;
    while (cur > 0 && (mix64((seed ^ kDupKey) ^ (cur * kGamma)) >> 32) < thr)
        cur = ((mix64((seed ^ kSrcKey) ^ (cur * kGamma)) & 0xFFFFFFFFull) * cur) >> 32;
    u64* row = out + j * words;
    for (u32 k = 0; k < words; ++k)
        row[k] = mix64(seed + (cur * 16 + k + 1) * kGamma);
}
}  // namespace

void launch_dedup_rows(u64 start, u64 count, u32 words, u64 seed, double dup, u64* out, hipStream_t stream)
{
    if (count == 0)
        return;
    const u64 thr = static_cast<u64>(dup * 4294967296.0);
    hipLaunchKernelGGL(k_dedup_rows, dim3(blocks_for(count, kBlock)), dim3(kBlock), 0, stream, start, count, words, seed, thr, out);
    launch_check("dedup rows");
}

void launch_hash_rows(const u64* rows, u64 n, u32 words, u64* out, hipStream_t stream)
{
    if (n == 0)
        return;
    hipLaunchKernelGGL(k_hash_rows, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, stream, rows, n, words, out);
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
    const u64 cap = std::max<u64>(64, static_cast<u64>(std::ceil(static_cast<double>(max_states + pending) / max_load)));
    if (cap >= (u64{1} << 32))
        throw std::invalid_argument("mymyr_amd: state set table capacity above 2^32 slots");
    s.v.words = words;
    s.v.capacity = cap;
    s.max_states = max_states;
    s.batch_cap = std::max<u64>(1, batch_cap);
    s.v.table = dev_alloc<u64>(cap, "state set table");
    s.v.arena = dev_alloc<u64>(max_states * words, "state set arena");
    s.v.hashes = dev_alloc<u64>(max_states, "state set hashes");
    s.cand_slot = dev_alloc<u64>(s.batch_cap, "state set batch slots");
    s.flags = dev_alloc<u32>(s.batch_cap, "state set batch flags");
    s.offsets = dev_alloc<u64>(s.batch_cap, "state set batch offsets");
    s.hashes_tmp = dev_alloc<u64>(s.batch_cap, "state set batch hashes");
    s.scan_scratch = dev_alloc<u64>(scan_scratch_words(s.batch_cap), "state set scan scratch");
    s.d_total = dev_alloc<u64>(2, "state set totals");
    s.d_status = dev_alloc<u32>(1, "state set status");
    hip_check(hipHostMalloc(reinterpret_cast<void**>(&s.h_pinned), sizeof(u64) * 2, hipHostMallocDefault), "pinned count");
    state_set_clear(s, stream);
}

void state_set_destroy(StateSet& s)
{
    dev_free(s.v.table);
    dev_free(s.v.arena);
    dev_free(s.v.hashes);
    dev_free(s.cand_slot);
    dev_free(s.flags);
    dev_free(s.offsets);
    dev_free(s.hashes_tmp);
    dev_free(s.scan_scratch);
    dev_free(s.d_total);
    dev_free(s.d_status);
    if (s.h_pinned)
        (void)hipHostFree(s.h_pinned);
    s = StateSet{};
}

void state_set_clear(StateSet& s, hipStream_t stream)
{
    hip_check(hipMemsetAsync(s.v.table, 0, s.v.capacity * sizeof(u64), stream), "clear state set");
    hip_check(hipMemsetAsync(s.d_status, 0, sizeof(u32), stream), "clear state set status");
    s.size = 0;
}

void state_set_probe(StateSet& s, const u64* rows, const u64* hashes, u64 n, hipStream_t stream, const u8* mask)
{
    if (n == 0)
        return;
    hipLaunchKernelGGL(k_probe, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, stream, s.v, rows, hashes, mask, n, s.cand_slot,
                       s.d_status);
    launch_check("state set probe");
}

void state_set_rank(StateSet& s, u64 n, hipStream_t stream)
{
    if (n == 0)
    {
        hip_check(hipMemsetAsync(s.d_total, 0, sizeof(u64), stream), "rank");
        return;
    }
    hipLaunchKernelGGL(k_flags, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, stream, s.v, s.cand_slot, n, s.flags);
    launch_check("state set flags");
    launch_exclusive_scan(s.flags, s.offsets, n, s.scan_scratch, s.d_total, stream);
    launch_check("state set scan");
}

void state_set_compact(StateSet& s, const u64* rows, const u64* hashes, u64 n, u64 base, u64 limit, i64* ids, u8* is_new,
                       hipStream_t stream)
{
    if (n == 0)
        return;
    hipLaunchKernelGGL(k_compact, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, stream, s.v, rows, hashes, s.cand_slot, s.flags,
                       s.offsets, n, base, limit, is_new);
    launch_check("state set compact");
    if (ids)
    {
        hipLaunchKernelGGL(k_resolve_ids, dim3(blocks_for(n, kBlock)), dim3(kBlock), 0, stream, s.v, s.cand_slot, n, ids);
        launch_check("state set ids");
    }
}

void state_set_insert(StateSet& s, const u64* rows, const u64* hashes, u64 n, i64* ids, u8* is_new, u64* new_count,
                      hipStream_t stream)
{
    u64 done = 0, added = 0;
    while (done < n)
    {
        const u64 m = std::min(n - done, s.batch_cap);
        if (s.size + m > s.max_states)
            throw std::length_error("mymyr_amd: state set full (" + std::to_string(s.size) + " of " + std::to_string(s.max_states) +
                                    " states; the batch could add " + std::to_string(m) + ")");
        const u64* r = rows + done * s.v.words;
        const u64* h = hashes ? hashes + done : s.hashes_tmp;
        if (!hashes)
            launch_hash_rows(r, m, s.v.words, s.hashes_tmp, stream);
        state_set_probe(s, r, h, m, stream);
        state_set_rank(s, m, stream);
        state_set_compact(s, r, h, m, s.size, s.max_states, ids ? ids + done : nullptr, is_new ? is_new + done : nullptr, stream);
        hip_check(hipMemcpyAsync(s.h_pinned, s.d_total, sizeof(u64), hipMemcpyDeviceToHost, stream), "read new count");
        u32 status = 0;
        hip_check(hipMemcpyAsync(reinterpret_cast<u32*>(s.h_pinned + 1), s.d_status, sizeof(u32), hipMemcpyDeviceToHost, stream),
                  "read status");
        hip_check(hipStreamSynchronize(stream), "state set insert");
        status = *reinterpret_cast<u32*>(s.h_pinned + 1);
        if (status & kStatusTableFull)
            throw std::length_error("mymyr_amd: state set table full");
        s.size += s.h_pinned[0];
        added += s.h_pinned[0];
        done += m;
    }
    if (new_count)
        *new_count = added;
}
}  // namespace mya
