#pragma once
// Wave64 and block prefix sums (exact integer scans) used for successor offsets and new-state ids, plus a
// three-launch device-wide exclusive scan over u32 counts with a u64 total.

#include "device_common.hpp"

namespace mya
{
constexpr int kWave = 64;

__device__ __forceinline__ u32 lane_id() { return __lane_id(); }

/// Inclusive prefix sum across the 64 lanes of a wave.
__device__ __forceinline__ u32 wave_inclusive(u32 v)
{
    const u32 lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1)
    {
        const u32 t = __shfl_up(v, d, kWave);
        if (lane >= static_cast<u32>(d))
            v += t;
    }
    return v;
}

__device__ __forceinline__ u64 wave_inclusive64(u64 v)
{
    const u32 lane = lane_id();
#pragma unroll
    for (int d = 1; d < kWave; d <<= 1)
    {
        const u64 t = __shfl_up(v, d, kWave);
        if (lane >= static_cast<u32>(d))
            v += t;
    }
    return v;
}

__device__ __forceinline__ u32 wave_sum(u32 v)
{
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1)
        v += __shfl_xor(v, d, kWave);
    return v;
}

__device__ __forceinline__ u64 wave_sum64(u64 v)
{
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1)
        v += __shfl_xor(v, d, kWave);
    return v;
}

/// Exclusive prefix of v over a block of BLOCK threads; *total receives the block sum. Uses BLOCK/64 words of LDS.
template<int BLOCK>
__device__ __forceinline__ u32 block_exclusive(u32 v, u32* lds, u32* total)
{
    const u32 lane = lane_id(), wave = threadIdx.x / kWave;
    const u32 inc = wave_inclusive(v);
    if (lane == kWave - 1)
        lds[wave] = inc;
    __syncthreads();
    if (wave == 0)
    {
        u32 s = lane < BLOCK / kWave ? lds[lane] : 0;
        const u32 si = wave_inclusive(s);
        if (lane < BLOCK / kWave)
            lds[lane] = si - s;
        if (lane == BLOCK / kWave - 1)
            lds[BLOCK / kWave] = si;
    }
    __syncthreads();
    const u32 r = lds[wave] + inc - v;
    *total = lds[BLOCK / kWave];
    __syncthreads();
    return r;
}

/// Device-wide exclusive scan of u32 counts into u64 offsets, in three launches: per-block sums, a one-block scan of
/// the sums, then the per-element offsets. `scratch` holds blocks(n) + 1 u64 words; `total` (device) receives the sum.
/// With `base` (device, optional) every offset and the total start at *base instead of 0 (`total` may be the element
/// after the last offset, and `base` the total of the previous piece, to scan a sequence piece by piece).
void launch_exclusive_scan(const u32* counts, u64* offsets, u64 n, u64* scratch, u64* total, hipStream_t stream,
                           const u64* base = nullptr);
constexpr u64 scan_scratch_words(u64 n) { return (n + 1023) / 1024 + 2; }

/// The ids of the winners among 64 consecutive candidates of a batch: bit t of `bits` marks candidate 64k + t a winner
/// and `base` is the id of the block's first winner. Winners take consecutive ids in candidate order, so a winner's id
/// is base + the winners before it in the block: 16 bytes per 64 candidates where an id per candidate takes 256.
struct alignas(16) WinnerBlock
{
    u64 bits;
    u32 base;
    u32 reserved;
};
constexpr u64 winner_blocks(u64 n) { return (n + 63) / 64; }
/// The id of winner j (j's bit set in its block b = blocks[j / 64]).
__host__ __device__ inline u64 winner_id(const WinnerBlock& b, u32 j)
{
    return b.base + static_cast<u64>(__builtin_popcountll(b.bits & ((u64{1} << (j & 63)) - 1)));
}

/// The indices j of the nonzero flags in order into list[0, winners) (flag bytes are 0 or 1; zero flags are reset to 1),
/// the winners' ids as WinnerBlocks from *total_base on (optional; *id_limit, when given, is reset to ~0 for a cut to
/// lower), is_new[j] = flags[j] (optional), and *total = *total_base + winners. Three launches; scratch as for
/// launch_exclusive_scan. flags must be 16-byte aligned.
void launch_winner_list(u8* flags, u64 n, u64* scratch, u64* total, const u64* total_base, u32* list, WinnerBlock* ids,
                        u64* id_limit, u8* is_new, hipStream_t stream);
}  // namespace mya
