#pragma once
// Integer primitives shared by every kernel (and usable on the host): the state hash, Philox-4x32-10 and the index
// draw. Bit-identical to the reference definitions:
//   mix64 / mulfold / words / state_words  include/mymyr/core/hash.hpp:12-53
//   philox4x32_10 / block / bits64 / below include/mymyr/rl/rng.hpp:45-83
// The 64x64->128 product uses __umul64hi on the device and unsigned __int128 on the host.

#include <hip/hip_runtime.h>

#include <cstdint>

namespace mya
{
using u8 = std::uint8_t;
using u32 = std::uint32_t;
using u64 = std::uint64_t;
using i32 = std::int32_t;
using i64 = std::int64_t;

#define MYA_HD __host__ __device__ __forceinline__

constexpr u64 kHashSeed = 0x2d358dccaa6c78a5ULL;
constexpr u64 kHashP1 = 0x8bb84b93962eacc9ULL;
constexpr u64 kHashP2 = 0x4b33a62ed433d4a3ULL;

MYA_HD u64 mix64(u64 x)
{
    x ^= x >> 30;
    x *= 0xbf58476d1ce4e5b9ULL;
    x ^= x >> 27;
    x *= 0x94d049bb133111ebULL;
    x ^= x >> 31;
    return x;
}

MYA_HD u64 mulfold(u64 a, u64 b)
{
#if defined(__HIP_DEVICE_COMPILE__)
    return (a * b) ^ __umul64hi(a, b);
#else
    const unsigned __int128 r = static_cast<unsigned __int128>(a) * b;
    return static_cast<u64>(r) ^ static_cast<u64>(r >> 64);
#endif
}

/// Hash of n words (order- and length-sensitive).
MYA_HD u64 hash_words(const u64* w, u32 n, u64 seed = kHashSeed)
{
    u64 h = seed ^ (static_cast<u64>(n) * kHashP1);
    u32 i = 0;
    for (; i + 1 < n; i += 2)
        h = mulfold(h ^ w[i] ^ kHashP1, w[i + 1] ^ kHashP2);
    if (i < n)
        h = mulfold(h ^ w[i] ^ kHashP1, kHashP2);
    return mix64(h);
}

MYA_HD u32 trimmed(const u64* w, u32 n)
{
    while (n > 0 && w[n - 1] == 0)
        --n;
    return n;
}

/// The public state hash: hash_words over the trimmed words.
MYA_HD u64 hash_state(const u64* w, u32 n) { return hash_words(w, trimmed(w, n)); }

// ------------------------------------------------------------------------------------------------------ Philox
struct Block4
{
    u32 v[4];
};

MYA_HD u32 mulhi32(u32 a, u32 b) { return static_cast<u32>((static_cast<u64>(a) * b) >> 32); }

MYA_HD Block4 philox4x32_10(Block4 c, u32 k0, u32 k1)
{
    constexpr u32 m0 = 0xD2511F53u, m1 = 0xCD9E8D57u, w0 = 0x9E3779B9u, w1 = 0xBB67AE85u;
#pragma unroll
    for (int r = 0; r < 10; ++r)
    {
        const u32 hi0 = mulhi32(m0, c.v[0]), lo0 = m0 * c.v[0];
        const u32 hi1 = mulhi32(m1, c.v[2]), lo1 = m1 * c.v[2];
        c = Block4{{hi1 ^ c.v[1] ^ k0, lo1, hi0 ^ c.v[3] ^ k1, lo0}};
        k0 += w0;
        k1 += w1;
    }
    return c;
}

/// Philox over the counter (draw low, draw high, env low, purpose) with the seed's halves as key; output words 0 and 1
/// joined into one 64-bit value (word 0 in the low half).
MYA_HD u64 philox_bits64(u64 seed, u64 env, u64 draw, u32 purpose)
{
    const Block4 b = philox4x32_10(Block4{{static_cast<u32>(draw), static_cast<u32>(draw >> 32), static_cast<u32>(env), purpose}},
                                   static_cast<u32>(seed), static_cast<u32>(seed >> 32));
    return static_cast<u64>(b.v[0]) | (static_cast<u64>(b.v[1]) << 32);
}

/// Lemire's multiply-shift reduction of a 64-bit draw onto [0, n): the upper 64 bits of the 128-bit product x * n,
/// assembled from x's two 32-bit halves so that host and device compute the same value.
MYA_HD u32 below(u64 x, u32 n)
{
    const u64 hi = (x >> 32) * n, lo = (x & 0xFFFFFFFFull) * n;
    return static_cast<u32>((hi + (lo >> 32)) >> 32);
}

MYA_HD u32 successor_index(u64 seed, u64 env, u64 draw, u32 count) { return below(philox_bits64(seed, env, draw, 0), count); }

// ------------------------------------------------------------------------------------------------------ instance draws
/// MurmurHash3's 32-bit finalizer.
MYA_HD u32 fmix32(u32 x)
{
    x = (x ^ (x >> 16)) * 0x85EBCA6Bu;
    x = (x ^ (x >> 13)) * 0xC2B2AE35u;
    return x ^ (x >> 16);
}

/// Which instance an env restarts in (rl::rng::instance_draw, include/mymyr/rl/rng.hpp:94-115). The seed, the env
/// number and its reset count are mixed into 32 bits; with m == 0 they scale uniformly onto [0, instances), otherwise
/// the draw selects indices[k], k being how many of the m - 1 sorted thresholds do not exceed it.
MYA_HD i32 instance_draw(u64 seed, u64 env, u32 reset_count, u32 instances, const u32* thresholds, const i32* indices, u32 m)
{
    const u32 key = fmix32(static_cast<u32>(seed) ^ fmix32(static_cast<u32>(seed >> 32) ^ 0x53414D50u));
    const u32 bits = fmix32(key ^ fmix32(static_cast<u32>(env)) ^ fmix32(reset_count ^ 0x9E3779B9u));
    if (m == 0)
        return static_cast<i32>((static_cast<u64>(bits) * instances) >> 32);
    u32 lo = 0, hi = m - 1;  // bisection for the first threshold greater than bits
    while (lo < hi)
    {
        const u32 mid = lo + (hi - lo) / 2;
        if (thresholds[mid] <= bits)
            lo = mid + 1;
        else
            hi = mid;
    }
    return indices[lo];
}

// ------------------------------------------------------------------------------------------------------ errors
/// Sticky device status bits (OR-ed into a device word, read by the host after the stream drains).
enum StatusBit : u32
{
    kStatusTableFull = 1u << 0,     // a hash-set probe wrapped around the whole table
    kStatusCapacity = 1u << 1,      // an output buffer was too small
    kStatusWideRow = 1u << 2,       // a state has bits beyond the task's words
    kStatusNoSlot = 1u << 3,        // an add effect without an atom slot
    kStatusPickFailed = 1u << 4,    // the chosen successor index was not found (internal inconsistency)
    kStatusGoalMask = 1u << 5,      // per-env goal masks set bits past the task's fluent slots
    kStatusTaskId = 1u << 6,        // a task id (of a row or of next_task_ids) names no instance of the table
};
/// GoalSpec::AnyOf on the device: goal k holds in a state iff the slots slots[off[2k], off[2k + 1]) are set and the
/// slots [off[2k + 1], off[2k + 2]) clear (count 0 with `any` set: no state is a goal).
struct AnyOfDev
{
    const u32* off;    // [2 count + 1]
    const u32* slots;
    u32 count;
    u32 any;           // 1: the AnyOf goals decide (0: the task's goal)
};

/// Whether one of the AnyOf goals holds in a row (one lane's view of it: bit s of the row).
template<class Bit>
__device__ __forceinline__ bool any_of_holds_dev(const AnyOfDev& g, Bit&& bit)
{
    for (u32 k = 0; k < g.count; ++k)
    {
        bool ok = true;
        for (u32 i = g.off[2 * k]; i < g.off[2 * k + 1] && ok; ++i)
            ok = bit(g.slots[i]);
        for (u32 i = g.off[2 * k + 1]; i < g.off[2 * k + 2] && ok; ++i)
            ok = !bit(g.slots[i]);
        if (ok)
            return true;
    }
    return false;
}

}  // namespace mya
