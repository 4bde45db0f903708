// Device-wide exclusive scan of u32 counts into u64 offsets (see scan.hpp).

#include "scan.hpp"

namespace mya
{
namespace
{
constexpr int kScanBlock = 256;
constexpr int kPerThread = 4;  // 1024 elements per block

__global__ __launch_bounds__(kScanBlock) void k_block_sums(const u32* __restrict__ counts, u64 n, u64* __restrict__ sums)
{
    __shared__ u64 lds[kScanBlock / kWave];
    const u64 base = static_cast<u64>(blockIdx.x) * kScanBlock * kPerThread;
    u64 s = 0;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k)
    {
        const u64 i = base + static_cast<u64>(k) * kScanBlock + threadIdx.x;
        if (i < n)
            s += counts[i];
    }
    s = wave_sum64(s);
    if (lane_id() == 0)
        lds[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        u64 t = 0;
        for (int w = 0; w < kScanBlock / kWave; ++w)
            t += lds[w];
        sums[blockIdx.x] = t;
    }
}

// One block scans the block sums in place (exclusive) and writes the grand total.
__global__ __launch_bounds__(1024) void k_scan_sums(u64* __restrict__ sums, u64 nb, u64* total, const u64* base)
{
    __shared__ u64 lds[1024 / kWave + 1];
    __shared__ u64 carry;
    if (threadIdx.x == 0)
        carry = base ? *base : 0;
    __syncthreads();
    for (u64 base = 0; base < nb; base += 1024)
    {
        const u64 i = base + threadIdx.x;
        const u64 v = i < nb ? sums[i] : 0;
        const u64 inc = wave_inclusive64(v);
        const u32 wave = threadIdx.x / kWave;
        if (lane_id() == kWave - 1)
            lds[wave] = inc;
        __syncthreads();
        if (threadIdx.x == 0)
        {
            u64 run = 0;
            for (int w = 0; w < 1024 / kWave; ++w)
            {
                const u64 t = lds[w];
                lds[w] = run;
                run += t;
            }
            lds[1024 / kWave] = run;
        }
        __syncthreads();
        if (i < nb)
            sums[i] = carry + lds[wave] + inc - v;
        __syncthreads();
        if (threadIdx.x == 0)
            carry += lds[1024 / kWave];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        *total = carry;
}

__global__ __launch_bounds__(kScanBlock) void k_offsets(const u32* __restrict__ counts, u64 n, const u64* __restrict__ sums,
                                                       u64* __restrict__ offsets)
{
    __shared__ u64 lds[kScanBlock / kWave + 1];
    const u64 base = static_cast<u64>(blockIdx.x) * kScanBlock * kPerThread;
    // each thread owns kPerThread consecutive elements
    const u64 first = base + static_cast<u64>(threadIdx.x) * kPerThread;
    u32 v[kPerThread];
    u64 s = 0;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k)
    {
        v[k] = first + k < n ? counts[first + k] : 0;
        s += v[k];
    }
    const u64 inc = wave_inclusive64(s);
    const u32 wave = threadIdx.x / kWave;
    if (lane_id() == kWave - 1)
        lds[wave] = inc;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        u64 run = 0;
        for (int w = 0; w < kScanBlock / kWave; ++w)
        {
            const u64 t = lds[w];
            lds[w] = run;
            run += t;
        }
    }
    __syncthreads();
    u64 off = sums[blockIdx.x] + lds[wave] + inc - s;
#pragma unroll
    for (int k = 0; k < kPerThread; ++k)
    {
        if (first + k < n)
            offsets[first + k] = off;
        off += v[k];
    }
}
// One block scans the block sums in place (exclusive, from 0) and writes *total = *total_base + the grand total. Each
// thread takes kSumsPerThread consecutive sums per pass.
constexpr int kSumsPerThread = 8;

__global__ __launch_bounds__(1024) void k_scan_sums_rel(u64* __restrict__ sums, u64 nb, u64* total, const u64* total_base)
{
    __shared__ u64 lds[1024 / kWave + 1];
    __shared__ u64 carry;
    if (threadIdx.x == 0)
        carry = 0;
    __syncthreads();
    for (u64 b0 = 0; b0 < nb; b0 += 1024 * kSumsPerThread)
    {
        const u64 i0 = b0 + static_cast<u64>(threadIdx.x) * kSumsPerThread;
        u64 v[kSumsPerThread];
        u64 s = 0;
#pragma unroll
        for (int k = 0; k < kSumsPerThread; ++k)
        {
            v[k] = i0 + k < nb ? sums[i0 + k] : 0;
            s += v[k];
        }
        const u64 inc = wave_inclusive64(s);
        const u32 wave = threadIdx.x / kWave;
        if (lane_id() == kWave - 1)
            lds[wave] = inc;
        __syncthreads();
        if (threadIdx.x == 0)
        {
            u64 run = 0;
            for (int w = 0; w < 1024 / kWave; ++w)
            {
                const u64 t = lds[w];
                lds[w] = run;
                run += t;
            }
            lds[1024 / kWave] = run;
        }
        __syncthreads();
        u64 run = carry + lds[wave] + inc - s;
#pragma unroll
        for (int k = 0; k < kSumsPerThread; ++k)
        {
            if (i0 + k < nb)
                sums[i0 + k] = run;
            run += v[k];
        }
        __syncthreads();
        if (threadIdx.x == 0)
            carry += lds[1024 / kWave];
        __syncthreads();
    }
    if (threadIdx.x == 0)
        *total = (total_base ? *total_base : 0) + carry;
}

// Winner flags are bytes (0 or 1), 16 per thread (one 16-byte access), 4096 per block.
constexpr int kFlagsPerThread = 16;
constexpr u64 kFlagsPerBlock = static_cast<u64>(kScanBlock) * kFlagsPerThread;

/// The thread's 16 flags (zeros past n) and their sum; `full` when all 16 lie below n (one 16-byte load).
__device__ __forceinline__ u32 load_flags(const u8* __restrict__ flags, u64 first, u64 n, uint4& v, bool& full)
{
    full = first + kFlagsPerThread <= n;
    if (full)
        v = *reinterpret_cast<const uint4*>(flags + first);
    else
    {
        u32 w[4] = {0, 0, 0, 0};
        for (int k = 0; k < kFlagsPerThread; ++k)
            if (first + k < n)
                w[k / 4] |= static_cast<u32>(flags[first + k]) << (8 * (k % 4));
        v = uint4{w[0], w[1], w[2], w[3]};
    }
    // bytes are 0 or 1: x * 0x01010101 sums the four bytes into the top byte
    return ((v.x * 0x01010101u) >> 24) + ((v.y * 0x01010101u) >> 24) + ((v.z * 0x01010101u) >> 24) + ((v.w * 0x01010101u) >> 24);
}

__global__ __launch_bounds__(kScanBlock) void k_flag_sums(const u8* __restrict__ flags, u64 n, u64* __restrict__ sums)
{
    __shared__ u32 lds[kScanBlock / kWave];
    uint4 v;
    bool full;
    u32 s = load_flags(flags, static_cast<u64>(blockIdx.x) * kFlagsPerBlock + threadIdx.x * kFlagsPerThread, n, v, full);
    s = wave_sum(s);
    if (lane_id() == 0)
        lds[threadIdx.x / kWave] = s;
    __syncthreads();
    if (threadIdx.x == 0)
    {
        u32 t = 0;
        for (int w = 0; w < kScanBlock / kWave; ++w)
            t += lds[w];
        sums[blockIdx.x] = t;
    }
}

// The winners' indices in order (list[rank] = j for flags[j] != 0), their ids base + rank as WinnerBlocks (optional;
// *id_limit reset to ~0), is_new[j] = flags[j] (optional), and the losers' flags reset to 1. kFused: `sums` holds the
// raw block sums, each block adds up those before it itself (few blocks), and the last block writes *total = *base +
// the grand total; else `sums` holds their exclusive scan.
template<bool kFused>
__global__ __launch_bounds__(kScanBlock) void k_winner_list(u8* __restrict__ flags, u64 n, const u64* __restrict__ sums,
                                                           const u64* __restrict__ base, u32* __restrict__ list,
                                                           WinnerBlock* __restrict__ ids, u64* __restrict__ id_limit,
                                                           u8* __restrict__ is_new, u64* __restrict__ total_out)
{
    __shared__ u32 lds[kScanBlock / kWave + 1];
    __shared__ u64 pre[kScanBlock / kWave];
    const u64 first = static_cast<u64>(blockIdx.x) * kFlagsPerBlock + threadIdx.x * kFlagsPerThread;
    uint4 v;
    bool full;
    const u32 s = load_flags(flags, first, n, v, full);
    u64 prefix;
    if constexpr (kFused)
    {
        u64 part = 0;
        for (u64 i = threadIdx.x; i < blockIdx.x; i += kScanBlock)
            part += sums[i];
        part = wave_sum64(part);
        if (lane_id() == 0)
            pre[threadIdx.x / kWave] = part;
        __syncthreads();
        prefix = 0;
        for (int w = 0; w < kScanBlock / kWave; ++w)
            prefix += pre[w];
    }
    else
        prefix = sums[blockIdx.x];
    u32 total;
    const u32 excl = block_exclusive<kScanBlock>(s, lds, &total);
    if constexpr (kFused)
        if (blockIdx.x + 1 == gridDim.x && threadIdx.x == 0)
            *total_out = (base ? *base : 0) + prefix + total;
    u64 off = prefix + excl;
    const u64 id0 = base ? *base : 0;
    const u32 w[4] = {v.x, v.y, v.z, v.w};
    if (ids)
    {
        // four consecutive threads hold 64 consecutive candidates: their 16-bit winner masks make the block's bits and
        // the first thread's first rank its base (the block's first winner, if any, is that thread's or a later one's)
        u32 m16 = 0;
#pragma unroll
        for (int k = 0; k < kFlagsPerThread; ++k)
            m16 |= ((w[k / 4] >> (8 * (k % 4))) & 1) << k;
        const u32 l0 = lane_id() & ~3u;
        u64 bits = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            bits |= static_cast<u64>(static_cast<u32>(__shfl(static_cast<int>(m16), static_cast<int>(l0 + r), kWave))) << (16 * r);
        if ((lane_id() & 3u) == 0 && first < n)
            ids[first / 64] = WinnerBlock{bits, static_cast<u32>(id0 + off), 0u};
        if (id_limit && blockIdx.x == 0 && threadIdx.x == 0)
            *id_limit = ~u64{0};
    }
#pragma unroll
    for (int k = 0; k < kFlagsPerThread; ++k)
        if ((w[k / 4] >> (8 * (k % 4))) & 1)
            list[off++] = static_cast<u32>(first + k);
    if (full)
    {
        if (s != kFlagsPerThread)
            *reinterpret_cast<uint4*>(flags + first) = uint4{0x01010101u, 0x01010101u, 0x01010101u, 0x01010101u};
        if (is_new)
            *reinterpret_cast<uint4*>(is_new + first) = v;
    }
    else
        for (int k = 0; k < kFlagsPerThread && first + k < n; ++k)
        {
            flags[first + k] = 1;
            if (is_new)
                is_new[first + k] = static_cast<u8>((w[k / 4] >> (8 * (k % 4))) & 1);
        }
}
}  // namespace

void launch_winner_list(u8* flags, u64 n, u64* scratch, u64* total, const u64* total_base, u32* list, WinnerBlock* ids,
                        u64* id_limit, u8* is_new, hipStream_t stream)
{
    const u64 nb = (n + kFlagsPerBlock - 1) / kFlagsPerBlock;
    // up to 1024 blocks (2^22 flags), each block adds up the block sums before it (at most 8 KiB, from L2) instead of a
    // third launch scanning them
    constexpr u64 kFusedBlocks = 1024;
    if (nb > 0)
        hipLaunchKernelGGL(k_flag_sums, dim3(static_cast<u32>(nb)), dim3(kScanBlock), 0, stream, flags, n, scratch);
    if (nb > 0 && nb <= kFusedBlocks)
    {
        hipLaunchKernelGGL(k_winner_list<true>, dim3(static_cast<u32>(nb)), dim3(kScanBlock), 0, stream, flags, n, scratch, total_base, list,
                           ids, id_limit, is_new, total);
        return;
    }
    hipLaunchKernelGGL(k_scan_sums_rel, dim3(1), dim3(1024), 0, stream, scratch, nb, total, total_base);
    if (nb > 0)
        hipLaunchKernelGGL(k_winner_list<false>, dim3(static_cast<u32>(nb)), dim3(kScanBlock), 0, stream, flags, n, scratch, total_base,
                           list, ids, id_limit, is_new, total);
}

void launch_exclusive_scan(const u32* counts, u64* offsets, u64 n, u64* scratch, u64* total, hipStream_t stream, const u64* base)
{
    const u64 nb = (n + kScanBlock * kPerThread - 1) / (kScanBlock * kPerThread);
    if (nb == 0)
    {
        // the total of an empty piece is its base
        hipLaunchKernelGGL(k_scan_sums, dim3(1), dim3(1024), 0, stream, scratch, u64{0}, total, base);
        return;
    }
    hipLaunchKernelGGL(k_block_sums, dim3(static_cast<u32>(nb)), dim3(kScanBlock), 0, stream, counts, n, scratch);
    hipLaunchKernelGGL(k_scan_sums, dim3(1), dim3(1024), 0, stream, scratch, nb, total, base);
    hipLaunchKernelGGL(k_offsets, dim3(static_cast<u32>(nb)), dim3(kScanBlock), 0, stream, counts, n, scratch, offsets);
}
}  // namespace mya
