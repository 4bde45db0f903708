// Lifted matching (lifted.hpp) and the device env step (env.hpp). A block holds up to kMaxWaves wavefronts that share
// the LDS copy of the task's hot tables; each wave steps one environment at a time in its own LDS region. Waves of a
// block run different environments, so every barrier inside the per-environment work is a wavefront barrier.

#include "env.hpp"
#include "runtime.hpp"
#include "state_set.hpp"

#include <algorithm>
#include <mutex>
#include <type_traits>
#include <unordered_map>

namespace mya
{
TaskDev task_dev(const u64* img, const DevTaskHeader& h)
{
    TaskDev t{};
    t.off_schemas = h.off_schemas;
    t.off_steps = h.off_steps;
    t.off_cons = h.off_cons;
    t.off_checks = h.off_checks;
    t.off_effects = h.off_effects;
    t.off_pairs = h.off_pairs;
    t.off_decode = h.off_decode;
    t.off_dom0 = h.off_dom0;
    t.off_goal_pos = h.off_goal_pos;
    t.off_goal_neg = h.off_goal_neg;
    t.off_pred_arity = h.off_pred_arity;
    t.off_pos_begin = h.off_pos_begin;
    t.off_pred_pairs = h.off_pred_pairs;
    t.off_pred_offset = h.off_pred_offset;
    t.image = img;
    t.rs = img + h.off_rs;
    t.slot_of = reinterpret_cast<const u32*>(img + h.off_slot_of);
    t.records = img + h.off_records;
    t.static_rows = img + h.off_static_rows;
    t.static_meta = reinterpret_cast<const DevStaticMeta*>(img + h.off_static_meta);
    t.static_words = img;
    t.initial = img + h.off_initial;
    t.witness = h.off_witness ? reinterpret_cast<const DevWitness*>(img + h.off_witness) : nullptr;
    t.fluent_count = h.fluent_count;
    t.hot_words = static_cast<u32>(h.hot_words);
    t.n = h.num_objects;
    t.ow = h.ow;
    t.W = h.words;
    t.num_schemas = h.num_schemas;
    t.num_pairs = h.num_pairs;
    t.view_words = h.view_words;
    t.ngp = h.num_goal_pos;
    t.ngn = h.num_goal_neg;
    t.goal_unsat = h.goal_unsat;
    t.dense = h.dense;
    t.label_width = h.label_width;
    t.fluent_slots = h.fluent_slots;
    t.num_decode = h.num_decode;
    t.decode_arith = h.decode_arith;
    t.max_step_words = h.max_step_words;
    t.lazy = h.lazy;
    t.missing = nullptr;
    return t;
}

namespace
{
constexpr int kMaxWaves = 4;
constexpr u64 kHotMax = 48 * 1024;  // hot tables above this size stay in global memory (read through the caches)
constexpr u32 kMaxEff = 32;  // effects per schema the step applies (more set kStatusCapacity)
static_assert(kCap == 64, "a level of the level-synchronous count holds one item per lane");

/// LDS-qualified types: their pointers are 32-bit LDS addresses.
template<class X>
using lds = __attribute__((address_space(3))) X;

/// A copy of the record at p (LDS or global).
template<class X>
__device__ __forceinline__ X ld(const X* p)
{
    return *p;
}
template<class X>
__device__ __forceinline__ X ld(lds<const X>* p)
{
    static_assert(sizeof(X) % 4 == 0, "records are whole 32-bit words");
    u32 w[sizeof(X) / 4];
    const lds<const u32>* src = (const lds<const u32>*)p;
#pragma unroll
    for (u32 i = 0; i < sizeof(X) / 4; ++i)
        w[i] = src[i];
    X x;
    __builtin_memcpy(&x, w, sizeof(X));
    return x;
}

/// The hot tables: in LDS (kStaged) or in the image in global memory.
template<bool kStaged>
struct Tab
{
    template<class X>
    using ptr = std::conditional_t<kStaged, lds<const X>*, const X*>;
    ptr<DevSchema> schemas;
    ptr<DevStep> steps;
    ptr<DevCons> cons;
    ptr<DevCheck> checks;
    ptr<DevEffect> effects;
    ptr<DevPair> pairs;
    ptr<DevPredDecode> decode;
    ptr<u64> dom0;
    ptr<u32> goal_pos;
    ptr<u32> goal_neg;
    ptr<u32> pred_arity;
    ptr<u32> pos_begin;
    ptr<u64> pred_pairs;
    ptr<u64> pred_offset;
};

template<bool kStaged, class Base>
__device__ __forceinline__ Tab<kStaged> tab_of(Base hot, const TaskDev& T)
{
    using H = Tab<kStaged>;
    H t;
    t.schemas = reinterpret_cast<typename H::template ptr<DevSchema>>(hot + T.off_schemas);
    t.steps = reinterpret_cast<typename H::template ptr<DevStep>>(hot + T.off_steps);
    t.cons = reinterpret_cast<typename H::template ptr<DevCons>>(hot + T.off_cons);
    t.checks = reinterpret_cast<typename H::template ptr<DevCheck>>(hot + T.off_checks);
    t.effects = reinterpret_cast<typename H::template ptr<DevEffect>>(hot + T.off_effects);
    t.pairs = reinterpret_cast<typename H::template ptr<DevPair>>(hot + T.off_pairs);
    t.decode = reinterpret_cast<typename H::template ptr<DevPredDecode>>(hot + T.off_decode);
    t.dom0 = hot + T.off_dom0;
    t.goal_pos = reinterpret_cast<typename H::template ptr<u32>>(hot + T.off_goal_pos);
    t.goal_neg = reinterpret_cast<typename H::template ptr<u32>>(hot + T.off_goal_neg);
    t.pred_arity = reinterpret_cast<typename H::template ptr<u32>>(hot + T.off_pred_arity);
    t.pos_begin = reinterpret_cast<typename H::template ptr<u32>>(hot + T.off_pos_begin);
    t.pred_pairs = hot + T.off_pred_pairs;
    t.pred_offset = hot + T.off_pred_offset;
    return t;
}

/// A wave's LDS region.
struct Lds
{
    lds<u64>* row;     // [W] the state
    lds<u64>* view;    // [view_words] rows of the non-bulk view pairs
    lds<u32>* qa;      // [kCap][A] item bindings of the current level of a level-synchronous count
    lds<u32>* qb;      // [kCap][A] the next level
    lds<u32>* ra;      // [kCap] root of each current item
    lds<u32>* rb;      // [kCap]
    lds<u32>* rc;      // [kCap] per-root counts
    lds<u32>* robj;    // [kCap] the objects of a pick round's roots
    lds<u32>* own;     // [kCap] the lane that makes each item of a level-expansion round
    lds<u32>* ub;      // [A] the wave-uniform binding (pick prefix, then the picked action)
    lds<u32>* bind;    // [A][64]: lane columns of the per-lane nested loop (count_from)
    lds<u64>* cur_m;   // [A][64]: its enumeration cursors (candidate bits left)
    lds<u32>* cur_w;   // [A][64]: its enumeration cursors (word index)
    lds<u32>* eff;     // [kMaxEff]: effect slots of a successor (lane k: effect k)
    lds<u32>* before;  // [kMaxEff]: their bits before the move
    lds<u32>* counts;  // [num_schemas]
    lds<u64>* dfs_m;   // [A] the successor enumeration's per-parameter candidates left in the current word
    lds<u32>* dfs_w;   // [A] and that word
};

template<bool kLevels>
__device__ __forceinline__ Lds lds_of(lds<u64>* base, const TaskDev& T)
{
    const u32 A = T.label_width ? T.label_width : 1;
    Lds l;
    lds<u64>* p = base;
    l.row = p;
    p += T.W;
    l.view = p;
    p += T.view_words;
    l.ub = reinterpret_cast<lds<u32>*>(p);
    p += (A + 1) / 2;
    l.bind = reinterpret_cast<lds<u32>*>(p);
    p += 32 * A;
    l.cur_m = p;
    p += 64 * A;
    l.cur_w = reinterpret_cast<lds<u32>*>(p);
    p += 32 * A;
    l.eff = reinterpret_cast<lds<u32>*>(p);
    p += kMaxEff / 2;
    l.before = reinterpret_cast<lds<u32>*>(p);
    p += kMaxEff / 2;
    l.counts = reinterpret_cast<lds<u32>*>(p);
    p += (T.num_schemas + 1) / 2;
    l.dfs_m = p;
    p += A;
    l.dfs_w = reinterpret_cast<lds<u32>*>(p);
    p += (A + 1) / 2;
    if constexpr (kLevels)
    {
        l.qa = reinterpret_cast<lds<u32>*>(p);
        p += kCap * A / 2;
        l.qb = reinterpret_cast<lds<u32>*>(p);
        p += kCap * A / 2;
        l.ra = reinterpret_cast<lds<u32>*>(p);
        p += kCap / 2;
        l.rb = reinterpret_cast<lds<u32>*>(p);
        p += kCap / 2;
        l.rc = reinterpret_cast<lds<u32>*>(p);
        p += kCap / 2;
        l.robj = reinterpret_cast<lds<u32>*>(p);
        p += kCap / 2;
        l.own = reinterpret_cast<lds<u32>*>(p);
    }
    return l;
}

/// Orders the wave's LDS accesses before and after this point (lanes of one wave run in lockstep).
__device__ __forceinline__ void wave_sync()
{
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

/// The hot tables of the block: copied into LDS at kernel start (whole block), or the image itself when they do not
/// fit. Returns the start of the waves' LDS regions.
template<bool kStaged>
__device__ __forceinline__ lds<u64>* stage_hot(u64* smem_generic, const TaskDev& T, Tab<kStaged>* H)
{
    lds<u64>* smem = (lds<u64>*)(smem_generic);
    if constexpr (kStaged)
    {
        for (u32 k = threadIdx.x; k < T.hot_words; k += blockDim.x)
            smem[k] = T.image[k];
        __syncthreads();
        *H = tab_of<true>(static_cast<lds<const u64>*>(smem), T);
        return smem + T.hot_words;
    }
    else
    {
        *H = tab_of<false>(T.image, T);
        return smem;
    }
}

/// 64 bits of a row (bit 0 = object row_lo, `words` words) for objects [obj_start, obj_start + 64); zeros outside.
template<class P>
__device__ __forceinline__ u64 extract64(P row, u32 words, u32 row_lo, u32 obj_start)
{
    const i64 bitpos = static_cast<i64>(obj_start) - static_cast<i64>(row_lo);
    const i64 wi = bitpos >> 6;
    const u32 sh = static_cast<u32>(bitpos & 63);
    const u64 lo = (wi >= 0 && wi < static_cast<i64>(words)) ? row[wi] : 0;
    if (sh == 0)
        return lo;
    const u64 hi = (wi + 1 >= 0 && wi + 1 < static_cast<i64>(words)) ? row[wi + 1] : 0;
    return (lo >> sh) | (hi << (64 - sh));
}

/// Bits [rel, rel + 64) of the `len`-bit segment that starts at bit `base` of the W-word row (zeros outside it).
template<class P>
__device__ __forceinline__ u64 seg_bits(P row, u32 W, u64 base, i64 rel, u32 len)
{
    if (rel >= static_cast<i64>(len) || rel <= -64)
        return 0;
    const i64 a = static_cast<i64>(base) + rel;
    const i64 wi = a >> 6;
    const u32 sh = static_cast<u32>(a & 63);
    const u64 lo = (wi >= 0 && wi < static_cast<i64>(W)) ? row[wi] : 0;
    u64 v = lo;
    if (sh)
    {
        const u64 hi = (wi + 1 >= 0 && wi + 1 < static_cast<i64>(W)) ? row[wi + 1] : 0;
        v = (lo >> sh) | (hi << (64 - sh));
    }
    if (rel < 0)
        v &= ~u64{0} << static_cast<u32>(-rel);
    const i64 keep = static_cast<i64>(len) - rel;  // valid bits from position 0
    if (keep < 64)
        v &= (u64{1} << static_cast<u32>(keep)) - 1;
    return v;
}

template<class P>
__device__ __forceinline__ bool row_bit(P row, u32 slot) { return (row[slot >> 6] >> (slot & 63)) & 1; }

/// The candidate bits of step `st` for objects [st.lo + 64 w, + 64) under the binding b (parameter p at b[p * bs]).
__device__ __forceinline__ u64 cand_word(const TaskDev& T, const auto& H, const Lds& L, const auto& st, u32 w, auto b, u32 bs)
{
    u64 a = ~u64{0};
    const u32 obj0 = st.lo + 64 * w;
    for (u32 ci = st.cons_begin; ci < st.cons_end; ++ci)
    {
        const DevCons c = ld(H.cons + ci);
        u64 v;
        if (c.kind == static_cast<u32>(ConsKind::Dom0))
            v = H.dom0[c.table + w];
        else if (c.kind == static_cast<u32>(ConsKind::StaticRow))
        {
            const u32 so = b[c.src * bs];
            v = extract64(T.static_rows + (static_cast<u64>(c.table) * T.n + so) * T.ow, T.ow, 0, obj0);
        }
        else
        {
            const auto& p = H.pairs[c.table];
            u32 ri = 0;
            if (c.kind == static_cast<u32>(ConsKind::ViewRow))
                ri = (c.src == kNone ? c.obj : b[c.src * bs]) - p.src_lo;
            if (ri >= p.src_n)
                v = 0;
            else if (p.bulk)
                v = seg_bits(L.row, T.W, p.bit0 + static_cast<u64>(ri) * p.row_bits, static_cast<i64>(obj0) - static_cast<i64>(p.dst_lo),
                             p.row_bits);
            else
                v = extract64(L.view + p.offset + static_cast<u64>(ri) * p.dst_words, p.dst_words, p.dst_lo, obj0);
        }
        a &= c.neg ? ~v : v;
    }
    return a;
}

/// Calls f(w, m) for the window words w >= w0 of step st whose candidate word m is nonzero, ascending, until f returns
/// true (then returns true). The binding b (stride bs) must hold the same prefix in every lane (the parameters before
/// st's): the words are evaluated 64 at a time, one per lane, and the nonzero ones taken from a ballot, so a wide
/// window with few candidates costs one evaluation instead of one per word.
template<class F>
__device__ __forceinline__ bool for_nonzero_words(const TaskDev& T, const auto& H, const Lds& L, const auto& st, u32 w0, auto b, u32 bs,
                                                  u32 lane, F&& f)
{
    for (u32 base = w0; base < st.words; base += kWave)
    {
        const u32 wl = base + lane;
        const u64 mine = wl < st.words ? cand_word(T, H, L, st, wl, b, bs) : 0;
        for (u64 nz = __ballot(mine != 0); nz; nz &= nz - 1)
        {
            const u32 k = static_cast<u32>(__builtin_ctzll(nz));
            if (f(base + k, __shfl(mine, static_cast<int>(k), kWave)))
                return true;
        }
    }
    return false;
}

__device__ __forceinline__ bool check_holds(const TaskDev& T, const auto& H, const Lds& L, const auto& c, auto b, u32 bs)
{
    u32 objs[6];
#pragma unroll
    for (int i = 0; i < 6; ++i)
    {
        const i32 t = c.terms[i];
        objs[i] = (static_cast<u32>(i) < c.nterms) ? (t < 0 ? static_cast<u32>(-(t + 1)) : b[t * bs]) : 0;
    }
    bool h;
    if (c.kind == static_cast<u32>(CheckKind::Fluent))
    {
        u64 key = H.pred_offset[c.pred];
        const u32 pb = H.pos_begin[c.pred];
#pragma unroll
        for (int i = 0; i < 6; ++i)
            if (static_cast<u32>(i) < c.nterms)
                key += T.rs[static_cast<u64>(pb + i) * T.n + objs[i]];
        if (key >= T.fluent_count)
            h = false;
        else
        {
            const u32 slot = T.dense ? static_cast<u32>(key) : T.slot_of[key];
            h = slot != kNone && row_bit(L.row, slot);
        }
    }
    else
    {
        const DevStaticMeta m = T.static_meta[c.pred];
        u64 key = 0;
#pragma unroll
        for (int i = 0; i < 6; ++i)
            if (static_cast<u32>(i) < c.nterms)
                key = key * T.n + objs[i];
        const u64* keys = T.static_words + m.keys;
        u64 lo = 0, hi = m.count;
        while (lo < hi)
        {
            const u64 mid = lo + (hi - lo) / 2;
            if (keys[mid] < key)
                lo = mid + 1;
            else
                hi = mid;
        }
        h = lo < m.count && keys[lo] == key;
    }
    return h == (c.pos != 0);
}

__device__ __forceinline__ bool checks_ok(const TaskDev& T, const auto& H, const Lds& L, u32 cb, u32 ce, auto b, u32 bs)
{
    for (u32 k = cb; k < ce; ++k)
        if (!check_holds(T, H, L, H.checks[k], b, bs))
            return false;
    return true;
}

/// Bindings completing steps [si, se) sequentially in this lane (its own binding column L.bind[p * 64 + lane]): an
/// iterative nested loop whose per-level cursor (current word index and remaining candidate bits) lives in the lane's
/// LDS columns. The fallback of count_multi for levels wider than its item capacity.
__device__ __forceinline__ u32 count_from(const TaskDev& T, const auto& H, const Lds& L, u32 si, u32 se, u32 lane)
{
    if (si == se)
        return 1;
    const auto b = L.bind + lane;
    u32 total = 0;
    u32 d = 0;  // level: step si + d
    L.cur_w[lane] = 0;
    L.cur_m[lane] = cand_word(T, H, L, H.steps[si], 0, b, 64);
    for (;;)
    {
        const auto& st = H.steps[si + d];
        u64 m = L.cur_m[d * 64 + lane];
        const bool last = si + d + 1 == se;
        const bool chk = st.check_begin != st.check_end;
        if (last && !chk)
        {
            total += static_cast<u32>(__popcll(m));
            m = 0;
        }
        if (m == 0)
        {
            // next word of this level, or back to the level above
            const u32 w = L.cur_w[d * 64 + lane] + 1;
            if (w < st.words)
            {
                L.cur_w[d * 64 + lane] = w;
                L.cur_m[d * 64 + lane] = cand_word(T, H, L, st, w, b, 64);
                continue;
            }
            if (d == 0)
                break;
            --d;
            continue;
        }
        const u32 bit = static_cast<u32>(__builtin_ctzll(m));
        L.cur_m[d * 64 + lane] = m & (m - 1);
        L.bind[st.param * 64 + lane] = st.lo + 64 * L.cur_w[d * 64 + lane] + bit;
        if (chk && !checks_ok(T, H, L, st.check_begin, st.check_end, b, 64))
            continue;
        if (last)
        {
            ++total;
            continue;
        }
        ++d;
        L.cur_w[d * 64 + lane] = 0;
        L.cur_m[d * 64 + lane] = cand_word(T, H, L, H.steps[si + d], 0, b, 64);
    }
    return total;
}

/// The candidates m of step st for item binding b that pass the step's k-ary checks (each bit bound in the lane's
/// column and checked).
__device__ __forceinline__ u64 checked(const TaskDev& T, const auto& H, const Lds& L, const auto& st, u32 w, u64 m, auto b,
                                       u32 A, u32 lane)
{
    for (u32 p = 0; p < A; ++p)
        L.bind[p * 64 + lane] = b[p];
    u64 keep = 0;
    for (u64 x = m; x;)
    {
        const u32 bit = static_cast<u32>(__builtin_ctzll(x));
        x &= x - 1;
        L.bind[st.param * 64 + lane] = st.lo + 64 * w + bit;
        if (checks_ok(T, H, L, st.check_begin, st.check_end, L.bind + lane, 64))
            keep |= u64{1} << bit;
    }
    return keep;
}

/// Position of the k-th (from 0) set bit of m (k < popcount(m)).
__device__ __forceinline__ u32 kth_bit(u64 m, u32 k)
{
    u32 pos = 0;
    u32 c = static_cast<u32>(__popc(static_cast<u32>(m)));
    if (k >= c)
    {
        k -= c;
        m >>= 32;
        pos += 32;
    }
#pragma unroll
    for (u32 sh = 16; sh; sh >>= 1)
    {
        c = static_cast<u32>(__popc(static_cast<u32>(m) & ((1u << sh) - 1)));
        if (k >= c)
        {
            k -= c;
            m >>= sh;
            pos += sh;
        }
    }
    return pos;
}

/// The OR of v over the wave.
__device__ __forceinline__ u64 wave_or64(u64 v)
{
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1)
        v |= __shfl_xor(v, d, kWave);
    return v;
}

/// (item, word) of pair p of a level with `words` words per item (p < 2^20): p / words by a float estimate and one
/// correction step.
__device__ __forceinline__ void pair_of(u32 p, u32 words, float rcp, u32* item, u32* w)
{
    if (words == 1)
    {
        *item = p;
        *w = 0;
        return;
    }
    u32 q = static_cast<u32>(static_cast<float>(p) * rcp);
    if (q * words > p)
        --q;
    else if ((q + 1) * words <= p)
        ++q;
    *item = q;
    *w = p - q * words;
}

/// Level-synchronous count: for each of the nroots roots (bindings L.qa[r * A ...], every parameter that steps
/// [si, se) read already bound), the number of full bindings completing steps [si, se) into L.rc[r]. Each level
/// spreads its (item, candidate word) pairs over the lanes; a non-last level turns the candidate bits into the next
/// level's items (their order does not matter for counting; item j of a round is made by lane j, which selects its
/// bit from the pair that holds it), the last level adds popcounts to the items' roots. A level with more than kCap
/// items continues in the lanes' nested loops (count_from) from the current items.
__device__ __forceinline__ void count_multi(const TaskDev& T, const auto& H, const Lds& L, u32 si, u32 se, u32 nroots, u32 lane)
{
    const u32 A = T.label_width ? T.label_width : 1;
    if (lane < kCap)
    {
        L.rc[lane] = (si == se && lane < nroots) ? 1u : 0u;
        L.ra[lane] = lane;
    }
    wave_sync();
    if (si == se || nroots == 0)
        return;
    lds<u32>* qa = L.qa;
    lds<u32>* qb = L.qb;
    lds<u32>* ra = L.ra;
    lds<u32>* rb = L.rb;
    u32 n = nroots;
    for (u32 k = si; k < se; ++k)
    {
        const DevStep st = ld(H.steps + k);
        const bool last = k + 1 == se;
        const bool chk = st.check_begin != st.check_end;
        const u32 pairs = n * st.words;
        const float rcp = 1.0f / static_cast<float>(st.words);
        u32 total1 = 0;  // a single root's count (a wave sum instead of LDS atomics)
        if (last)
        {
            for (u32 p0 = 0; p0 < pairs; p0 += kWave)
            {
                const u32 p = p0 + lane;
                if (p < pairs)
                {
                    u32 item, w;
                    pair_of(p, st.words, rcp, &item, &w);
                    u64 m = cand_word(T, H, L, st, w, qa + item * A, 1);
                    if (chk && m)
                        m = checked(T, H, L, st, w, m, qa + item * A, A, lane);
                    const u32 c = static_cast<u32>(__popcll(m));
                    if (c && nroots > 1)
                        __hip_atomic_fetch_add(L.rc + ra[item], c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                    if (nroots == 1)
                        total1 += c;
                }
            }
            if (nroots == 1)
            {
                const u32 t1 = wave_sum(total1);
                if (lane == 0)
                    L.rc[0] = t1;
            }
            wave_sync();
            return;
        }
        // the next level's items: the current item's binding with the step's parameter bound to each candidate
        u32 base = 0;
        bool wide = false;
        for (u32 p0 = 0; p0 < pairs && !wide; p0 += kWave)
        {
            const u32 p = p0 + lane;
            u64 m = 0;
            u32 item = 0, w = 0;
            if (p < pairs)
            {
                pair_of(p, st.words, rcp, &item, &w);
                m = cand_word(T, H, L, st, w, qa + item * A, 1);
                if (chk && m)
                    m = checked(T, H, L, st, w, m, qa + item * A, A, lane);
            }
            const u32 c = static_cast<u32>(__popcll(m));
            const u32 incl = wave_inclusive(c);
            const u32 round = __shfl(incl, kWave - 1, kWave);
            if (base + round > kCap)
            {
                wide = true;
                break;
            }
            if (round == 0)
                continue;
            const u32 o = incl - c;
            if (__ballot(c > 4) == 0)
            {
                // few candidates per pair: each lane writes its own items
                u32 dst = base + o;
                for (u64 x = m; x; ++dst)
                {
                    const u32 bit = static_cast<u32>(__builtin_ctzll(x));
                    x &= x - 1;
                    for (u32 q = 0; q < A; ++q)
                        qb[dst * A + q] = qa[item * A + q];
                    qb[dst * A + st.param] = st.lo + 64 * w + bit;
                    rb[dst] = ra[item];
                }
                base += round;
                wave_sync();
                continue;
            }
            // output j of the round comes from the lane whose range [incl - c, incl) holds j
            const u64 starts = wave_or64(c ? u64{1} << o : 0);
            if (c)
                L.own[o] = lane;
            wave_sync();
            u32 src = 0, sp = 0;
            if (lane < round)
            {
                const u64 le = lane == 63 ? ~u64{0} : (u64{2} << lane) - 1;
                sp = 63u - static_cast<u32>(__clzll(starts & le));
                src = L.own[sp];
            }
            const u64 sm = __shfl(m, static_cast<int>(src), kWave);
            const u32 sitem = __shfl(item, static_cast<int>(src), kWave);
            const u32 sw = __shfl(w, static_cast<int>(src), kWave);
            if (lane < round)
            {
                const u32 bit = kth_bit(sm, lane - sp);
                const u32 dst = base + lane;
                for (u32 q = 0; q < A; ++q)
                    qb[dst * A + q] = qa[sitem * A + q];
                qb[dst * A + st.param] = st.lo + 64 * sw + bit;
                rb[dst] = ra[sitem];
            }
            base += round;
            wave_sync();
        }
        if (wide)
        {
            // too wide for the item levels: each lane completes its items with the nested loop
            for (u32 item = lane; item < n; item += kWave)
            {
                for (u32 q = 0; q < A; ++q)
                    L.bind[q * 64 + lane] = qa[item * A + q];
                const u32 c = count_from(T, H, L, k, se, lane);
                if (c)
                    __hip_atomic_fetch_add(L.rc + ra[item], c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            }
            wave_sync();
            return;
        }
        if (base == 0)
            return;
        lds<u32>* t = qa;
        qa = qb;
        qb = t;
        t = ra;
        ra = rb;
        rb = t;
        n = base;
    }
}

/// Bindings completing steps [si, se) from the empty binding: the first step's candidates split over the lanes (one
/// bit per lane), each lane completing its own with the nested loop. Wave-uniform result.
__device__ __forceinline__ u32 count_wave(const TaskDev& T, const auto& H, const Lds& L, u32 si, u32 se, u32 lane)
{
    if (si == se)
        return 1;
    const DevStep st = ld(H.steps + si);
    const bool chk = st.check_begin != st.check_end;
    const bool last = si + 1 == se;
    u32 mine = 0;
    for (u32 w = 0; w < st.words; ++w)
    {
        const u64 m = cand_word(T, H, L, st, w, L.bind + lane, 64);
        if (last && !chk)
        {
            mine += lane == 0 ? static_cast<u32>(__popcll(m)) : 0;
            continue;
        }
        if (!((m >> lane) & 1))
            continue;
        L.bind[st.param * 64 + lane] = st.lo + 64 * w + lane;
        if (chk && !checks_ok(T, H, L, st.check_begin, st.check_end, L.bind + lane, 64))
            continue;
        mine += count_from(T, H, L, si + 1, se, lane);
    }
    return wave_sum(mine);
}

/// The successors of schema s: level-synchronous (kLevels) or split over the first step's candidates.
template<bool kLevels>
__device__ __forceinline__ u32 schema_count(const TaskDev& T, const auto& H, const Lds& L, u32 s, u32 lane)
{
    const auto& S = H.schemas[s];
    if (S.never || !checks_ok(T, H, L, S.ground_begin, S.ground_end, L.ub, 1))
        return 0;
    if constexpr (kLevels)
    {
        count_multi(T, H, L, S.plan_begin[0], S.plan_begin[1], 1, lane);
        const u32 c = L.rc[0];
        wave_sync();
        return c;
    }
    else
        return count_wave(T, H, L, S.plan_begin[0], S.plan_begin[1], lane);
}

/// Successors of the state (witness pruning off); the per-schema counts into LDS.
template<bool kLevels>
__device__ __forceinline__ u32 count_all(const TaskDev& T, const auto& H, const Lds& L, u32 lane)
{
    u32 total = 0;
    for (u32 s = 0; s < T.num_schemas; ++s)
    {
        const u32 c = schema_count<kLevels>(T, H, L, s, lane);
        if (lane == 0)
            L.counts[s] = c;
        total += c;
    }
    wave_sync();
    return total;
}

/// The successor counts after a move by an action of schema `applied` from the state whose counts L.counts holds: a
/// schema the action cannot affect (DevSchema::affects) keeps its count, the others are counted again.
template<bool kLevels>
__device__ __forceinline__ u32 count_after(const TaskDev& T, const auto& H, const Lds& L, u32 lane, u32 applied)
{
    const u32 mask = H.schemas[applied].affects;
    u32 total = 0;
    for (u32 s = 0; s < T.num_schemas; ++s)
    {
        u32 c;
        if (s >= 32 || ((mask >> s) & 1))
        {
            c = schema_count<kLevels>(T, H, L, s, lane);
            if (lane == 0)
                L.counts[s] = c;
        }
        else
            c = L.counts[s];
        total += c;
    }
    wave_sync();
    return total;
}

/// The per-env goal test (mask_goal, src/mymyr/rl/env.cpp:55-61): the LDS row against a row of goal masks.
__device__ __forceinline__ bool mask_goal(const lds<u64>* row, const u64* gp, const u64* gn, u32 W, u32 lane)
{
    bool ok = true;
    for (u32 w = lane; w < W; w += kWave)
    {
        const u64 x = row[w];
        ok = ok && (x & gp[w]) == gp[w] && (x & gn[w]) == 0;
    }
    return __ballot(!ok) == 0;
}

/// Whether a row of goal masks sets only the task's fluent slots (words past W and bits past the last slot clear).
__device__ __forceinline__ bool goal_masks_fit(const u64* gp, const u64* gn, u32 words, const TaskDev& T, u32 lane)
{
    bool fit = true;
    for (u32 w = lane; w < words; w += kWave)
    {
        const u64 x = gp[w] | gn[w];
        if (w >= T.W)
            fit = fit && x == 0;
        else if (w == T.W - 1 && (T.fluent_slots & 63))
            fit = fit && (x >> (T.fluent_slots & 63)) == 0;
    }
    return __ballot(!fit) == 0;
}

/// A 64-bit fingerprint of the state (the count cache's check that a row still holds the state its counts are of).
__device__ __forceinline__ u64 state_fingerprint(const lds<u64>* row, u32 W, u32 lane)
{
    u64 acc = 0;
    for (u32 w = lane; w < W; w += kWave)
        acc += mix64(row[w] ^ (static_cast<u64>(w + 1) * 0x9E3779B97F4A7C15ull));
    return wave_sum64(acc);
}

/// The per-schema counts of a count-cache row into LDS; returns their total.
__device__ __forceinline__ u32 load_counts(const TaskDev& T, const Lds& L, const u32* crow, u32 lane)
{
    u32 part = 0;
    for (u32 s = lane; s < T.num_schemas; s += kWave)
    {
        const u32 c = crow[s];
        L.counts[s] = c;
        part += c;
    }
    wave_sync();
    return wave_sum(part);
}

/// A count-cache row of `cw` words from the per-schema counts in LDS (zeros past the instance's schemas, as for a
/// suite's narrower domains) and the fingerprint of the LDS state plus the instance's salt in its last two words.
__device__ __forceinline__ void store_counts(const TaskDev& T, const Lds& L, u32* crow, u32 cw, u32 lane, u64 salt)
{
    const u64 fp = state_fingerprint(L.row, T.W, lane) + salt;
    for (u32 s = lane; s < cw - 2; s += kWave)
        crow[s] = s < T.num_schemas ? L.counts[s] : 0;
    if (lane == 0)
    {
        crow[cw - 2] = static_cast<u32>(fp);
        crow[cw - 1] = static_cast<u32>(fp >> 32);
    }
}

/// The schema holding successor `a` (< total) and the rank within it.
__device__ __forceinline__ void select_schema(const TaskDev& T, const Lds& L, u32 a, u32* schema, u32* rank)
{
    for (u32 s = 0; s < T.num_schemas; ++s)
    {
        const u32 c = L.counts[s];
        if (a < c)
        {
            *schema = s;
            *rank = a;
            return;
        }
        a -= c;
    }
    *schema = kNone;
    *rank = 0;
}

/// The rank-th applicable binding of schema s in lexicographic order into L.ub. false: not found. Per parameter i in
/// order, each window word of its candidates (given parameters [0, i) in L.ub) makes up to 64 roots whose completions
/// count_multi counts; the prefix over the roots in object order locates the rank.
__device__ __forceinline__ bool pick_levels(const TaskDev& T, const auto& H, const Lds& L, u32 s, u32 rank, u32 lane)
{
    const auto& S = H.schemas[s];
    const u32 A = T.label_width ? T.label_width : 1;
    u32 a = rank;
    for (u32 i = 0; i < S.arity; ++i)
    {
        const DevStep F = ld(H.steps + S.filter_step[i]);
        const u32 pb = S.plan_begin[i + 1], pe = S.plan_begin[i + 2];
        const bool chk = F.check_begin != F.check_end;
        const bool found = for_nonzero_words(T, H, L, F, 0, L.ub, 1, lane, [&](u32 w, u64 m) {
            if (chk)
            {
                // lane b checks candidate b
                bool ok = false;
                if ((m >> lane) & 1)
                {
                    for (u32 q = 0; q < A; ++q)
                        L.bind[q * 64 + lane] = L.ub[q];
                    L.bind[i * 64 + lane] = F.lo + 64 * w + lane;
                    ok = checks_ok(T, H, L, F.check_begin, F.check_end, L.bind + lane, 64);
                }
                m = __ballot(ok);
            }
            if (m == 0)
                return false;
            const u32 nr = static_cast<u32>(__popcll(m));
            // root r = the r-th candidate in object order
            if ((m >> lane) & 1)
            {
                const u32 r = static_cast<u32>(__popcll(m & ((u64{1} << lane) - 1)));
                for (u32 q = 0; q < A; ++q)
                    L.qa[r * A + q] = L.ub[q];
                L.qa[r * A + i] = F.lo + 64 * w + lane;
                L.robj[r] = F.lo + 64 * w + lane;
            }
            wave_sync();
            count_multi(T, H, L, pb, pe, nr, lane);
            const u32 c = lane < nr ? L.rc[lane] : 0;
            const u32 incl = wave_inclusive(c);
            const u32 tot = __shfl(incl, kWave - 1, kWave);
            bool hit = false;
            if (a < tot)
            {
                const u64 over = __ballot(incl > a);
                const u32 win = static_cast<u32>(__builtin_ctzll(over));
                a -= __shfl(incl - c, win, kWave);
                const u32 obj = L.robj[win];
                wave_sync();
                if (lane == 0)
                    L.ub[i] = obj;
                hit = true;
            }
            else
                a -= tot;
            wave_sync();
            return hit;
        });
        if (!found)
            return false;
    }
    return true;
}

/// The rank-th applicable binding of schema s in lexicographic order into L.ub, by prefix counting over the lanes:
/// per parameter i, lane b takes candidate b of each window word and completes it with the nested loop.
__device__ __forceinline__ bool pick_lanes(const TaskDev& T, const auto& H, const Lds& L, u32 s, u32 rank, u32 lane)
{
    const auto& S = H.schemas[s];
    u32 a = rank;
    for (u32 i = 0; i < S.arity; ++i)
    {
        const DevStep F = ld(H.steps + S.filter_step[i]);
        const u32 pb = S.plan_begin[i + 1], pe = S.plan_begin[i + 2];
        const bool chk = F.check_begin != F.check_end;
        bool found = false;
        for (u32 w = 0; w < F.words && !found; ++w)
        {
            const u64 m = cand_word(T, H, L, F, w, L.bind + lane, 64);
            u32 c = 0;
            if ((m >> lane) & 1)
            {
                L.bind[i * 64 + lane] = F.lo + 64 * w + lane;
                if (!chk || checks_ok(T, H, L, F.check_begin, F.check_end, L.bind + lane, 64))
                    c = count_from(T, H, L, pb, pe, lane);
            }
            const u32 incl = wave_inclusive(c);
            const u32 tot = __shfl(incl, kWave - 1, kWave);
            if (a < tot)
            {
                const u64 over = __ballot(incl > a);
                const u32 win = static_cast<u32>(__builtin_ctzll(over));
                a -= __shfl(incl - c, win, kWave);
                L.bind[i * 64 + lane] = F.lo + 64 * w + win;
                found = true;
            }
            else
                a -= tot;
        }
        if (!found)
            return false;
    }
    wave_sync();
    if (lane < S.arity)
        L.ub[lane] = L.bind[lane * 64];
    wave_sync();
    return true;
}

/// Whether the binding in L.ub (parameters [0, arity)) of schema s is applicable, for a schema with at least one
/// applicable binding (its ground preconditions hold): parameter i's object is a candidate of its filter step given
/// parameters [0, i), the test that makes a picked binding applicable (every precondition is checked at the step of its
/// last parameter). Wave-uniform.
__device__ __forceinline__ bool label_applicable(const TaskDev& T, const auto& H, const Lds& L, u32 s)
{
    const auto& S = H.schemas[s];
    for (u32 i = 0; i < S.arity; ++i)
    {
        const DevStep F = ld(H.steps + S.filter_step[i]);
        const u32 o = L.ub[i];
        if (o < F.lo || o - F.lo >= 64 * F.words)
            return false;
        const u32 w = (o - F.lo) >> 6, b = (o - F.lo) & 63;
        if (!((cand_word(T, H, L, F, w, L.ub, 1) >> b) & 1))
            return false;
        if (F.check_begin != F.check_end && !checks_ok(T, H, L, F.check_begin, F.check_end, L.ub, 1))
            return false;
    }
    return true;
}

/// Witness pruning (include/mymyr/successor/detail/engine.hpp:345-356): whether the witness objects of the full binding
/// in L.ub are the ones the reference's matcher binds first for its effect-relevant objects, i.e. the first completion
/// of the witnesses in the matcher's witness order, each witness taking its lowest object that the later ones can
/// complete. Per witness t, lane b tests candidate b of each window word (its checks, then whether the count plan of
/// the later witnesses finds a completion); the lowest passing candidate is the matcher's, and the binding is not the
/// one emitted as soon as one differs. The lanes' binding columns hold L.ub again on return. Wave-uniform.
__device__ __forceinline__ bool witness_first(const TaskDev& T, const auto& H, const Lds& L, const DevWitness* X, u32 arity, u32 lane)
{
    for (u32 q = 0; q < arity; ++q)
        L.bind[q * 64 + lane] = L.ub[q];
    const u32 n = X->n;
    bool first = true;
    for (u32 t = 0; t < n && first; ++t)
    {
        const u32 v = X->param[t];
        const DevStep F = ld(H.steps + X->filter[t]);
        const u32 lo = X->plan_lo[t], hi = X->plan_hi[t];
        u32 found = kNone;
        for (u32 w = 0; w < F.words && found == kNone; ++w)
        {
            const u64 m = cand_word(T, H, L, F, w, L.bind + lane, 64);
            bool ok = false;
            if ((m >> lane) & 1)
            {
                L.bind[v * 64 + lane] = F.lo + 64 * w + lane;
                ok = F.check_begin == F.check_end || checks_ok(T, H, L, F.check_begin, F.check_end, L.bind + lane, 64);
                if (ok && lo != hi)
                    ok = count_from(T, H, L, lo, hi, lane) != 0;
            }
            const u64 okm = __ballot(ok);
            if (okm)
                found = F.lo + 64 * w + static_cast<u32>(__builtin_ctzll(okm));
        }
        first = found == L.ub[v];
        L.bind[v * 64 + lane] = found;
    }
    for (u32 q = 0; q < arity; ++q)
        L.bind[q * 64 + lane] = L.ub[q];
    wave_sync();
    return first;
}

/// Calls emit(k, s) for the successors of the state in canonical order (schema, then lexicographic binding),
/// k = 0, 1, ...; L.ub holds the binding during the call, and emit returns false to stop. Each schema with successors
/// (L.counts from count_all) is enumerated depth first over its parameters in order, so the bindings come in the order
/// pick(rank) finds them for rank 0, 1, .... A level takes the window words of its parameter's filter step one at a
/// time: lane b tests candidate b against the step's checks and counts its completions over the rest of the plan (as
/// pick does), and only candidates with completions are visited, lowest first; the leaf level emits its candidates.
/// Counting thus happens once per node of the binding tree instead of once per successor and parameter. The levels'
/// words and candidates left live in L.dfs_w / L.dfs_m; L.bind holds the binding's prefix in every lane's column.
/// Returns the successors enumerated.
template<bool kLevels, bool kWitness = false, class Emit>
__device__ __forceinline__ u32 for_each_successor(const TaskDev& T, const auto& H, const Lds& L, u32 lane, Emit&& emit, u32 s_begin = 0,
                                                  u32 s_end = kNone)
{
    const u32 A = T.label_width ? T.label_width : 1;
    u32 k = 0;
    for (u32 s = s_begin; s < T.num_schemas && s < s_end; ++s)
    {
        if (L.counts[s] == 0)
            continue;
        const auto& S = H.schemas[s];
        // witness pruning: only the full bindings whose witnesses the matcher binds first are successors
        [[maybe_unused]] const DevWitness* X = nullptr;
        if constexpr (kWitness)
            X = (T.witness && T.witness[s].n) ? T.witness + s : nullptr;
        if (S.arity == 0)
        {
            if (!emit(k++, s))
                return k;
            continue;
        }
        // the candidates of parameter i in word w (candidate word m) with at least one completion (wave-uniform mask)
        auto live_mask = [&](u32 i, u32 w, u64 m) -> u64 {
            const DevStep F = ld(H.steps + S.filter_step[i]);
            bool live = false;
            if ((m >> lane) & 1)
            {
                L.bind[i * 64 + lane] = F.lo + 64 * w + lane;
                live = F.check_begin == F.check_end || checks_ok(T, H, L, F.check_begin, F.check_end, L.bind + lane, 64);
                if (live && i + 1 < S.arity)
                    live = count_from(T, H, L, S.plan_begin[i + 1], S.plan_begin[i + 2], lane) != 0;
            }
            return __ballot(live);
        };
        auto word_mask = [&](u32 i, u32 w) -> u64 {
            const DevStep F = ld(H.steps + S.filter_step[i]);
            const u64 m = cand_word(T, H, L, F, w, L.bind + lane, 64);
            bool live = false;
            if ((m >> lane) & 1)
            {
                L.bind[i * 64 + lane] = F.lo + 64 * w + lane;
                live = F.check_begin == F.check_end || checks_ok(T, H, L, F.check_begin, F.check_end, L.bind + lane, 64);
                if (live && i + 1 < S.arity)
                    live = count_from(T, H, L, S.plan_begin[i + 1], S.plan_begin[i + 2], lane) != 0;
            }
            return __ballot(live);
        };
        // parameter i from its first word with live candidates (false: none). Tasks with wide candidate windows (the
        // level-synchronous kernels) skip empty words 64 at a time; the split kernels' narrow windows go word by word.
        auto open = [&](u32 i, u32 w0) -> bool {
            const DevStep F = ld(H.steps + S.filter_step[i]);
            if constexpr (kLevels)
                return for_nonzero_words(T, H, L, F, w0, L.bind + lane, 64, lane, [&](u32 w, u64 cm) {
                    const u64 m = live_mask(i, w, cm);
                    if (!m)
                        return false;
                    wave_sync();
                    if (lane == 0)
                    {
                        L.dfs_m[i] = m;
                        L.dfs_w[i] = w;
                    }
                    wave_sync();
                    return true;
                });
            else
            {
                for (u32 w = w0; w < F.words; ++w)
                {
                    const u64 m = word_mask(i, w);
                    if (m)
                    {
                        wave_sync();
                        if (lane == 0)
                        {
                            L.dfs_m[i] = m;
                            L.dfs_w[i] = w;
                        }
                        wave_sync();
                        return true;
                    }
                }
                return false;
            }
        };
        u32 i = 0;
        bool have = open(0, 0);
        for (;;)
        {
            if (!have)
            {
                if (i == 0)
                    break;
                --i;
                have = L.dfs_m[i] != 0 || open(i, L.dfs_w[i] + 1);
                continue;
            }
            // the level's lowest live candidate
            const u64 m = L.dfs_m[i];
            const u32 w = L.dfs_w[i];
            const u32 o = ld(H.steps + S.filter_step[i]).lo + 64 * w + static_cast<u32>(__builtin_ctzll(m));
            wave_sync();
            if (lane == 0)
            {
                L.dfs_m[i] = m & (m - 1);
                L.ub[i] = o;
            }
            L.bind[i * 64 + lane] = o;
            for (u32 q = 0; q < i && q < A; ++q)
                L.bind[q * 64 + lane] = L.ub[q];
            wave_sync();
            if (i + 1 == S.arity)
            {
                bool take = true;
                if constexpr (kWitness)
                    take = !X || witness_first(T, H, L, X, S.arity, lane);
                if (take && !emit(k++, s))
                    return k;
                have = L.dfs_m[i] != 0 || open(i, w + 1);
                continue;
            }
            ++i;
            have = open(i, 0);
        }
    }
    return k;
}

template<bool kLevels>
__device__ __forceinline__ bool pick(const TaskDev& T, const auto& H, const Lds& L, u32 s, u32 rank, u32 lane)
{
    if constexpr (kLevels)
        return pick_levels(T, H, L, s, rank, lane);
    else
        return pick_lanes(T, H, L, s, rank, lane);
}

/// The slot of an effect's atom under the wave's binding (kNone: none); its canonical id in *cid.
__device__ __forceinline__ u32 effect_slot(const TaskDev& T, const Lds& L, const auto& e, u64* cid_out)
{
    u64 cid = e.base;
    for (u32 v = 0; v < e.nvar; ++v)
        cid += T.rs[static_cast<u64>(e.var_pos[v]) * T.n + L.ub[e.var_param[v]]];
    *cid_out = cid;
    if (cid >= T.fluent_count)
        return kNone;
    return T.dense ? static_cast<u32>(cid) : T.slot_of[cid];
}

/// An added atom without a slot: an error under frozen slots; lazy slots record it for the host to intern (the
/// successor written is then incomplete, and the launch is repeated once the atom has a slot).
__device__ __forceinline__ void missing_atom(const TaskDev& T, u64 cid, u32* status)
{
    if (T.missing && cid < T.fluent_count)
        atomicOr(reinterpret_cast<unsigned long long*>(T.missing + (cid >> 6)), 1ull << (cid & 63));
    atomicOr(status, kStatusNoSlot);
}

/// Predicate and the first two arguments of atom slot s: arithmetic for dense slots over contiguous domains, else the
/// slot's record.
__device__ __forceinline__ void decode_slot(const TaskDev& T, const auto& H, u32 s, u32* pred, u32* a0, u32* a1)
{
    if (T.decode_arith)
    {
        u32 k = 0;
        while (k + 1 < T.num_decode && H.decode[k + 1].offset <= s)
            ++k;
        const auto& d = H.decode[k];
        const u32 rem = static_cast<u32>(s - d.offset);
        *pred = d.pred;
        if (d.arity >= 2)
        {
            const u32 r0 = rem / d.d1;
            *a0 = d.lo0 + r0;
            *a1 = d.lo1 + (rem - r0 * d.d1);
        }
        else
        {
            *a0 = d.lo0 + rem;
            *a1 = 0;
        }
        return;
    }
    const u64 rec = T.records[s];
    *pred = static_cast<u32>(rec & 0xFFFF);
    *a0 = static_cast<u32>((rec >> 16) & 0xFFFF);
    *a1 = static_cast<u32>((rec >> 32) & 0xFFFF);
}

/// The view word and bit of atom (pred, a0, a1) in the non-bulk pairs of its predicate: calls f(word pointer, bit).
template<class F>
__device__ __forceinline__ void for_view_bits(const auto& H, const Lds& L, u32 pred, u32 a0, u32 a1, F&& f)
{
    const u64 pp = H.pred_pairs[pred];
    if (pp == ~u64{0})
        return;
    const u32 ar = H.pred_arity[pred];
    for (int d = 0; d < 2; ++d)
    {
        const u32 pi = d == 0 ? static_cast<u32>(pp) : static_cast<u32>(pp >> 32);
        if (pi == kNone)
            continue;
        const auto& P = H.pairs[pi];
        if (P.bulk)
            continue;
        u32 ri, bi;
        if (ar == 1)
        {
            ri = 0;
            bi = a0 - P.dst_lo;
        }
        else if (d == 0)
        {
            ri = a0 - P.src_lo;
            bi = a1 - P.dst_lo;
        }
        else
        {
            ri = a1 - P.src_lo;
            bi = a0 - P.dst_lo;
        }
        f(L.view + P.offset + static_cast<u64>(ri) * P.dst_words + (bi >> 6), u64{1} << (bi & 63));
    }
}

/// Builds the view of the wave's row (all lanes). With kByPredicate and arithmetic slot decoding the row is read
/// predicate by predicate: only the slot ranges of predicates with scattered view rows, each with its decoding and its
/// two pairs read once (the level-synchronous kernels, whose wide rows hold many atoms); otherwise every set bit is
/// decoded on its own (the split kernels keep this shorter code: the other costs them registers for little).
template<bool kByPredicate>
__device__ __forceinline__ void build_view(const TaskDev& T, const auto& H, const Lds& L, u32 lane)
{
    for (u32 k = lane; k < T.view_words; k += kWave)
        L.view[k] = 0;
    wave_sync();
    if (kByPredicate && T.decode_arith)
    {
        for (u32 k = 0; k < T.num_decode; ++k)
        {
            const DevPredDecode d = ld(H.decode + k);
            const u64 end = min(d.offset + d.size, static_cast<u64>(T.fluent_slots));
            if (!d.has_scatter || end <= d.offset)
                continue;
            // the predicate's scattered pairs: forward (or unary) and backward
            const u64 pp = H.pred_pairs[d.pred];
            const u32 ar = H.pred_arity[d.pred];
            u32 on[2], off[2], src_lo[2], dst_lo[2], dst_words[2];
#pragma unroll
            for (int q = 0; q < 2; ++q)
            {
                const u32 pi = q == 0 ? static_cast<u32>(pp) : static_cast<u32>(pp >> 32);
                on[q] = 0;
                off[q] = src_lo[q] = dst_lo[q] = dst_words[q] = 0;
                if (pp != ~u64{0} && pi != kNone)
                {
                    const DevPair P = ld(H.pairs + pi);
                    on[q] = P.bulk ? 0 : 1;
                    off[q] = P.offset;
                    src_lo[q] = P.src_lo;
                    dst_lo[q] = P.dst_lo;
                    dst_words[q] = P.dst_words;
                }
            }
            const u32 w0 = static_cast<u32>(d.offset >> 6), w1 = static_cast<u32>((end - 1) >> 6);
            for (u32 w = w0 + lane; w <= w1; w += kWave)
            {
                u64 x = L.row[w];
                if (w == w0)
                    x &= ~u64{0} << (d.offset & 63);
                if (w == w1 && (end & 63))
                    x &= (u64{1} << (end & 63)) - 1;
                while (x)
                {
                    const u32 rem = static_cast<u32>(w * 64 + static_cast<u32>(__builtin_ctzll(x)) - d.offset);
                    x &= x - 1;
                    u32 a0, a1;
                    if (d.arity >= 2)
                    {
                        const u32 r0 = rem / d.d1;
                        a0 = d.lo0 + r0;
                        a1 = d.lo1 + (rem - r0 * d.d1);
                    }
                    else
                    {
                        a0 = d.lo0 + rem;
                        a1 = 0;
                    }
                    // the atom's bits in the pairs' rows, as for_view_bits places them
#pragma unroll
                    for (int q = 0; q < 2; ++q)
                    {
                        if (!on[q])
                            continue;
                        u32 ri, bi;
                        if (ar == 1)
                        {
                            ri = 0;
                            bi = a0 - dst_lo[q];
                        }
                        else if (q == 0)
                        {
                            ri = a0 - src_lo[q];
                            bi = a1 - dst_lo[q];
                        }
                        else
                        {
                            ri = a1 - src_lo[q];
                            bi = a0 - dst_lo[q];
                        }
                        __hip_atomic_fetch_or(L.view + off[q] + static_cast<u64>(ri) * dst_words[q] + (bi >> 6), u64{1} << (bi & 63),
                                              __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                    }
                }
            }
        }
        wave_sync();
        return;
    }
    for (u32 w = lane; w < T.W; w += kWave)
    {
        u64 x = L.row[w];
        while (x)
        {
            const u32 s = w * 64 + static_cast<u32>(__builtin_ctzll(x));
            x &= x - 1;
            if (s >= T.fluent_slots)
                break;  // bits past the task's slots belong to no atom
            u32 pred, a0, a1;
            decode_slot(T, H, s, &pred, &a0, &a1);
            for_view_bits(H, L, pred, a0, a1, [](lds<u64>* word, u64 bit) {
                __hip_atomic_fetch_or(word, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            });
        }
    }
    wave_sync();
}

/// Loads row i (W words of `words`) into the wave's LDS row.
__device__ __forceinline__ void load_row_lds(const TaskDev& T, const Lds& L, const u64* src, u32 lane)
{
    if (T.W <= kWave)  // one load per lane
    {
        if (lane < T.W)
            L.row[lane] = src[lane];
        wave_sync();
        return;
    }
    // up to 8 loads of a lane in flight before their LDS stores: a wide row arrives in about one load latency
    constexpr u32 kBatch = 8;
    for (u32 k0 = 0; k0 < T.W; k0 += kBatch * kWave)
    {
        u64 v[kBatch];
#pragma unroll
        for (u32 j = 0; j < kBatch; ++j)
        {
            const u32 k = k0 + j * kWave + lane;
            v[j] = k < T.W ? src[k] : 0;
        }
#pragma unroll
        for (u32 j = 0; j < kBatch; ++j)
        {
            const u32 k = k0 + j * kWave + lane;
            if (k < T.W)
                L.row[k] = v[j];
        }
    }
    wave_sync();
}

/// Loads the first n words of a row into the wave's LDS row and zeroes the rest of its T.W words (rows narrower than
/// the task: a lazy task's rows grow as atoms intern).
__device__ __forceinline__ void load_row_lds_n(const TaskDev& T, const Lds& L, const u64* src, u32 n, u32 lane)
{
    for (u32 k = lane; k < T.W; k += kWave)
        L.row[k] = k < n ? src[k] : 0;
    wave_sync();
}

/// dst[k] = k < n ? src[k] : 0 for k < z (global to global), up to 8 loads of a lane in flight.
__device__ __forceinline__ void copy_words(u64* dst, const u64* src, u32 n, u32 z, u32 lane)
{
    if (z <= kWave)  // one word per lane
    {
        if (lane < z)
            dst[lane] = lane < n ? src[lane] : 0;
        return;
    }
    constexpr u32 kBatch = 8;
    for (u32 k0 = 0; k0 < z; k0 += kBatch * kWave)
    {
        u64 v[kBatch];
#pragma unroll
        for (u32 j = 0; j < kBatch; ++j)
        {
            const u32 k = k0 + j * kWave + lane;
            v[j] = k < n ? src[k] : 0;
        }
#pragma unroll
        for (u32 j = 0; j < kBatch; ++j)
        {
            const u32 k = k0 + j * kWave + lane;
            if (k < z)
                dst[k] = v[j];
        }
    }
}

/// The ascending set-bit slots of `row` (W words) into out[0, max_atoms), -1 padded (all lanes). A lane takes kPer
/// consecutive words per round (one wave scan per kPer * 64 words; wide rows take 4); a lane's atoms are consecutive
/// in the output, and the lanes' ranges follow each other.
template<u32 kPer = 1, class P>
__device__ __forceinline__ void encode_row(P row, u32 W, i32* out, u32 max_atoms, u32 lane, u32* status)
{
    u32 base = 0;
    for (u32 w0 = 0; w0 < W; w0 += kWave * kPer)
    {
        const u32 wl = w0 + lane * kPer;
        u64 x[kPer];
        u32 c = 0;
#pragma unroll
        for (u32 j = 0; j < kPer; ++j)
        {
            x[j] = wl + j < W ? row[wl + j] : 0;
            c += static_cast<u32>(__popcll(x[j]));
        }
        const u32 incl = wave_inclusive(c);
        u32 k = base + incl - c;
#pragma unroll
        for (u32 j = 0; j < kPer; ++j)
            for (u64 y = x[j]; y; y &= y - 1)
            {
                if (k < max_atoms)
                    out[k] = static_cast<i32>((wl + j) * 64 + static_cast<u32>(__builtin_ctzll(y)));
                ++k;
            }
        base += __shfl(incl, kWave - 1, kWave);
    }
    for (u32 k = base + lane; k < max_atoms; k += kWave)
        out[k] = -1;
    if (base > max_atoms && lane == 0)
        atomicOr(status, kStatusCapacity);
}

template<class P>
__device__ __forceinline__ bool goal_test(const TaskDev& T, const auto& H, P row, u32 lane)
{
    bool ok = true;
    for (u32 i = lane; i < T.ngp; i += kWave)
        ok = ok && row_bit(row, H.goal_pos[i]);
    for (u32 i = lane; i < T.ngn; i += kWave)
        ok = ok && !row_bit(row, H.goal_neg[i]);
    return !T.goal_unsat && __ballot(!ok) == 0;
}

/// Applies the effects of the picked binding of schema s to the LDS row and the view: delete, then add. One effect per
/// lane: its slot (the table reads of the effects overlap instead of following each other), then the deletes, the adds,
/// and the view bits of the atoms whose bit changed. View pairs exist for predicates of arity 1 and 2 only, so a view bit
/// stands for one atom: lanes that list the same slot write the same value. Returns the lane's effect slot (kNone: no
/// effect or no slot): the row words that can have changed are the words of these slots.
__device__ __forceinline__ u32 apply_effects(const TaskDev& T, const auto& H, const Lds& L, u32 s, u32 lane, u32* status)
{
    const auto& S = H.schemas[s];
    const u32 ne = min(S.eff_end - S.eff_begin, kMaxEff);
    if (lane == 0 && S.eff_end - S.eff_begin > kMaxEff)
        atomicOr(status, kStatusCapacity);
    const bool mine = lane < ne;
    const bool add = lane < S.nadd;
    u32 sl = kNone;
    bool before = false;
    if (mine)
    {
        u64 cid;
        sl = effect_slot(T, L, H.effects[S.eff_begin + lane], &cid);
        before = sl != kNone && row_bit(L.row, sl);
        if (add && sl == kNone)
            missing_atom(T, cid, status);
    }
    wave_sync();
    if (mine && !add && sl != kNone)
        __hip_atomic_fetch_and(L.row + (sl >> 6), ~(u64{1} << (sl & 63)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
    wave_sync();
    if (mine && add && sl != kNone)
        __hip_atomic_fetch_or(L.row + (sl >> 6), u64{1} << (sl & 63), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
    wave_sync();
    if (mine && sl != kNone && sl < T.fluent_slots)
    {
        const bool now = row_bit(L.row, sl);
        if (now != before)
        {
            u32 pred, a0, a1;
            decode_slot(T, H, sl, &pred, &a0, &a1);
            for_view_bits(H, L, pred, a0, a1, [now](lds<u64>* word, u64 bit) {
                if (now)
                    __hip_atomic_fetch_or(word, bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
                else
                    __hip_atomic_fetch_and(word, ~bit, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            });
        }
    }
    wave_sync();
    return sl;
}

/// Whether the task's hot tables are staged in LDS.
bool staged(const TaskDev& T) { return static_cast<u64>(T.hot_words) * 8 <= kHotMax; }

/// Whether counts and picks run level-synchronously (candidate windows of several words, where the lanes' nested
/// loops would walk long word sequences) or split over the lanes.
bool levels(const TaskDev& T) { return T.max_step_words >= 4; }

/// The kernel variant for the task.
template<class F>
F variant(const TaskDev& T, F ss, F sl, F gs, F gl)
{
    return staged(T) ? (levels(T) ? sl : ss) : (levels(T) ? gl : gs);
}

bool levels(const TaskDev& T);

/// The waves per block that keep the most waves resident on a CU (its 160 KiB of LDS shared by whole blocks), for
/// hot tables of `hot` bytes staged once per block and `wave` bytes per wave; a smaller block is taken only for at
/// least 1/8 more resident waves (a larger one stages the hot tables fewer times).
unsigned block_shape(size_t hot, size_t wave, size_t* lds_bytes)
{
    constexpr size_t kCuLds = 160 * 1024;
    constexpr int kCuWaves = 24;  // waves per CU the kernels' register use allows
    int nw = 1, best = 0;
    for (int k = kMaxWaves; k >= 1; --k)
    {
        const size_t block = hot + static_cast<size_t>(k) * wave;
        if (block > kCuLds)
            continue;
        const int resident = std::min(kCuWaves, k * static_cast<int>(kCuLds / block));
        if (8 * resident > 9 * best)
        {
            best = resident;
            nw = k;
        }
    }
    *lds_bytes = hot + static_cast<size_t>(nw) * wave;
    if (*lds_bytes > kCuLds)
        throw std::invalid_argument("mymyr_amd: env: the task's per-state LDS (" + std::to_string(*lds_bytes) +
                                    " bytes) exceeds the 160 KiB of a gfx950 workgroup");
    return static_cast<unsigned>(nw);
}

void check_schemas(const TaskDev& T)
{
    if (T.num_schemas > kMaxEnvSchemas)
        throw std::invalid_argument("mymyr_amd: env: the device step keeps the successor counts of at most " + std::to_string(kMaxEnvSchemas) +
                                    " schemas (the task has " + std::to_string(T.num_schemas) + ")");
}

unsigned waves_per_block(const TaskDev& T, size_t* lds_bytes)
{
    check_schemas(T);
    const size_t hot = staged(T) ? static_cast<size_t>(T.hot_words) * 8 : 0, wave = static_cast<size_t>(wave_lds_words(T, levels(T))) * 8;
    return block_shape(hot, wave, lds_bytes);
}

/// hash_state of a row (its trimmed words; include/mymyr/core/hash.hpp:56-60), one lane.
template<class P>
__device__ __forceinline__ u64 row_hash(P row, u32 W)
{
    u32 n = W;
    while (n > 0 && row[n - 1] == 0)
        --n;
    u64 h = kHashSeed ^ (static_cast<u64>(n) * kHashP1);
    u32 k = 0;
    for (; k + 1 < n; k += 2)
        h = mulfold(h ^ row[k] ^ kHashP1, row[k + 1] ^ kHashP2);
    if (k < n)
        h = mulfold(h ^ row[k] ^ kHashP1, kHashP2);
    return mix64(h);
}

constexpr u64 kVisitedZero = 0x9E3779B97F4A7C15ull;  // the key of hash 0 (0 marks an empty slot)

/// visited_insert (include/mymyr/rl/visited.hpp:31-52), one lane: whether the key was present; a new key above
/// floor(3H/4) entries is skipped and the count saturates at H.
__device__ __forceinline__ bool visited_insert(u64* table, u32 H, i32& count, u64 hash)
{
    const u64 key = hash ? hash : kVisitedZero;
    u32 at = static_cast<u32>(key) & (H - 1);
    for (u32 probe = 0; probe < H; ++probe, at = (at + 1) & (H - 1))
    {
        const u64 x = table[at];
        if (x == key)
            return true;
        if (!x)
        {
            if (count >= static_cast<i32>((static_cast<u64>(H) * 3) / 4))
                count = static_cast<i32>(H);
            else
            {
                table[at] = key;
                ++count;
            }
            return false;
        }
    }
    count = static_cast<i32>(H);
    return false;
}

/// visited_clear + visited_insert of one hash over a row's table (all lanes; every slot written once, the key's own
/// slot with the key); the count becomes 1 (lane 0).
__device__ __forceinline__ void visited_restart(u64* table, u32 H, i32* count, u64 hash, u32 lane)
{
    const u64 key = hash ? hash : kVisitedZero;
    const u32 at = static_cast<u32>(key) & (H - 1);
    for (u32 q = lane; q < H; q += kWave)
        table[q] = q == at ? key : 0;
    if (lane == 0)
        *count = 1;
}

/// visited_mask (include/mymyr/rl/visited.hpp:63-74), one lane per successor: whether succ_hash[j] is in the table of
/// row parent[j] (or rows[parent[j]]). Padding (-1) and parents or rows outside the tables read as not visited.
__global__ __launch_bounds__(256) void k_visited_mask(const u64* table, const i32* count, u64 table_rows, u32 H, const u64* succ_hash,
                                                      const i32* parent, const i32* rows, u64 parents, u64 size, u8* out)
{
    const u64 stride = u64{gridDim.x} * blockDim.x;
    for (u64 j = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; j < size; j += stride)
    {
        const i32 p = parent[j];
        bool hit = false;
        const i32 row = p < 0 || static_cast<u64>(p) >= parents ? -1 : rows ? rows[p] : p;
        if (row >= 0 && static_cast<u64>(row) < table_rows && count[row])
        {
            const u64 h = succ_hash[j], key = h ? h : kVisitedZero;
            const u64* t = table + static_cast<u64>(row) * H;
            u32 at = static_cast<u32>(key) & (H - 1);
            for (u32 probe = 0; probe < H; ++probe, at = (at + 1) & (H - 1))
            {
                const u64 x = t[at];
                if (x == key)
                {
                    hit = true;
                    break;
                }
                if (!x)
                    break;
            }
        }
        out[j] = hit ? 1 : 0;
    }
}

/// One environment's step (HostEnv::step_row_impl, src/mymyr/rl/env.cpp:351-528): row i of instance k, whose tables
/// are T / H and whose wave region is L. An autoreset restarts the row in next_task_ids[i] when that names an instance
/// (else in k), writing the new instance's initial state and goal masks over the words the row may have dirtied
/// (TaskSuite::initial_row, src/mymyr/rl/task_suite.cpp:130-138) and its id into task_ids.
template<bool kLevels, bool kOne, bool kVisited, bool kPlain = false>
__device__ __forceinline__ void step_row(const EnvArgs& A, const TaskDev& T, const auto& H, const Lds& L, u64 i, u32 k, u32 lane, u64 seed)
{
    static_assert(!kPlain || (kOne && !kVisited), "the plain step is a one-instance step without visited tables");
    // the plain step (an env pool's step: the random policy over one instance, the env's RNG key and env ids first_env +
    // row, the task's goal, steps and draws kept, no labels or final states) knows the optional inputs it does not
    // take at compile time, so their pointers and tests take no registers
    const i64* const actions = kPlain ? nullptr : A.actions;
    const i32* const label_schema = kPlain ? nullptr : A.label_schema;
    const u64* const seeds = kPlain ? nullptr : A.seeds;
    const u32* const env_ids = kPlain ? nullptr : A.env_ids;
    const u64* const goal_pos = kPlain ? nullptr : A.goal_pos;
    u64* const final_states = kPlain ? nullptr : A.final_states;
    u32* const reset_counts = kPlain ? nullptr : A.reset_counts;
    i32* const steps = A.steps;
    u64* const draws = A.draws;
    const bool have_steps = kPlain || A.steps != nullptr;
    const bool have_draws = kPlain || A.draws != nullptr;
    const u32 Lw = A.label_width;
    u64* grow = A.states + i * A.words;
    // the row's scalars are read before its words, so that their latencies overlap with the row's
    const bool already_goal = A.at_goal[i] != 0;
    const i64 act_in = actions ? actions[i] : 0;
    const u64 draws0 = have_draws ? draws[i] : 0;
    const i32 steps0 = have_steps ? steps[i] : 0;
    const i32 next_in = (!kOne && A.next_task_ids) ? A.next_task_ids[i] : 0;
    const i32 label_in = label_schema ? label_schema[i] : -1;
    // the count cache row: its counts stand for the row's state (and instance) when its fingerprint matches (reset,
    // refresh and step write it; a state written directly since is counted again)
    const u32 cw = A.cache_width;
    u32* crow = A.counts ? A.counts + i * cw : nullptr;
    const u64 fp_cached = crow ? (static_cast<u64>(crow[cw - 2]) | (static_cast<u64>(crow[cw - 1]) << 32)) : 0;
    load_row_lds(T, L, grow, lane);
    build_view<kLevels>(T, H, L, lane);
    const u64 salt = instance_salt(k);
    bool cached = false;
    if (crow)
        cached = fp_cached == state_fingerprint(L.row, T.W, lane) + salt;
    enum
    {
        kOk = 0,
        kStuck = 1,
        kInvalid = 2,
        kGoal = 3
    };
    // phase 0 counts s, chooses, picks and moves; phase 1 counts the reached state s' (one copy of the count)
    u32 c = 0, c2 = 0, st = kOk, schema = kNone;
    u32 moved_slot = kNone;  // the lane's effect slot of the applied move (its word is the only one it can change)
    bool g = already_goal;
    for (u32 phase = 0; phase < 2; ++phase)
    {
        const u32 cc = (phase == 1 && T.num_schemas > 1) ? count_after<kLevels>(T, H, L, lane, schema)
                       : ((phase == 0 && cached) ? load_counts(T, L, crow, lane) : count_all<kLevels>(T, H, L, lane));
        if (phase == 1)
        {
            c2 = cc;
            break;
        }
        c = c2 = cc;
        // 2. the choice (env.cpp:416-440)
        st = already_goal ? kGoal : kOk;
        u32 a = 0;
        bool labelled = false;  // the move is the row's label (no pick)
        if (!already_goal && c == 0)
            st = kStuck;
        else if (!already_goal && label_schema)
        {
            // label mode (env.cpp:376-398, 423-425): the label moves where it is applicable, else the row is invalid
            bool ok = label_in >= 0 && static_cast<u32>(label_in) < T.num_schemas && L.counts[label_in] > 0;
            if (ok)
            {
                const u32 arity = H.schemas[label_in].arity;
                if (lane < arity)
                    L.ub[lane] = static_cast<u32>(A.label_binding[i * A.label_stride + lane]);
                wave_sync();
                ok = label_applicable(T, H, L, static_cast<u32>(label_in));
            }
            if (ok)
            {
                schema = static_cast<u32>(label_in);
                labelled = true;
            }
            else
                st = kInvalid;
        }
        else if (!already_goal && actions)
        {
            const i64 act = act_in;
            if (act < 0 || static_cast<u64>(act) >= c)
                st = kInvalid;
            else
                a = static_cast<u32>(act);
        }
        else if (!already_goal)
        {
            // the key: the row's own, or the env's (read here in the batch-order path, which keeps fewer values live)
            const u64 key = seeds ? seeds[i] : (kOne ? *A.seed : seed);
            a = successor_index(key, env_ids ? static_cast<u64>(env_ids[i]) : A.first_env + i, draws0, c);
        }
        u32 rank = 0;
        if (st == kOk && !labelled)
        {
            select_schema(T, L, a, &schema, &rank);
            if (schema == kNone || !pick<kLevels>(T, H, L, schema, rank, lane))
            {
                if (lane == 0)
                    atomicOr(A.status, kStatusPickFailed);
                st = kStuck;
            }
        }
        if (lane == 0)
        {
            if (have_draws)
                draws[i] = draws0 + 1;
            if (A.schema)
                A.schema[i] = st == kOk ? static_cast<i32>(schema) : -1;
            if (A.invalid)
                A.invalid[i] = st == kInvalid ? 1 : 0;
        }
        if (A.binding)
        {
            const u32 arity = st == kOk ? H.schemas[schema].arity : 0;
            for (u32 q = lane; q < Lw; q += kWave)
                A.binding[i * Lw + q] = (st == kOk && q < arity) ? static_cast<i32>(L.ub[q]) : -1;
        }
        if (st != kOk)
            break;
        // 3. the move, goal and (next phase) the successor count of the reached state
        moved_slot = apply_effects(T, H, L, schema, lane, A.status);
        g = goal_pos ? mask_goal(L.row, goal_pos + i * A.words, A.goal_neg + i * A.words, T.W, lane)
                     : goal_test(T, H, L.row, lane);
    }
    // 4. rewards, termination, truncation (env.cpp:466-485)
    const bool dead = !A.cfg.dead_end_none && !g && ((st == kOk && c2 == 0) || st == kStuck);
    const bool term = g || (dead && A.cfg.dead_end_terminal);
    const bool absorbed = already_goal || (st == kStuck && dead && A.cfg.dead_end_terminal);
    const i32 t2 = have_steps ? steps0 + (absorbed ? 0 : 1) : 0;
    const bool trunc = !term && A.cfg.max_steps && t2 >= static_cast<i32>(A.cfg.max_steps);
    if (lane == 0)
    {
        if (A.reward)
        {
            float r = 0.0f;
            if (!absorbed)
            {
                r = A.cfg.step_reward + (g ? A.cfg.goal_reward : 0.0f);
                r = r + (dead ? A.cfg.dead_end_reward : 0.0f);
            }
            A.reward[i] = r;
        }
        if (A.terminated)
            A.terminated[i] = term ? 1 : 0;
        if (A.truncated)
            A.truncated[i] = trunc ? 1 : 0;
        if (A.goal)
            A.goal[i] = g ? 1 : 0;
    }
    if (final_states)
    {
        const u32 FW = A.final_words;
        u64* f = final_states + i * FW;
        for (u32 q = lane; q < FW; q += kWave)
            f[q] = q < T.W ? L.row[q] : 0;
    }
    // the reached state's key into the row's visited table unless its episode is over without autoreset (env.cpp:487-499)
    if (kVisited && (A.visited.capacity || A.revisited))
    {
        bool revisited = false;
        const bool over = !A.cfg.autoreset && (absorbed || (A.cfg.max_steps && steps0 >= static_cast<i32>(A.cfg.max_steps)));
        if (lane == 0 && A.visited.capacity && !over)
        {
            const u32 H = A.visited.capacity;
            i32 cnt = A.visited.count[i];
            revisited = visited_insert(A.visited.table + i * H, H, cnt, row_hash(L.row, T.W));
            A.visited.count[i] = cnt;
            if (cnt == static_cast<i32>(H))
                atomicOr(A.visited.status + (A.visited.status_per_row ? i : 0), 1);
        }
        if (lane == 0 && A.revisited)
            A.revisited[i] = revisited ? 1 : 0;
        wave_sync();
    }
    // 5. the autoreset, or the bookkeeping of the move (the LDS row holds s'). The instance an autoreset restarts in:
    // next_task_ids[i], where an id outside the table sets the status (in every row, as the reference checks the whole
    // array) and keeps the row's instance
    u32 next = k;
    if (!kOne && A.next_task_ids)
    {
        const i32 v = next_in;
        if (v < 0 || static_cast<u32>(v) >= A.instances)
        {
            if (lane == 0)
                atomicOr(A.status, kStatusTaskId);
        }
        else
            next = static_cast<u32>(v);
    }
    const bool reset = A.cfg.autoreset && (term || trunc);
    if (reset)
    {
        // every autoreset advances the row's reset counter (a sampled restart comes in as next_task_ids, drawn before the
        // step with the counter's value before this advance)
        if (reset_counts && lane == 0)
            reset_counts[i] += 1;
        const InstDev& J = A.inst[next];  // a one-instance env restarts in instance 0
        const u32 z = min(A.words, max(J.W, T.W));  // the words the row may have dirtied: its old and new instance's
        copy_words(grow, J.initial, J.W, z, lane);
        if (goal_pos)
        {
            copy_words(A.goal_pos + i * A.words, J.goal_pos, J.W, z, lane);
            copy_words(A.goal_neg + i * A.words, J.goal_neg, J.W, z, lane);
        }
        if (lane == 0)
        {
            if (!kOne && A.task_ids)
                A.task_ids[i] = static_cast<i32>(next);
            if (A.count)
                A.count[i] = static_cast<i32>(J.init_count);
            A.at_goal[i] = J.init_goal ? 1 : 0;
            if (have_steps)
                steps[i] = 0;
        }
        if (crow)
            for (u32 q = lane; q < cw; q += kWave)
                crow[q] = J.init_cache[q];
        if (kVisited && A.visited.capacity)
            visited_restart(A.visited.table + i * A.visited.capacity, A.visited.capacity, A.visited.count + i, J.init_hash, lane);
    }
    else
    {
        // a move changes only the words of its effects' slots. The level-synchronous kernel (wide candidate windows,
        // rows of up to thousands of words) writes back just those, one per effect lane (lanes sharing a word write the
        // same value); the split kernel copies its row whole, which keeps the slot out of the registers it holds
        // across the count of s' (an extra live value there costs it more than the few stores)
        if constexpr (kLevels)
        {
            if (st == kOk && moved_slot != kNone)
                grow[moved_slot >> 6] = L.row[moved_slot >> 6];
        }
        else if (st == kOk)
            for (u32 q = lane; q < T.W; q += kWave)
                grow[q] = L.row[q];
        if (lane == 0)
        {
            A.at_goal[i] = g ? 1 : 0;
            if (have_steps)
                steps[i] = t2;
            if (A.count)
                A.count[i] = static_cast<i32>(c2);
        }
        // the count cache of the state the row now holds: the counts in LDS (of s' after a move, of s otherwise)
        // unless they came from the cache
        if (crow && (st == kOk || !cached))
            store_counts(T, L, crow, cw, lane, salt);
    }
    // 6. the observation's encoding: true-atom slots and applicable-schema masks (LDS holds the per-schema counts of
    // the state the row holds unless the row was reset)
    if (A.atoms || A.masks)
    {
        wave_sync();
        if (A.atoms)
        {
            if (reset)
                encode_row<kLevels ? 4 : 1>(A.inst[next].initial, A.inst[next].W, A.atoms + i * A.max_atoms,
                           A.max_atoms, lane, A.status);
            else
                encode_row<kLevels ? 4 : 1>(L.row, T.W, A.atoms + i * A.max_atoms, A.max_atoms, lane, A.status);
        }
        if (A.masks)
            for (u32 q = lane; q < A.mask_width; q += kWave)
                A.masks[i * A.mask_width + q] = reset ? A.inst[next].init_masks[q] : (q < T.num_schemas && L.counts[q] > 0 ? 1 : 0);
    }
    wave_sync();
}

/// Waves per SIMD the env step is compiled for: the split count (transport-like tasks) holds 5 at the price of a few
/// spilled registers, faster than the 4 its register use gives unconstrained; the level-synchronous count keeps the 3
/// its registers allow (spills cost it more than a wave gains).
template<bool kLevels>
constexpr int kEnvStepWaves = kLevels ? 3 : 5;

/// The step of a batch of one instance: every row in batch order with the kernel-argument tables, as instance 0 (the
/// host checks given task ids and next_task_ids with launch_check_ids first); with kGroup, the rows of one instance's
/// group of a batch grouped by instance.
template<bool kStaged, bool kLevels, bool kGroup, bool kVisited, bool kPlain = false>
__global__ __launch_bounds__(kMaxWaves * kWave) __attribute__((amdgpu_waves_per_eu(kEnvStepWaves<kLevels>))) void k_env_step(EnvArgs A)
{
    extern __shared__ u64 smem[];
    const TaskDev& T = A.T;
    const u32 lane = lane_id(), wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    if constexpr (kGroup)
    {
        // the rows of instance A.instance of a batch grouped by instance; blocks past them leave before staging
        const u32 lo = A.groups.starts[A.instance], hi = A.groups.starts[A.instance + 1];
        if (lo + static_cast<u64>(blockIdx.x) * nw >= hi)
            return;
        Tab<kStaged> H;
        lds<u64>* waves = stage_hot<kStaged>(smem, T, &H);
        const Lds L = lds_of<kLevels>(waves + static_cast<u64>(wave) * wave_lds_words(T, kLevels), T);
        const u64 seed = *A.seed;
        for (u64 j = lo + static_cast<u64>(blockIdx.x) * nw + wave; j < hi; j += static_cast<u64>(gridDim.x) * nw)
            step_row<kLevels, false, kVisited>(A, T, H, L, A.groups.order[j], A.instance, lane, seed);
    }
    else
    {
        Tab<kStaged> H;
        lds<u64>* waves = stage_hot<kStaged>(smem, T, &H);
        const Lds L = lds_of<kLevels>(waves + static_cast<u64>(wave) * wave_lds_words(T, kLevels), T);
        for (u64 i = static_cast<u64>(blockIdx.x) * nw + wave; i < A.rows; i += static_cast<u64>(gridDim.x) * nw)
            step_row<kLevels, true, kVisited, kPlain>(A, T, H, L, i, 0, lane, 0);
    }
}

/// Instance k's tables, read through the constant address space: loads of them are invariant, so the compiler
/// re-reads a field with a scalar load where it needs it instead of holding the whole record in registers.
__device__ __forceinline__ const TaskDev& instance_tables(const TaskDev* tasks, u32 k)
{
    typedef __attribute__((address_space(4))) const TaskDev ConstTaskDev;
    return *(const TaskDev*)((const ConstTaskDev*)tasks + k);
}

/// The instance of chunk c: the last k with chunk_start[k] <= c (chunk_start is non-decreasing, chunk_start[0] = 0).
__device__ __forceinline__ u32 chunk_instance(const u32* chunk_start, u32 instances, u32 c)
{
    u32 lo = 0, hi = instances;
    while (hi - lo > 1)
    {
        const u32 mid = (lo + hi) / 2;
        if (chunk_start[mid] <= c)
            lo = mid;
        else
            hi = mid;
    }
    return lo;
}

/// The step of the rows of the instances of variant kVariant of a batch grouped by instance: each block takes chunks
/// of kChunkRows rows of one instance, stages that instance's hot tables and steps the chunk's rows (one per wave).
template<bool kStaged, bool kLevels>
__global__ __launch_bounds__(kMaxWaves * kWave) void k_env_step_grouped(EnvArgs A, u32 variant)
{
    extern __shared__ u64 smem[];
    const u32 lane = lane_id(), wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    const u32 chunks = A.groups.chunk_start[A.instances];
    for (u32 c = blockIdx.x; c < chunks; c += gridDim.x)
    {
        const u32 k = chunk_instance(A.groups.chunk_start, A.instances, c);
        if (A.inst[k].variant != variant)
            continue;
        const TaskDev& T = instance_tables(A.tasks, k);
        __syncthreads();  // every wave is done with the tables of the block's previous chunk
        Tab<kStaged> H;
        lds<u64>* waves = stage_hot<kStaged>(smem, T, &H);
        const Lds L = lds_of<kLevels>(waves + static_cast<u64>(wave) * A.wave_words, T);
        const u32 r0 = A.groups.starts[k] + (c - A.groups.chunk_start[k]) * kChunkRows;
        const u32 r1 = min(r0 + kChunkRows, A.groups.starts[k + 1]);
        const u64 seed = *A.seed;
        for (u32 j = r0 + wave; j < r1; j += nw)
            step_row<kLevels, false, true>(A, T, H, L, A.groups.order[j], k, lane, seed);
    }
}

__global__ __launch_bounds__(kWave) void k_encode(const u64* states, u64 rows, u32 words, u32 W, i32* out, u32 max_atoms, u32* status)
{
    const u32 lane = threadIdx.x;
    for (u64 i = blockIdx.x; i < rows; i += gridDim.x)
        encode_row<4>(states + i * words, W, out + i * max_atoms, max_atoms, lane, status);
}

/// The count of row i of instance k (HostEnv::refresh / count_row, src/mymyr/rl/env.cpp:283-322): successors, goal
/// (per-env masks, checked against the instance's slots, or the instance's goal test), masks and the count cache.
template<bool kLevels>
__device__ __forceinline__ void count_row(const CountArgs& A, const TaskDev& T, const auto& H, const Lds& L, u64 i, u32 k, u32 lane)
{
    load_row_lds(T, L, A.states + i * A.words, lane);
    build_view<kLevels>(T, H, L, lane);
    const u32 c = count_all<kLevels>(T, H, L, lane);
    bool g;
    if (A.goal_pos)
    {
        const u64* gp = A.goal_pos + i * A.words;
        const u64* gn = A.goal_neg + i * A.words;
        if (!goal_masks_fit(gp, gn, A.words, T, lane) && lane == 0 && A.status)
            atomicOr(A.status, kStatusGoalMask);
        g = mask_goal(L.row, gp, gn, T.W, lane);
    }
    else
        g = goal_test(T, H, L.row, lane);
    if (lane == 0)
    {
        if (A.count)
            A.count[i] = static_cast<i32>(c);
        if (A.goal)
            A.goal[i] = g ? 1 : 0;
    }
    if (A.masks)
        for (u32 q = lane; q < A.mask_width; q += kWave)
            A.masks[i * A.mask_width + q] = q < T.num_schemas && L.counts[q] > 0 ? 1 : 0;
    if (A.cache)
        store_counts(T, L, A.cache + i * A.cache_width, A.cache_width, lane, instance_salt(k));
    wave_sync();
}

/// The count of a batch of one instance (A.instance) in batch order (rows whose task id is not 0 set kStatusTaskId and
/// are not counted); with kGroup, the rows of instance A.instance's group.
template<bool kStaged, bool kLevels, bool kGroup>
__global__ __launch_bounds__(kMaxWaves * kWave) void k_env_count(CountArgs A)
{
    extern __shared__ u64 smem[];
    const TaskDev& T = A.T;
    const u32 lane = lane_id(), wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    if constexpr (kGroup)
    {
        const u32 lo = A.groups.starts[A.instance], hi = A.groups.starts[A.instance + 1];
        if (lo + static_cast<u64>(blockIdx.x) * nw >= hi)
            return;
        Tab<kStaged> H;
        lds<u64>* waves = stage_hot<kStaged>(smem, T, &H);
        const Lds L = lds_of<kLevels>(waves + static_cast<u64>(wave) * wave_lds_words(T, kLevels), T);
        for (u64 j = lo + static_cast<u64>(blockIdx.x) * nw + wave; j < hi; j += static_cast<u64>(gridDim.x) * nw)
            count_row<kLevels>(A, T, H, L, A.groups.order[j], A.instance, lane);
    }
    else
    {
        Tab<kStaged> H;
        lds<u64>* waves = stage_hot<kStaged>(smem, T, &H);
        const Lds L = lds_of<kLevels>(waves + static_cast<u64>(wave) * wave_lds_words(T, kLevels), T);
        for (u64 i = static_cast<u64>(blockIdx.x) * nw + wave; i < A.rows; i += static_cast<u64>(gridDim.x) * nw)
        {
            if (A.task_ids && A.task_ids[i] != 0)
            {
                if (lane == 0 && A.status)
                    atomicOr(A.status, kStatusTaskId);
                continue;
            }
            count_row<kLevels>(A, T, H, L, i, A.instance, lane);
        }
    }
}

/// The count of the rows of the instances of variant `variant` of a batch grouped by instance (as k_env_step_grouped).
template<bool kStaged, bool kLevels>
__global__ __launch_bounds__(kMaxWaves * kWave) void k_env_count_grouped(CountArgs A, u32 variant)
{
    extern __shared__ u64 smem[];
    const u32 lane = lane_id(), wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    const u32 chunks = A.groups.chunk_start[A.instances];
    for (u32 c = blockIdx.x; c < chunks; c += gridDim.x)
    {
        const u32 k = chunk_instance(A.groups.chunk_start, A.instances, c);
        if (A.inst[k].variant != variant)
            continue;
        const TaskDev& T = instance_tables(A.tasks, k);
        __syncthreads();
        Tab<kStaged> H;
        lds<u64>* waves = stage_hot<kStaged>(smem, T, &H);
        const Lds L = lds_of<kLevels>(waves + static_cast<u64>(wave) * A.wave_words, T);
        const u32 r0 = A.groups.starts[k] + (c - A.groups.chunk_start[k]) * kChunkRows;
        const u32 r1 = min(r0 + kChunkRows, A.groups.starts[k + 1]);
        for (u32 j = r0 + wave; j < r1; j += nw)
            count_row<kLevels>(A, T, H, L, A.groups.order[j], k, lane);
    }
}

/// The instance a reset puts row i in: task_ids[i] (null: 0); an id outside the table resets into instance 0.
__device__ __forceinline__ u32 reset_instance(const i32* task_ids, u64 i, u32 instances, bool* bad)
{
    const i32 v = task_ids ? task_ids[i] : 0;
    *bad = v < 0 || static_cast<u32>(v) >= instances;
    return *bad ? 0u : static_cast<u32>(v);
}

/// One thread per state word of the batch (reset_row with a dirtied row: zeros up to the batch's words).
__global__ void k_env_reset(const InstDev* inst, u32 instances, u64* states, u64 rows, u32 words, const u8* mask, i32* task_ids,
                            i32* steps, u8* at_goal, i32* count, u32* status)
{
    const u64 total = rows * words;
    for (u64 e = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; e < total; e += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        const u64 i = e / words;
        const u32 w = static_cast<u32>(e - i * words);
        if (mask && !mask[i])
            continue;
        // the word-0 thread writes a corrected id (0) while the row's other threads may read it: either value they
        // see resets the row into instance 0
        bool bad = false;
        const u32 k = reset_instance(task_ids, i, instances, &bad);
        const InstDev& J = inst[k];
        states[e] = w < J.W ? J.initial[w] : 0;
        if (w == 0)
        {
            if (bad)
            {
                atomicOr(status, kStatusTaskId);
                task_ids[i] = 0;
            }
            if (steps)
                steps[i] = 0;
            if (at_goal)
                at_goal[i] = J.init_goal ? 1 : 0;
            if (count)
                count[i] = static_cast<i32>(J.init_count);
        }
    }
}

/// One wave per row: the masked rows' visited tables restarted with the initial state's key of the row's instance, or
/// (current) the key of the row's state.
__global__ __launch_bounds__(256) void k_visited_restart(VisitedDev v, const InstDev* inst, u32 instances, const u64* states, u64 rows,
                                                         u32 words, const u8* mask, const i32* task_ids, u32 current)
{
    const u32 lane = lane_id(), nw = blockDim.x / kWave;
    for (u64 i = static_cast<u64>(blockIdx.x) * nw + threadIdx.x / kWave; i < rows; i += static_cast<u64>(gridDim.x) * nw)
    {
        if (mask && !mask[i])
            continue;
        bool bad = false;
        const InstDev& J = inst[reset_instance(task_ids, i, instances, &bad)];
        u64 h = J.init_hash;
        if (current)
        {
            u64 mine = 0;
            if (lane == 0)
                mine = row_hash(states + i * words, J.W);
            h = __shfl(mine, 0, kWave);
        }
        visited_restart(v.table + i * v.capacity, v.capacity, v.count + i, h, lane);
    }
}

/// Per row before a reset: the drawn task id (sample) and the advanced reset counter.
__global__ void k_env_reset_draw(SamplerDev sampler, const u64* seed, u64 first_env, u64 rows, const u8* mask, u32 sample, i32* task_ids,
                                 u32* reset_counts, const u64* sampling_seeds, const u32* env_ids)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows; i += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        if (mask && !mask[i])
            continue;
        if (!reset_counts)
            continue;
        const u32 rc = reset_counts[i];
        if (sample && task_ids)
            task_ids[i] = instance_draw(sampling_seeds ? sampling_seeds[i] : *seed, env_ids ? static_cast<u64>(env_ids[i]) : first_env + i, rc,
                                        sampler.instances, sampler.thresholds, sampler.indices, sampler.m);
        reset_counts[i] = rc + 1;
    }
}

/// The random policy's next choices without a step (DeviceEnv::random_actions, include/mymyr/cuda/env.hpp:189-192):
/// out[i] = successor_index(key, env id, draws[i], min(count[i], max_actions)), 0 where that is 0.
__global__ void k_env_random_actions(const u64* seed, const u64* seeds, const u32* env_ids, u64 first_env, const u64* draws, const i32* count,
                                     u64 rows, u32 max_actions, i64* out)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows; i += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        const u32 c = min(static_cast<u32>(max(count[i], 0)), max_actions);
        out[i] = c ? static_cast<i64>(successor_index(seeds ? seeds[i] : *seed, env_ids ? static_cast<u64>(env_ids[i]) : first_env + i, draws[i], c))
                   : 0;
    }
}

/// kStatusTaskId if some ids[i] is outside [0, instances).
__global__ void k_check_ids(const i32* ids, u64 rows, u32 instances, u32* status)
{
    bool bad = false;
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows; i += static_cast<u64>(gridDim.x) * blockDim.x)
        bad = bad || ids[i] < 0 || static_cast<u32>(ids[i]) >= instances;
    if (bad)
        atomicOr(status, kStatusTaskId);
}

/// The device seed word of an env, written in stream order.
__global__ void k_set_word(u64* p, u64 v) { *p = v; }

/// Per row: the instance its next autoreset would draw (with the row's current reset counter), for a step without
/// next_task_ids over a batch with reset counters and an env with a sampler.
__global__ void k_env_sample_next(SamplerDev sampler, const u64* seed, u64 first_env, u64 rows, const u32* reset_counts, const u64* sampling_seeds,
                                  const u32* env_ids, i32* next)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows; i += static_cast<u64>(gridDim.x) * blockDim.x)
        next[i] = instance_draw(sampling_seeds ? sampling_seeds[i] : *seed, env_ids ? static_cast<u64>(env_ids[i]) : first_env + i,
                                reset_counts[i], sampler.instances, sampler.thresholds, sampler.indices, sampler.m);
}

/// Per row: the instance's goal into the row's goal masks, or (keep) the given masks checked against the instance's
/// fluent slots and tested on its initial state. Runs after k_env_reset, so task ids are valid.
__global__ void k_env_reset_goals(const InstDev* inst, u32 instances, u64 rows, u32 words, const u8* mask, const i32* task_ids,
                                  u64* goal_pos, u64* goal_neg, u32 keep, u8* at_goal, u32* status)
{
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows; i += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        if (mask && !mask[i])
            continue;
        bool bad = false;
        const InstDev& J = inst[reset_instance(task_ids, i, instances, &bad)];
        u64* gp = goal_pos + i * words;
        u64* gn = goal_neg + i * words;
        if (!keep)
        {
            for (u32 w = 0; w < words; ++w)
            {
                gp[w] = w < J.W ? J.goal_pos[w] : 0;
                gn[w] = w < J.W ? J.goal_neg[w] : 0;
            }
            continue;
        }
        bool ok = true, fit = true;
        for (u32 w = 0; w < words; ++w)
        {
            const u64 p = gp[w], n = gn[w], x = w < J.W ? J.initial[w] : 0;
            ok = ok && (x & p) == p && (x & n) == 0;
            if (w >= J.W)
                fit = fit && (p | n) == 0;
            else if (w == J.W - 1 && (J.fluent_slots & 63))
                fit = fit && ((p | n) >> (J.fluent_slots & 63)) == 0;
        }
        if (!fit)
            atomicOr(status, kStatusGoalMask);
        if (at_goal)
            at_goal[i] = ok ? 1 : 0;
    }
}

/// One thread per count-cache word: the initial state's row of the row's instance. Runs after k_env_reset.
__global__ void k_env_reset_cache(const InstDev* inst, u32 instances, u64 rows, u32 width, const u8* mask, const i32* task_ids, u32* cache)
{
    const u64 total = rows * width;
    for (u64 e = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; e < total; e += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        const u64 i = e / width;
        if (mask && !mask[i])
            continue;
        bool bad = false;
        cache[e] = inst[reset_instance(task_ids, i, instances, &bad)].init_cache[e - i * width];
    }
}

// ------------------------------------------------------------------------------------------ grouping by instance
constexpr u32 kGroupBlock = 1024;
constexpr u32 kGroupRowsPerThread = 4;
constexpr u32 kLdsInstances = 4096;  // instances whose block-local counters fit LDS

/// hist[k] += rows with task id k (block-local counters in LDS when the table is small); ids outside the table set
/// kStatusTaskId.
__global__ __launch_bounds__(kGroupBlock) void k_group_count(const i32* task_ids, u64 rows, u32 instances, u32* hist, u32* status)
{
    __shared__ u32 sh[kLdsInstances];
    const bool local = instances <= kLdsInstances;
    if (local)
    {
        for (u32 k = threadIdx.x; k < instances; k += blockDim.x)
            sh[k] = 0;
        __syncthreads();
    }
    const u64 base = static_cast<u64>(blockIdx.x) * blockDim.x * kGroupRowsPerThread;
    bool bad = false;
    for (u32 r = 0; r < kGroupRowsPerThread; ++r)
    {
        const u64 i = base + static_cast<u64>(r) * blockDim.x + threadIdx.x;
        if (i >= rows)
            break;
        const i32 v = task_ids[i];
        if (v < 0 || static_cast<u32>(v) >= instances)
        {
            bad = true;
            continue;
        }
        if (local)
            atomicAdd(&sh[v], 1u);
        else
            atomicAdd(&hist[v], 1u);
    }
    if (bad)
        atomicOr(status, kStatusTaskId);
    if (local)
    {
        __syncthreads();
        for (u32 k = threadIdx.x; k < instances; k += blockDim.x)
            if (sh[k])
                atomicAdd(&hist[k], sh[k]);
    }
}

/// One block: starts = exclusive scan of hist, chunk_start = exclusive scan of ceil(hist / kChunkRows) (both
/// [instances + 1]); hist becomes each group's write cursor (its start).
__global__ __launch_bounds__(kGroupBlock) void k_group_scan(u32* hist, u32 instances, u32* starts, u32* chunk_start)
{
    __shared__ u32 sr[kGroupBlock], sc[kGroupBlock];
    const u32 per = (instances + kGroupBlock - 1) / kGroupBlock;
    const u32 lo = min(instances, threadIdx.x * per), hi = min(instances, lo + per);
    u32 r = 0, c = 0;
    for (u32 k = lo; k < hi; ++k)
    {
        r += hist[k];
        c += (hist[k] + kChunkRows - 1) / kChunkRows;
    }
    sr[threadIdx.x] = r;
    sc[threadIdx.x] = c;
    __syncthreads();
    // inclusive Hillis-Steele scan of the per-thread sums
    for (u32 d = 1; d < kGroupBlock; d <<= 1)
    {
        const u32 ar = threadIdx.x >= d ? sr[threadIdx.x - d] : 0;
        const u32 ac = threadIdx.x >= d ? sc[threadIdx.x - d] : 0;
        __syncthreads();
        sr[threadIdx.x] += ar;
        sc[threadIdx.x] += ac;
        __syncthreads();
    }
    r = sr[threadIdx.x] - r;
    c = sc[threadIdx.x] - c;
    for (u32 k = lo; k < hi; ++k)
    {
        const u32 h = hist[k];
        starts[k] = r;
        chunk_start[k] = c;
        hist[k] = r;
        r += h;
        c += (h + kChunkRows - 1) / kChunkRows;
    }
    if (threadIdx.x == kGroupBlock - 1)
    {
        starts[instances] = sr[kGroupBlock - 1];
        chunk_start[instances] = sc[kGroupBlock - 1];
    }
}

/// order[cursor[k]++] = i for each row i of instance k (block-local ranks in LDS, one global reservation per block and
/// instance, when the table is small). Rows in a group come in no particular order; each row's results do not depend
/// on it.
__global__ __launch_bounds__(kGroupBlock) void k_group_scatter(const i32* task_ids, u64 rows, u32 instances, u32* cursor, u32* order)
{
    __shared__ u32 sh[kLdsInstances];
    const bool local = instances <= kLdsInstances;
    if (local)
    {
        for (u32 k = threadIdx.x; k < instances; k += blockDim.x)
            sh[k] = 0;
        __syncthreads();
    }
    const u64 base = static_cast<u64>(blockIdx.x) * blockDim.x * kGroupRowsPerThread;
    u32 pos[kGroupRowsPerThread];
    i32 ids[kGroupRowsPerThread];
    for (u32 r = 0; r < kGroupRowsPerThread; ++r)
    {
        const u64 i = base + static_cast<u64>(r) * blockDim.x + threadIdx.x;
        ids[r] = -1;
        if (i >= rows)
            continue;
        const i32 v = task_ids[i];
        if (v < 0 || static_cast<u32>(v) >= instances)
            continue;
        ids[r] = v;
        pos[r] = local ? atomicAdd(&sh[v], 1u) : atomicAdd(&cursor[v], 1u);
    }
    if (local)
    {
        __syncthreads();
        for (u32 k = threadIdx.x; k < instances; k += blockDim.x)
        {
            const u32 n = sh[k];
            if (n)
                sh[k] = atomicAdd(&cursor[k], n);
        }
        __syncthreads();
    }
    for (u32 r = 0; r < kGroupRowsPerThread; ++r)
        if (ids[r] >= 0)
            order[(local ? sh[ids[r]] : 0u) + pos[r]] = static_cast<u32>(base + static_cast<u64>(r) * blockDim.x + threadIdx.x);
}

/// Applies the effects of the picked binding of schema s to the LDS row only (the view stays the parent's), keeping
/// the effect slots and their prior bits for succ_revert. Returns whether no bit changed (a no-op successor). One effect
/// per lane (lane k: slot L.eff[k], prior bit L.before[k]); deletes, then adds.
__device__ __forceinline__ bool succ_apply(const TaskDev& T, const auto& H, const Lds& L, u32 s, u32 lane, u32* status)
{
    const auto& S = H.schemas[s];
    const u32 ne = min(S.eff_end - S.eff_begin, kMaxEff);
    if (lane == 0 && S.eff_end - S.eff_begin > kMaxEff)
        atomicOr(status, kStatusCapacity);
    const bool mine = lane < ne;
    const bool add = lane < S.nadd;
    u32 sl = kNone;
    bool before = false;
    if (mine)
    {
        u64 cid;
        sl = effect_slot(T, L, H.effects[S.eff_begin + lane], &cid);
        before = sl != kNone && row_bit(L.row, sl);
        L.eff[lane] = sl;
        L.before[lane] = before ? 1u : 0u;
        if (add && sl == kNone)
            missing_atom(T, cid, status);
    }
    wave_sync();
    if (mine && !add && sl != kNone)
        __hip_atomic_fetch_and(L.row + (sl >> 6), ~(u64{1} << (sl & 63)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
    wave_sync();
    if (mine && add && sl != kNone)
        __hip_atomic_fetch_or(L.row + (sl >> 6), u64{1} << (sl & 63), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
    wave_sync();
    const bool changed = mine && sl != kNone && row_bit(L.row, sl) != before;
    return __ballot(changed) == 0;
}

/// Restores the parent row after succ_apply (lanes listing one slot hold the same prior bit).
__device__ __forceinline__ void succ_revert(const auto& H, const Lds& L, u32 s, u32 lane)
{
    const auto& S = H.schemas[s];
    const u32 ne = min(S.eff_end - S.eff_begin, kMaxEff);
    if (lane < ne)
    {
        const u32 sl = L.eff[lane];
        if (sl != kNone)
        {
            if (L.before[lane])
                __hip_atomic_fetch_or(L.row + (sl >> 6), u64{1} << (sl & 63), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
            else
                __hip_atomic_fetch_and(L.row + (sl >> 6), ~(u64{1} << (sl & 63)), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WAVEFRONT);
        }
    }
    wave_sync();
}

/// 1 + the index of the highest nonzero word of the LDS row (0 for an empty row), on every lane.
__device__ __forceinline__ u32 trimmed_words(const lds<u64>* row, u32 W, u32 lane)
{
    u32 top = 0;
    for (u32 w = lane; w < W; w += kWave)
        if (row[w])
            top = w + 1;
#pragma unroll
    for (int d = kWave / 2; d > 0; d >>= 1)
        top = max(top, static_cast<u32>(__shfl_xor(static_cast<int>(top), d, kWave)));
    return top;
}

/// Witness pruning (include/mymyr/successor/successors.hpp:154-248 with witness pruning on): the successor counts of
/// the schemas with witness parameters become the number of full bindings whose witnesses the matcher binds first (one
/// per effect-relevant binding), counted by enumerating those schemas; `total` (count_all's) is corrected to match.
template<bool kLevels>
__device__ __forceinline__ u32 witness_counts(const TaskDev& T, const auto& H, const Lds& L, u32 lane, u32 total)
{
    if (!T.witness)
        return total;
    for (u32 s = 0; s < T.num_schemas; ++s)
    {
        const u32 all = L.counts[s];
        if (T.witness[s].n == 0 || all == 0)
            continue;
        const u32 kept = for_each_successor<kLevels, true>(T, H, L, lane, [](u32, u32) { return true; }, s, s + 1);
        wave_sync();
        if (lane == 0)
            L.counts[s] = kept;
        wave_sync();
        total = total - all + kept;
    }
    return total;
}

/// The expansion of row i (pass 0: its counts and the validation of its words; pass 1: its successors from
/// offsets[i] on) with the tables of its instance.
template<bool kLevels, bool kWitness>
__device__ __forceinline__ void expand_row(const ExpandArgs& A, const TaskDev& T, const auto& H, const Lds& L, u64 i, u32 lane)
{
    const u32 Lw = A.label_width;
    const u64* src = A.states + i * A.words;
    if (A.pass == 0)
    {
        // rows must hold no atoms past the task's slots (ExpandOptions::validate)
        bool wide = false;
        for (u32 w = lane; w < A.words; w += kWave)
        {
            const u64 x = src[w];
            if (w >= T.W)
                wide = wide || x != 0;
            else if (w == T.W - 1 && (T.fluent_slots & 63))
                wide = wide || (x >> (T.fluent_slots & 63)) != 0;
        }
        if (__ballot(wide) && lane == 0)
            atomicOr(A.status, kStatusWideRow);
    }
    load_row_lds_n(T, L, src, min(A.words, T.W), lane);
    build_view<kLevels>(T, H, L, lane);
    u32 c = count_all<kLevels>(T, H, L, lane);
    if constexpr (kWitness)
        c = witness_counts<kLevels>(T, H, L, lane, c);
    if (A.pass == 0 && !A.drop_noops)
    {
        if (lane == 0)
            A.counts[i] = c;
        return;
    }
    const bool keep_all = A.pass == 1 && A.drop_noops && A.noops[i] == c;
    u32 noops = 0, kept = 0;
    const u32 listed = for_each_successor<kLevels, kWitness>(T, H, L, lane, [&](u32 k, u32 s) {
        const bool noop = succ_apply(T, H, L, s, lane, A.status);
        noops += noop ? 1 : 0;
        if (A.pass == 1 && (!A.drop_noops || !noop || keep_all))
        {
            const u64 pos = A.offsets[i] - A.offset_base + (A.drop_noops ? kept : k);
            ++kept;
            const u32 n = (A.succ || A.succ_hash) ? trimmed_words(L.row, T.W, lane) : 0;
            const bool fits = n <= A.out_words;
            if (A.succ && !fits && lane == 0)
                atomicMax(A.words_needed, n);
            if (pos < A.capacity)
            {
                if (A.succ)
                {
                    u64* dst = A.succ + pos * A.out_words;
                    for (u32 w = lane; w < A.out_words; w += kWave)
                        dst[w] = (fits && w < T.W) ? L.row[w] : 0;
                }
                if (A.goal)
                {
                    const bool g = A.any_goal.any
                                       ? any_of_holds_dev(A.any_goal, [&](u32 s) { return s < 64 * T.W && row_bit(L.row, s); })
                                       : goal_test(T, H, L.row, lane);
                    if (lane == 0)
                        A.goal[pos] = g ? 1 : 0;
                }
                if (lane == 0)
                {
                    if (A.succ_hash)
                    {
                        // hash_state over the trimmed words: the pairs chained in order
                        u64 h = kHashSeed ^ (static_cast<u64>(n) * kHashP1);
                        for (u32 w = 0; w < n; w += 2)
                            h = mulfold(h ^ L.row[w] ^ kHashP1, (w + 1 < n ? L.row[w + 1] : 0) ^ kHashP2);
                        A.succ_hash[pos] = mix64(h);
                    }
                    if (A.noop)
                        A.noop[pos] = noop ? 1 : 0;
                    if (A.index)
                        A.index[pos] = static_cast<i32>(k);
                    if (A.parent)
                        A.parent[pos] = static_cast<i32>(i);
                    if (A.schema)
                        A.schema[pos] = static_cast<i32>(s);
                }
                if (A.binding)
                {
                    const u32 arity = H.schemas[s].arity;
                    for (u32 q = lane; q < Lw; q += kWave)
                        A.binding[pos * Lw + q] = q < arity ? static_cast<i32>(L.ub[q]) : -1;
                }
            }
        }
        succ_revert(H, L, s, lane);
        return true;
    });
    if (listed != c && lane == 0)
        atomicOr(A.status, kStatusPickFailed);
    if (A.pass == 0 && lane == 0)
    {
        A.counts[i] = c;
        A.noops[i] = noops;
    }
    wave_sync();
}

/// The expansion of a batch of one instance in batch order, or with kGroup of one instance's group of a batch grouped
/// by instance.
template<bool kStaged, bool kLevels, bool kGroup, bool kWitness = false>
__global__ __launch_bounds__(kMaxWaves * kWave) void k_expand(ExpandArgs A)
{
    extern __shared__ u64 smem[];
    const TaskDev& T = A.T;
    const u32 lane = lane_id(), wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    u64 lo = 0, hi = A.rows;
    if constexpr (kGroup)
    {
        lo = A.groups.starts[A.instance];
        hi = A.groups.starts[A.instance + 1];
        if (lo + static_cast<u64>(blockIdx.x) * nw >= hi)
            return;
    }
    Tab<kStaged> H;
    lds<u64>* waves = stage_hot<kStaged>(smem, T, &H);
    const Lds L = lds_of<kLevels>(waves + static_cast<u64>(wave) * wave_lds_words(T, kLevels), T);
    for (u64 j = lo + static_cast<u64>(blockIdx.x) * nw + wave; j < hi; j += static_cast<u64>(gridDim.x) * nw)
        expand_row<kLevels, kWitness>(A, T, H, L, kGroup ? A.groups.order[j] : j, lane);
}

__global__ void k_offsets_i32(const u64* src, u64 n, i32* dst)
{
    const u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < n)
        dst[i] = static_cast<i32>(src[i]);
}

__global__ void k_kept_counts(const u32* counts, const u32* noops, u64 rows, u32* kept)
{
    const u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i < rows)
        kept[i] = noops[i] == counts[i] ? counts[i] : counts[i] - noops[i];
}

// Padded view of a flat expansion, one wave per row: the row's k slots are contiguous in every output, so the lanes
// walk each output row (scalars over the k slots, succ over k * words, binding over k * label_width) with coalesced
// stores, reading the flat rows b .. b + k - 1 that are also contiguous.
__global__ __launch_bounds__(256) void k_pad(PadArgs a)
{
    const u32 lane = lane_id();
    const u64 nw = u64{gridDim.x} * (blockDim.x / kWave);
    const u32 K = a.k;
    for (u64 i = static_cast<u64>(blockIdx.x) * (blockDim.x / kWave) + threadIdx.x / kWave; i < a.rows; i += nw)
    {
        const u64 b = static_cast<u64>(static_cast<i64>(a.offsets[i]));
        const u64 c = static_cast<u64>(static_cast<i64>(a.offsets[i + 1])) - b;
        // valid slots: k < min(c, K) with b + k < capacity
        const u64 room = b < a.capacity ? a.capacity - b : 0;
        const u32 n = static_cast<u32>(std::min<u64>(std::min<u64>(c, K), room));
        if (lane == 0)
        {
            if (a.count)
                a.count[i] = static_cast<i32>(c);
            if (c > K || n < std::min<u64>(c, K))
                atomicOr(a.overflow, 1u);
        }
        const u64 base = i * K;
        for (u32 k = lane; k < K; k += kWave)
        {
            const bool valid = k < n;
            const u64 j = b + k, at = base + k;
            if (a.out_index)
                a.out_index[at] = valid ? static_cast<i32>(j) : -1;
            if (a.mask)
                a.mask[at] = valid ? 1 : 0;
            if (a.canonical)
                a.canonical[at] = valid && a.index ? a.index[j] : -1;
            if (a.out_schema)
                a.out_schema[at] = valid && a.schema ? a.schema[j] : -1;
            if (a.out_goal)
                a.out_goal[at] = valid && a.goal ? a.goal[j] : 0;
            if (a.out_succ_hash)
                a.out_succ_hash[at] = valid && a.succ_hash ? a.succ_hash[j] : 0;
            if (a.out_noop)
                a.out_noop[at] = valid && a.noop ? a.noop[j] : 0;
        }
        if (a.out_succ)
        {
            const u32 W = a.words, FW = a.succ ? a.flat_words : 0;
            u64* dst = a.out_succ + base * W;
            const u64 total = u64{K} * W;
            for (u64 t = lane; t < total; t += kWave)
            {
                const u32 k = static_cast<u32>(t / W), w = static_cast<u32>(t - u64{k} * W);
                dst[t] = k < n && w < FW ? a.succ[(b + k) * FW + w] : 0;
            }
        }
        if (a.out_binding)
        {
            const u32 L = a.label_width, FL = a.binding ? a.flat_label_width : 0;
            i32* dst = a.out_binding + base * L;
            const u64 total = u64{K} * L;
            for (u64 t = lane; t < total; t += kWave)
            {
                const u32 k = static_cast<u32>(t / L), w = static_cast<u32>(t - u64{k} * L);
                dst[t] = k < n && w < FL ? a.binding[(b + k) * FL + w] : -1;
            }
        }
    }
}

// The position of each row's label in its flat expansion (canonical order): one lane per row scans the row's successors
// for the label's schema and the objects of its binding (the flat binding's -1 columns lie past the arity and match
// anything); -1 when no successor carries the label.
__global__ __launch_bounds__(256) void k_label_actions(const i32* offsets, const i32* schema, const i32* binding, u32 L, u64 rows,
                                                       const i32* label_schema, const i32* label_binding, u32 stride, i64* actions)
{
    const u64 step = u64{gridDim.x} * blockDim.x;
    for (u64 i = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; i < rows; i += step)
    {
        const i64 b = offsets[i], e = offsets[i + 1];
        const i32 ls = label_schema[i];
        const i32* lb = label_binding + i * stride;
        i64 act = -1;
        for (i64 j = b; j < e && act < 0; ++j)
        {
            if (schema[j] != ls)
                continue;
            const i32* fb = binding + static_cast<u64>(j) * L;
            bool same = true;
            for (u32 k = 0; k < L && same; ++k)
                same = fb[k] < 0 || fb[k] == lb[k];
            if (same)
                act = j - b;
        }
        actions[i] = act;
    }
}

// Successor listing: successor k of row i is pick(k) applied to a copy of the row.
template<bool kStaged, bool kLevels>
__global__ __launch_bounds__(kMaxWaves * kWave) void k_successors(TaskDev T, const u64* states, u64 rows, u32 words, u32 cap, i32* count,
                                                                  i32* schema, i32* binding, u64* succ, u32* status)
{
    extern __shared__ u64 smem[];
    Tab<kStaged> H;
    lds<u64>* waves = stage_hot<kStaged>(smem, T, &H);
    const u32 lane = lane_id(), wave = threadIdx.x / kWave, nw = blockDim.x / kWave;
    const Lds L = lds_of<kLevels>(waves + static_cast<u64>(wave) * wave_lds_words(T, kLevels), T);
    const u32 Lw = T.label_width;
    for (u64 i = static_cast<u64>(blockIdx.x) * nw + wave; i < rows; i += static_cast<u64>(gridDim.x) * nw)
    {
        load_row_lds_n(T, L, states + i * words, min(words, T.W), lane);
        build_view<kLevels>(T, H, L, lane);
        const u32 c = count_all<kLevels>(T, H, L, lane);
        if (lane == 0 && count)
            count[i] = static_cast<i32>(c);
        const u32 listed = cap == 0 ? 0 : for_each_successor<kLevels>(T, H, L, lane, [&](u32 k, u32 s) {
            const u64 o = i * cap + k;
            if (lane == 0 && schema)
                schema[o] = static_cast<i32>(s);
            const auto& S = H.schemas[s];
            if (binding)
                for (u32 q = lane; q < Lw; q += kWave)
                    binding[o * Lw + q] = q < S.arity ? static_cast<i32>(L.ub[q]) : -1;
            if (succ)
            {
                // the successor on the LDS row (one effect per lane), copied out, then the row restored
                succ_apply(T, H, L, s, lane, status);
                u64* dst = succ + o * words;
                for (u32 q = lane; q < words; q += kWave)
                    dst[q] = q < T.W ? L.row[q] : 0;
                // a successor with atoms past the rows' words (a lazy task's rows outgrew them) is an error
                bool wide = false;
                for (u32 q = words + lane; q < T.W; q += kWave)
                    wide = wide || L.row[q] != 0;
                if (__ballot(wide) && lane == 0)
                    atomicOr(status, kStatusWideRow);
                succ_revert(H, L, s, lane);
            }
            wave_sync();
            return k + 1 < cap;
        });
        if (listed != min(c, cap) && lane == 0)
            atomicOr(status, kStatusPickFailed);
        wave_sync();
    }
}

unsigned grid_for(u64 rows, unsigned nw) { return static_cast<unsigned>(std::min<u64>((rows + nw - 1) / nw, u64{1} << 20)); }

/// Raises a kernel's dynamic LDS limit once per (kernel, size): later launches make no runtime call besides the launch,
/// so a step recorded into a HIP graph after a first eager call holds kernel nodes only.
void set_lds(const void* fn, size_t bytes)
{
    if (bytes <= 64 * 1024)
        return;
    static std::mutex mu;
    static std::unordered_map<const void*, size_t> done;
    std::lock_guard lock(mu);
    size_t& have = done[fn];
    if (bytes <= have)
        return;
    hip_check(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)), "LDS size");
    have = bytes;
}
}  // namespace

/// Blocks of a one-instance launch: a row per wave in batch order; over one group of a grouped batch (whose size only the
/// device knows) a bounded grid whose blocks stride over the group.
/// Compute units of the current device (queried once per device).
unsigned device_cus()
{
    static std::mutex mu;
    static std::unordered_map<int, unsigned> cus;
    int dev = 0;
    hip_check(hipGetDevice(&dev), "device");
    std::lock_guard lock(mu);
    unsigned& n = cus[dev];
    if (n == 0)
    {
        int v = 0;
        hip_check(hipDeviceGetAttribute(&v, hipDeviceAttributeMultiprocessorCount, dev), "compute units");
        n = static_cast<unsigned>(std::max(1, v));
    }
    return n;
}

/// The grid of a one-instance launch. `resident`: `over` times the blocks that are resident at once (LDS bytes `lds` and
/// nw waves per block), each looping over rows, so that a block stages the hot tables once for many rows (env steps and
/// counts); else one block per nw rows. A grouped launch keeps its cap.
unsigned one_instance_grid(u64 rows, unsigned nw, bool group, size_t lds, bool resident = true, unsigned over = 1)
{
    constexpr u64 kGroupBlocks = 8192;
    constexpr size_t kCuLds = 160 * 1024;
    constexpr unsigned kCuWaves = 24;
    const unsigned g = grid_for(rows, nw);
    if (group)
        return static_cast<unsigned>(std::min<u64>(g, kGroupBlocks));
    if (!resident)
        return g;
    const unsigned per_cu = std::max<unsigned>(1, std::min<unsigned>(lds ? static_cast<unsigned>(kCuLds / lds) : kCuWaves, kCuWaves / nw));
    return std::min<unsigned>(g, per_cu * device_cus() * over);
}

void launch_env_step(const EnvArgs& a, hipStream_t stream)
{
    if (a.rows == 0)
        return;
    size_t lds = 0;
    const unsigned nw = waves_per_block(a.T, &lds);
    const bool group = a.groups.order != nullptr;
    // the visited tables' code only in the launches that use it (it keeps more kernel arguments live); the plain step
    // (an env pool's random-policy step over one instance) compiles the optional inputs it does not take away
    const bool visited = a.visited.capacity || a.revisited;
    const bool plain = !group && !visited && !a.actions && !a.label_schema && !a.seeds && !a.env_ids && !a.goal_pos && !a.final_states &&
                       !a.reset_counts && !a.next_task_ids && a.steps && a.draws;
    const auto fn = group     ? variant(a.T, k_env_step<true, false, true, true>, k_env_step<true, true, true, true>,
                                        k_env_step<false, false, true, true>, k_env_step<false, true, true, true>)
                    : visited ? variant(a.T, k_env_step<true, false, false, true>, k_env_step<true, true, false, true>,
                                        k_env_step<false, false, false, true>, k_env_step<false, true, false, true>)
                    : plain   ? variant(a.T, k_env_step<true, false, false, false, true>, k_env_step<true, true, false, false, true>,
                                        k_env_step<false, false, false, false, true>, k_env_step<false, true, false, false, true>)
                              : variant(a.T, k_env_step<true, false, false, false>, k_env_step<true, true, false, false>,
                                        k_env_step<false, false, false, false>, k_env_step<false, true, false, false>);
    set_lds(reinterpret_cast<const void*>(fn), lds);
    // several resident grids' worth of blocks: a block whose rows take longer no longer holds the launch's end, the
    // dispatcher hands its CU the next block (transport_xl, 262,144 envs: 24.2 ms per step on one resident grid, 15.7 ms
    // on 16; transport's lane-split step is best at 4)
    hipLaunchKernelGGL(fn, dim3(one_instance_grid(a.rows, nw, group, lds, true, levels(a.T) ? 16 : 4)), dim3(nw * kWave), lds, stream, a);
    launch_check("env step");
}

void launch_env_count(const CountArgs& a, hipStream_t stream)
{
    if (a.rows == 0)
        return;
    size_t lds = 0;
    const unsigned nw = waves_per_block(a.T, &lds);
    const bool group = a.groups.order != nullptr;
    const auto fn = group ? variant(a.T, k_env_count<true, false, true>, k_env_count<true, true, true>, k_env_count<false, false, true>,
                                    k_env_count<false, true, true>)
                          : variant(a.T, k_env_count<true, false, false>, k_env_count<true, true, false>, k_env_count<false, false, false>,
                                    k_env_count<false, true, false>);
    set_lds(reinterpret_cast<const void*>(fn), lds);
    hipLaunchKernelGGL(fn, dim3(one_instance_grid(a.rows, nw, group, lds)), dim3(nw * kWave), lds, stream, a);
    launch_check("env count");
}

void launch_env_count(const TaskDev& T, const u64* states, u64 rows, u32 words, i32* count, u8* goal, u8* masks, u32* cache,
                      hipStream_t stream, const u64* goal_pos, const u64* goal_neg, u32* status, u32 instance, u32 schemas)
{
    CountArgs a{};
    a.T = T;
    a.mask_width = schemas ? schemas : T.num_schemas;
    a.cache_width = a.mask_width + 2;
    a.instances = 1;
    a.states = states;
    a.rows = rows;
    a.words = words;
    a.count = count;
    a.goal = goal;
    a.masks = masks;
    a.cache = cache;
    a.goal_pos = goal_pos;
    a.goal_neg = goal_neg;
    a.status = status;
    a.instance = instance;
    launch_env_count(a, stream);
}

u32 env_variant(const TaskDev& T)
{
    check_schemas(T);
    return (staged(T) ? 1u : 0u) | (levels(T) ? 2u : 0u);
}

unsigned grouped_shape(const TaskDev* const* tasks, u32 n, size_t* lds_bytes, u32* wave_words)
{
    size_t hot = 0;
    u32 wave = 0;
    for (u32 k = 0; k < n; ++k)
    {
        const TaskDev& T = *tasks[k];
        check_schemas(T);
        if (staged(T))
            hot = std::max(hot, static_cast<size_t>(T.hot_words) * 8);
        wave = std::max(wave, wave_lds_words(T, levels(T)));
    }
    *wave_words = wave;
    return block_shape(hot, static_cast<size_t>(wave) * 8, lds_bytes);
}

namespace
{
/// Blocks of a grouped launch: at most one chunk per block (chunks number at most rows / kChunkRows + instances).
unsigned grouped_grid(u64 rows, u32 instances)
{
    return static_cast<unsigned>(std::min<u64>((rows + kChunkRows - 1) / kChunkRows + instances, u64{1} << 20));
}

template<class F>
F variant_of(u32 v, F gs, F ss, F gl, F sl)
{
    return v == 0 ? gs : v == 1 ? ss : v == 2 ? gl : sl;
}
}  // namespace

void prepare_env_launches(const TaskDev& T)
{
    size_t lds = 0;
    waves_per_block(T, &lds);
    for (const void* fn : {reinterpret_cast<const void*>(variant(T, k_env_step<true, false, false, false>, k_env_step<true, true, false, false>,
                                                                 k_env_step<false, false, false, false>, k_env_step<false, true, false, false>)),
                           reinterpret_cast<const void*>(variant(T, k_env_step<true, false, false, false, true>, k_env_step<true, true, false, false, true>,
                                                                 k_env_step<false, false, false, false, true>, k_env_step<false, true, false, false, true>)),
                           reinterpret_cast<const void*>(variant(T, k_env_step<true, false, false, true>, k_env_step<true, true, false, true>,
                                                                 k_env_step<false, false, false, true>, k_env_step<false, true, false, true>)),
                           reinterpret_cast<const void*>(variant(T, k_env_step<true, false, true, true>, k_env_step<true, true, true, true>,
                                                                 k_env_step<false, false, true, true>, k_env_step<false, true, true, true>)),
                           reinterpret_cast<const void*>(variant(T, k_env_count<true, false, false>, k_env_count<true, true, false>,
                                                                 k_env_count<false, false, false>, k_env_count<false, true, false>)),
                           reinterpret_cast<const void*>(variant(T, k_env_count<true, false, true>, k_env_count<true, true, true>,
                                                                 k_env_count<false, false, true>, k_env_count<false, true, true>))})
        set_lds(fn, lds);
}

void prepare_grouped_launches(u32 v, size_t lds)
{
    set_lds(reinterpret_cast<const void*>(variant_of(v, k_env_step_grouped<false, false>, k_env_step_grouped<true, false>,
                                                     k_env_step_grouped<false, true>, k_env_step_grouped<true, true>)),
            lds);
    set_lds(reinterpret_cast<const void*>(variant_of(v, k_env_count_grouped<false, false>, k_env_count_grouped<true, false>,
                                                     k_env_count_grouped<false, true>, k_env_count_grouped<true, true>)),
            lds);
}

void launch_env_step_grouped(const EnvArgs& a, u32 v, unsigned nw, size_t lds, hipStream_t stream)
{
    if (a.rows == 0)
        return;
    const auto fn = variant_of(v, k_env_step_grouped<false, false>, k_env_step_grouped<true, false>, k_env_step_grouped<false, true>,
                               k_env_step_grouped<true, true>);
    set_lds(reinterpret_cast<const void*>(fn), lds);
    hipLaunchKernelGGL(fn, dim3(grouped_grid(a.rows, a.instances)), dim3(nw * kWave), lds, stream, a, v);
    launch_check("env step (grouped)");
}

void launch_env_count_grouped(const CountArgs& a, u32 v, unsigned nw, size_t lds, hipStream_t stream)
{
    if (a.rows == 0)
        return;
    const auto fn = variant_of(v, k_env_count_grouped<false, false>, k_env_count_grouped<true, false>, k_env_count_grouped<false, true>,
                               k_env_count_grouped<true, true>);
    set_lds(reinterpret_cast<const void*>(fn), lds);
    hipLaunchKernelGGL(fn, dim3(grouped_grid(a.rows, a.instances)), dim3(nw * kWave), lds, stream, a, v);
    launch_check("env count (grouped)");
}

void launch_group_rows(const i32* task_ids, u64 rows, u32 instances, u32* hist, u32* order, u32* starts, u32* chunk_start, u32* status,
                       hipStream_t stream)
{
    launch_fill_u32(hist, instances + 1, 0, stream);
    const unsigned blocks = static_cast<unsigned>(std::max<u64>(1, (rows + kGroupBlock * kGroupRowsPerThread - 1) / (kGroupBlock * kGroupRowsPerThread)));
    if (rows)
    {
        hipLaunchKernelGGL(k_group_count, dim3(blocks), dim3(kGroupBlock), 0, stream, task_ids, rows, instances, hist, status);
        launch_check("group count");
    }
    hipLaunchKernelGGL(k_group_scan, dim3(1), dim3(kGroupBlock), 0, stream, hist, instances, starts, chunk_start);
    launch_check("group scan");
    if (rows)
    {
        hipLaunchKernelGGL(k_group_scatter, dim3(blocks), dim3(kGroupBlock), 0, stream, task_ids, rows, instances, hist, order);
        launch_check("group scatter");
    }
}

void launch_expand(const ExpandArgs& a, hipStream_t stream)
{
    if (a.rows == 0)
        return;
    size_t lds = 0;
    const unsigned nw = waves_per_block(a.T, &lds);
    const bool group = a.groups.order != nullptr;
    if (a.witness && group)
        throw std::invalid_argument("mymyr_amd: expand: witness pruning over a task table is not supported by the device expansion");
    const auto fn = group ? variant(a.T, k_expand<true, false, true>, k_expand<true, true, true>, k_expand<false, false, true>,
                                    k_expand<false, true, true>)
                    : a.witness ? variant(a.T, k_expand<true, false, false, true>, k_expand<true, true, false, true>,
                                          k_expand<false, false, false, true>, k_expand<false, true, false, true>)
                                : variant(a.T, k_expand<true, false, false>, k_expand<true, true, false>, k_expand<false, false, false>,
                                          k_expand<false, true, false>);
    set_lds(reinterpret_cast<const void*>(fn), lds);
    // one block per nw rows: rows differ widely in successors, and the dispatcher balances them as blocks finish
    hipLaunchKernelGGL(fn, dim3(one_instance_grid(a.rows, nw, group, 0, false)), dim3(nw * kWave), lds, stream, a);
    launch_check("expand");
}

void launch_offsets_i32(const u64* src, u64 n, i32* dst, hipStream_t stream)
{
    hipLaunchKernelGGL(k_offsets_i32, dim3(blocks_for(n, 256)), dim3(256), 0, stream, src, n, dst);
    launch_check("expand offsets");
}

void launch_kept_counts(const u32* counts, const u32* noops, u64 rows, u32* kept, hipStream_t stream)
{
    if (rows == 0)
        return;
    hipLaunchKernelGGL(k_kept_counts, dim3(blocks_for(rows, 256)), dim3(256), 0, stream, counts, noops, rows, kept);
    launch_check("expand kept counts");
}

void launch_pad(const PadArgs& a, hipStream_t stream)
{
    if (a.rows == 0)
        return;
    constexpr unsigned nw = 4;
    hipLaunchKernelGGL(k_pad, dim3(grid_for(a.rows, nw)), dim3(nw * kWave), 0, stream, a);
    launch_check("pad");
}

void launch_label_actions(const i32* offsets, const i32* schema, const i32* binding, u32 L, u64 rows, const i32* label_schema,
                          const i32* label_binding, u32 stride, i64* actions, hipStream_t stream)
{
    if (rows == 0)
        return;
    hipLaunchKernelGGL(k_label_actions, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(rows, 256), 16384))), dim3(256), 0, stream, offsets,
                       schema, binding, L, rows, label_schema, label_binding, stride, actions);
    launch_check("label actions");
}

void launch_encode_atoms(const u64* states, u64 rows, u32 words, u32 W, i32* out, u32 max_atoms, u32* status, hipStream_t stream)
{
    if (rows == 0)
        return;
    hipLaunchKernelGGL(k_encode, dim3(grid_for(rows, 1)), dim3(kWave), 0, stream, states, rows, words, W, out, max_atoms, status);
    launch_check("encode atoms");
}

void launch_env_reset(const InstDev* inst, u32 instances, u64* states, u64 rows, u32 words, const u8* mask, i32* task_ids, i32* steps,
                      u8* at_goal, i32* count, u32* cache, u32 cache_width, u32* status, hipStream_t stream)
{
    if (rows == 0)
        return;
    const u64 total = rows * words;
    hipLaunchKernelGGL(k_env_reset, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(total, 256), 65536))), dim3(256), 0, stream, inst,
                       instances, states, rows, words, mask, task_ids, steps, at_goal, count, status);
    launch_check("env reset");
    if (cache)
    {
        const u64 cells = rows * cache_width;
        hipLaunchKernelGGL(k_env_reset_cache, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(cells, 256), 65536))), dim3(256), 0,
                           stream, inst, instances, rows, cache_width, mask, task_ids, cache);
        launch_check("env reset cache");
    }
}

void launch_env_random_actions(const u64* seed, const u64* seeds, const u32* env_ids, u64 first_env, const u64* draws, const i32* count,
                               u64 rows, u32 max_actions, i64* out, hipStream_t stream)
{
    if (rows == 0)
        return;
    hipLaunchKernelGGL(k_env_random_actions, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(rows, 256), 4096))), dim3(256), 0, stream,
                       seed, seeds, env_ids, first_env, draws, count, rows, max_actions, out);
    launch_check("env random actions");
}

void launch_check_ids(const i32* ids, u64 rows, u32 instances, u32* status, hipStream_t stream)
{
    if (rows == 0 || !ids)
        return;
    hipLaunchKernelGGL(k_check_ids, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(rows, 256), 1024))), dim3(256), 0, stream, ids, rows,
                       instances, status);
    launch_check("check task ids");
}

void launch_set_word(u64* p, u64 v, hipStream_t stream)
{
    hipLaunchKernelGGL(k_set_word, dim3(1), dim3(1), 0, stream, p, v);
    launch_check("set word");
}

void launch_env_sample_next(const SamplerDev& sampler, const u64* seed, u64 first_env, u64 rows, const u32* reset_counts,
                            const u64* sampling_seeds, const u32* env_ids, i32* next, hipStream_t stream)
{
    if (rows == 0)
        return;
    hipLaunchKernelGGL(k_env_sample_next, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(rows, 256), 4096))), dim3(256), 0, stream,
                       sampler, seed, first_env, rows, reset_counts, sampling_seeds, env_ids, next);
    launch_check("env sample next");
}

void launch_visited_restart(const VisitedDev& v, const InstDev* inst, u32 instances, const u64* states, u64 rows, u32 words,
                            const u8* mask, const i32* task_ids, bool current, hipStream_t stream)
{
    if (rows == 0 || !v.capacity)
        return;
    hipLaunchKernelGGL(k_visited_restart, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(rows, 4), 16384))), dim3(256), 0, stream, v, inst,
                       instances, states, rows, words, mask, task_ids, current ? 1u : 0u);
    launch_check("visited restart");
}

void launch_visited_mask(const u64* table, const i32* count, u64 table_rows, u32 capacity, const u64* succ_hash, const i32* parent,
                         const i32* rows, u64 parents, u64 size, u8* out, hipStream_t stream)
{
    if (size == 0)
        return;
    hipLaunchKernelGGL(k_visited_mask, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(size, 256), 16384))), dim3(256), 0, stream, table,
                       count, table_rows, capacity, succ_hash, parent, rows, parents, size, out);
    launch_check("visited mask");
}

void launch_env_reset_draw(const SamplerDev& sampler, const u64* seed, u64 first_env, u64 rows, const u8* mask, bool sample, i32* task_ids,
                           u32* reset_counts, const u64* sampling_seeds, const u32* env_ids, hipStream_t stream)
{
    if (rows == 0 || !reset_counts)
        return;
    hipLaunchKernelGGL(k_env_reset_draw, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(rows, 256), 4096))), dim3(256), 0, stream,
                       sampler, seed, first_env, rows, mask, sample ? 1u : 0u, task_ids, reset_counts, sampling_seeds, env_ids);
    launch_check("env reset draw");
}

void launch_env_reset_goals(const InstDev* inst, u32 instances, u64 rows, u32 words, const u8* mask, const i32* task_ids, u64* goal_pos,
                            u64* goal_neg, bool keep_goals, u8* at_goal, u32* status, hipStream_t stream)
{
    if (rows == 0)
        return;
    hipLaunchKernelGGL(k_env_reset_goals, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(rows, 256), 4096))), dim3(256), 0, stream, inst,
                       instances, rows, words, mask, task_ids, goal_pos, goal_neg, keep_goals ? 1u : 0u, at_goal, status);
    launch_check("env reset goals");
}

void launch_successors(const TaskDev& T, const u64* states, u64 rows, u32 words, u32 cap, i32* count, i32* schema, i32* binding,
                       u64* succ, u32* status, hipStream_t stream)
{
    if (rows == 0)
        return;
    size_t lds = 0;
    const unsigned nw = waves_per_block(T, &lds);
    const auto fn = variant(T, k_successors<true, false>, k_successors<true, true>, k_successors<false, false>, k_successors<false, true>);
    set_lds(reinterpret_cast<const void*>(fn), lds);
    hipLaunchKernelGGL(fn, dim3(grid_for(rows, nw)), dim3(nw * kWave), lds, stream, T, states, rows, words, cap, count, schema,
                       binding, succ, status);
    launch_check("successors");
}
}  // namespace mya
