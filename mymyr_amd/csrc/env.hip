// Lifted matching (lifted.hpp) and the device env step (env.hpp). One 64-lane block per state row.

#include "env.hpp"
#include "runtime.hpp"

namespace mya
{
TaskDev task_dev(const u64* img, const DevTaskHeader& h)
{
    TaskDev t{};
    t.schemas = reinterpret_cast<const DevSchema*>(img + h.off_schemas);
    t.steps = reinterpret_cast<const DevStep*>(img + h.off_steps);
    t.cons = reinterpret_cast<const DevCons*>(img + h.off_cons);
    t.checks = reinterpret_cast<const DevCheck*>(img + h.off_checks);
    t.effects = reinterpret_cast<const DevEffect*>(img + h.off_effects);
    t.pairs = reinterpret_cast<const DevPair*>(img + h.off_pairs);
    t.rs = img + h.off_rs;
    t.slot_of = reinterpret_cast<const u32*>(img + h.off_slot_of);
    t.records = img + h.off_records;
    t.dom0 = img + h.off_dom0;
    t.static_rows = img + h.off_static_rows;
    t.static_meta = reinterpret_cast<const DevStaticMeta*>(img + h.off_static_meta);
    t.static_words = img;
    t.goal_pos = reinterpret_cast<const u32*>(img + h.off_goal_pos);
    t.goal_neg = reinterpret_cast<const u32*>(img + h.off_goal_neg);
    t.initial = img + h.off_initial;
    t.pred_arity = reinterpret_cast<const u32*>(img + h.off_pred_arity);
    t.pos_begin = reinterpret_cast<const u32*>(img + h.off_pos_begin);
    t.pred_pairs = img + h.off_pred_pairs;
    t.pred_offset = img + h.off_pred_offset;
    t.fluent_count = h.fluent_count;
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
    return t;
}

size_t env_lds_bytes(const DevTaskHeader& h) { return static_cast<size_t>(lds_words(h)) * sizeof(u64); }

namespace
{
constexpr int kEB = 64;  // one wavefront per block

struct Lds
{
    u64* view;    // [view_words]
    u32* bind;    // [kMaxParams][64]: lane columns
    u32* counts;  // [kCountCache]
    u64* cur_m;   // [kMaxParams][64]: enumeration cursors (candidate bits left)
    u32* cur_w;   // [kMaxParams][64]: enumeration cursors (word index)
    u32* eff;     // [64]: effect slots (lane 0)
    u32* before;  // [64]: effect atoms' bits before the move (lane 0)
};

__device__ __forceinline__ Lds lds_layout(u64* base, const TaskDev& T)
{
    Lds l;
    u64* p = base;
    l.view = p;
    p += T.view_words;
    l.bind = reinterpret_cast<u32*>(p);
    p += (kMaxParams * 64) / 2;
    l.counts = reinterpret_cast<u32*>(p);
    p += kCountCache / 2;
    l.cur_m = p;
    p += kMaxParams * 64;
    l.cur_w = reinterpret_cast<u32*>(p);
    p += (kMaxParams * 64) / 2;
    l.eff = reinterpret_cast<u32*>(p);
    p += 32;
    l.before = reinterpret_cast<u32*>(p);
    return l;
}

/// 64 bits of a row (bit 0 = object row_lo, `words` words) for objects [obj_start, obj_start + 64); zeros outside.
__device__ __forceinline__ u64 extract64(const u64* row, u32 words, u32 row_lo, u32 obj_start)
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

__device__ __forceinline__ bool row_bit(const u64* row, u32 slot) { return (row[slot >> 6] >> (slot & 63)) & 1; }

/// The candidate bits of step `st` for objects [st.lo + 64 w, + 64) under the lane's bindings.
__device__ u64 cand_word(const TaskDev& T, const Lds& L, const DevStep& st, u32 w, u32 lane)
{
    u64 a = ~u64{0};
    const u32 obj0 = st.lo + 64 * w;
    for (u32 ci = st.cons_begin; ci < st.cons_end; ++ci)
    {
        const DevCons c = T.cons[ci];
        u64 v;
        if (c.kind == static_cast<u32>(ConsKind::Dom0))
            v = T.dom0[c.table + w];
        else if (c.kind == static_cast<u32>(ConsKind::ViewUnary))
        {
            const DevPair p = T.pairs[c.table];
            v = extract64(L.view + p.offset, p.dst_words, p.dst_lo, obj0);
        }
        else if (c.kind == static_cast<u32>(ConsKind::ViewRow))
        {
            const DevPair p = T.pairs[c.table];
            const u32 so = c.src == kNone ? c.obj : L.bind[c.src * 64 + lane];
            const u32 ri = so - p.src_lo;
            v = ri < p.src_n ? extract64(L.view + p.offset + static_cast<u64>(ri) * p.dst_words, p.dst_words, p.dst_lo, obj0) : 0;
        }
        else
        {
            const u32 so = L.bind[c.src * 64 + lane];
            v = extract64(T.static_rows + (static_cast<u64>(c.table) * T.n + so) * T.ow, T.ow, 0, obj0);
        }
        a &= c.neg ? ~v : v;
    }
    return a;
}

__device__ bool check_holds(const TaskDev& T, const Lds& L, const DevCheck& c, const u64* row, u32 lane)
{
    u32 objs[6];
#pragma unroll
    for (int i = 0; i < 6; ++i)
    {
        const i32 t = c.terms[i];
        objs[i] = (static_cast<u32>(i) < c.nterms) ? (t < 0 ? static_cast<u32>(-(t + 1)) : L.bind[t * 64 + lane]) : 0;
    }
    bool h;
    if (c.kind == static_cast<u32>(CheckKind::Fluent))
    {
        u64 key = T.pred_offset[c.pred];
        const u32 pb = T.pos_begin[c.pred];
#pragma unroll
        for (int i = 0; i < 6; ++i)
            if (static_cast<u32>(i) < c.nterms)
                key += T.rs[static_cast<u64>(pb + i) * T.n + objs[i]];
        if (key >= T.fluent_count)
            h = false;
        else
        {
            const u32 slot = T.dense ? static_cast<u32>(key) : T.slot_of[key];
            h = slot != kNone && row_bit(row, slot);
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

__device__ __forceinline__ bool checks_ok(const TaskDev& T, const Lds& L, u32 b, u32 e, const u64* row, u32 lane)
{
    for (u32 k = b; k < e; ++k)
        if (!check_holds(T, L, T.checks[k], row, lane))
            return false;
    return true;
}

/// Bindings completing steps [si, se) sequentially in this lane (its own binding column): an iterative nested loop
/// whose per-level cursor (current word index and remaining candidate bits) lives in the lane's LDS columns.
__device__ u32 count_from(const TaskDev& T, const Lds& L, const u64* row, u32 si, u32 se, u32 lane)
{
    if (si == se)
        return 1;
    u32 total = 0;
    u32 d = 0;  // level: step si + d
    L.cur_w[lane] = 0;
    L.cur_m[lane] = cand_word(T, L, T.steps[si], 0, lane);
    for (;;)
    {
        const DevStep st = T.steps[si + d];
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
            u32 w = L.cur_w[d * 64 + lane] + 1;
            if (w < st.words)
            {
                L.cur_w[d * 64 + lane] = w;
                L.cur_m[d * 64 + lane] = cand_word(T, L, st, w, lane);
                continue;
            }
            if (d == 0)
                break;
            --d;
            continue;
        }
        const u32 b = static_cast<u32>(__builtin_ctzll(m));
        L.cur_m[d * 64 + lane] = m & (m - 1);
        L.bind[st.param * 64 + lane] = st.lo + 64 * L.cur_w[d * 64 + lane] + b;
        if (chk && !checks_ok(T, L, st.check_begin, st.check_end, row, lane))
            continue;
        if (last)
        {
            ++total;
            continue;
        }
        ++d;
        L.cur_w[d * 64 + lane] = 0;
        L.cur_m[d * 64 + lane] = cand_word(T, L, T.steps[si + d], 0, lane);
    }
    return total;
}

/// Bindings completing steps [si, se), the first step's candidates split over the lanes (one bit per lane); the
/// bound prefix must be in every lane's column. Wave-uniform result.
__device__ u32 count_wave(const TaskDev& T, const Lds& L, const u64* row, u32 si, u32 se, u32 lane)
{
    if (si == se)
        return 1;
    const DevStep st = T.steps[si];
    const bool chk = st.check_begin != st.check_end;
    u32 mine = 0;
    for (u32 w = 0; w < st.words; ++w)
    {
        const u64 m = cand_word(T, L, st, w, lane);
        if (!((m >> lane) & 1))
            continue;
        L.bind[st.param * 64 + lane] = st.lo + 64 * w + lane;
        if (chk && !checks_ok(T, L, st.check_begin, st.check_end, row, lane))
            continue;
        mine += count_from(T, L, row, si + 1, se, lane);
    }
    return wave_sum(mine);
}

__device__ __forceinline__ u32 schema_count(const TaskDev& T, const Lds& L, const u64* row, u32 s, u32 lane)
{
    const DevSchema& S = T.schemas[s];
    if (S.never || !checks_ok(T, L, S.ground_begin, S.ground_end, row, lane))
        return 0;
    return count_wave(T, L, row, S.plan_begin[0], S.plan_begin[1], lane);
}

/// Successors of the state (witness pruning off); per-schema counts of the first kCountCache schemas into LDS.
__device__ u32 count_all(const TaskDev& T, const Lds& L, const u64* row, u32 lane)
{
    u32 total = 0;
    for (u32 s = 0; s < T.num_schemas; ++s)
    {
        const u32 c = schema_count(T, L, row, s, lane);
        if (s < kCountCache && lane == 0)
            L.counts[s] = c;
        total += c;
    }
    __syncthreads();
    return total;
}

/// The schema holding successor `a` (< total) and the rank within it.
__device__ void select_schema(const TaskDev& T, const Lds& L, const u64* row, u32 a, u32 lane, u32* schema, u32* rank)
{
    for (u32 s = 0; s < T.num_schemas; ++s)
    {
        const u32 c = s < kCountCache ? L.counts[s] : schema_count(T, L, row, s, lane);
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

__device__ __forceinline__ void set_bind_all(const Lds& L, u32 param, u32 obj, u32 lane) { L.bind[param * 64 + lane] = obj; }

/// The rank-th applicable binding of schema s in lexicographic order into every lane's column. false: not found.
__device__ bool pick(const TaskDev& T, const Lds& L, const u64* row, u32 s, u32 rank, u32 lane)
{
    const DevSchema& S = T.schemas[s];
    u32 a = rank;
    for (u32 i = 0; i < S.arity; ++i)
    {
        const DevStep F = T.steps[S.filter_step[i]];
        const u32 pb = S.plan_begin[i + 1], pe = S.plan_begin[i + 2];
        const bool chk = F.check_begin != F.check_end;
        bool found = false;
        for (u32 w = 0; w < F.words && !found; ++w)
        {
            const u64 m = cand_word(T, L, F, w, lane);
            u32 c = 0;
            if ((m >> lane) & 1)
            {
                L.bind[i * 64 + lane] = F.lo + 64 * w + lane;
                if (!chk || checks_ok(T, L, F.check_begin, F.check_end, row, lane))
                    c = count_from(T, L, row, pb, pe, lane);
            }
            const u32 incl = wave_inclusive(c);
            const u32 tot = __shfl(incl, kWave - 1, kWave);
            if (a < tot)
            {
                const u64 over = __ballot(incl > a);
                const u32 win = static_cast<u32>(__builtin_ctzll(over));
                const u32 before = __shfl(incl - c, win, kWave);
                a -= before;
                set_bind_all(L, i, F.lo + 64 * w + win, lane);
                found = true;
            }
            else
                a -= tot;
        }
        if (!found)
            return false;
    }
    return true;
}

__device__ __forceinline__ u32 effect_slot(const TaskDev& T, const Lds& L, const DevEffect& e, u32 lane)
{
    u64 cid = e.base;
    for (u32 v = 0; v < e.nvar; ++v)
        cid += T.rs[static_cast<u64>(e.var_pos[v]) * T.n + L.bind[e.var_param[v] * 64 + lane]];
    if (cid >= T.fluent_count)
        return kNone;
    return T.dense ? static_cast<u32>(cid) : T.slot_of[cid];
}

/// Sets (on) or clears the view bits of atom slot s (one lane).
__device__ void view_update(const TaskDev& T, const Lds& L, u32 s, bool on)
{
    const u64 rec = T.records[s];
    const u32 pred = static_cast<u32>(rec & 0xFFFF), a0 = static_cast<u32>((rec >> 16) & 0xFFFF), a1 = static_cast<u32>((rec >> 32) & 0xFFFF);
    const u64 pp = T.pred_pairs[pred];
    const u32 ar = T.pred_arity[pred];
    for (int d = 0; d < 2; ++d)
    {
        const u32 pi = d == 0 ? static_cast<u32>(pp) : static_cast<u32>(pp >> 32);
        if (pi == kNone)
            continue;
        const DevPair P = T.pairs[pi];
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
        u64* w = L.view + P.offset + static_cast<u64>(ri) * P.dst_words + (bi >> 6);
        const u64 bit = u64{1} << (bi & 63);
        if (on)
            *w |= bit;
        else
            *w &= ~bit;
    }
}

/// Builds the view of `row` (all lanes).
__device__ void build_view(const TaskDev& T, const Lds& L, const u64* row, u32 lane)
{
    for (u32 k = lane; k < T.view_words; k += kWave)
        L.view[k] = 0;
    __syncthreads();
    for (u32 w = lane; w < T.W; w += kWave)
    {
        u64 x = row[w];
        while (x)
        {
            const u32 s = w * 64 + static_cast<u32>(__builtin_ctzll(x));
            x &= x - 1;
            if (s >= T.fluent_slots)
                break;  // bits past the task's slots belong to no atom
            const u64 rec = T.records[s];
            const u32 pred = static_cast<u32>(rec & 0xFFFF);
            const u64 pp = T.pred_pairs[pred];
            if (pp == ~u64{0})
                continue;
            const u32 a0 = static_cast<u32>((rec >> 16) & 0xFFFF), a1 = static_cast<u32>((rec >> 32) & 0xFFFF);
            const u32 ar = T.pred_arity[pred];
            for (int d = 0; d < 2; ++d)
            {
                const u32 pi = d == 0 ? static_cast<u32>(pp) : static_cast<u32>(pp >> 32);
                if (pi == kNone)
                    continue;
                const DevPair P = T.pairs[pi];
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
                atomicOr(reinterpret_cast<unsigned long long*>(L.view + P.offset + static_cast<u64>(ri) * P.dst_words + (bi >> 6)),
                         1ull << (bi & 63));
            }
        }
    }
    __syncthreads();
}

/// The ascending set-bit slots of `row` (W words) into out[0, max_atoms), -1 padded (all lanes).
__device__ void encode_row(const u64* row, u32 W, i32* out, u32 max_atoms, u32 lane, u32* status)
{
    u32 base = 0;
    for (u32 w0 = 0; w0 < W; w0 += kWave)
    {
        const u32 w = w0 + lane;
        u64 x = w < W ? row[w] : 0;
        const u32 c = static_cast<u32>(__popcll(x));
        const u32 incl = wave_inclusive(c);
        u32 k = base + incl - c;
        while (x)
        {
            const u32 b = static_cast<u32>(__builtin_ctzll(x));
            x &= x - 1;
            if (k < max_atoms)
                out[k] = static_cast<i32>(w * 64 + b);
            ++k;
        }
        base += __shfl(incl, kWave - 1, kWave);
    }
    for (u32 k = base + lane; k < max_atoms; k += kWave)
        out[k] = -1;
    if (base > max_atoms && lane == 0)
        atomicOr(status, kStatusCapacity);
}

__device__ bool goal_test(const TaskDev& T, const u64* row, u32 lane)
{
    bool ok = true;
    for (u32 i = lane; i < T.ngp; i += kWave)
        ok = ok && row_bit(row, T.goal_pos[i]);
    for (u32 i = lane; i < T.ngn; i += kWave)
        ok = ok && !row_bit(row, T.goal_neg[i]);
    return !T.goal_unsat && __ballot(!ok) == 0;
}

/// Applies the effects of the picked binding of schema s to `row` (global) and the view: delete, then add.
__device__ void apply_effects(const TaskDev& T, const Lds& L, u64* row, u32 s, u32 lane, u32* status)
{
    const DevSchema& S = T.schemas[s];
    if (lane == 0)
    {
        constexpr u32 kMaxEff = 64;
        u32* slot = L.eff;
        u32* before = L.before;
        const u32 ne = min(S.eff_end - S.eff_begin, kMaxEff);
        if (S.eff_end - S.eff_begin > kMaxEff)
            atomicOr(status, kStatusCapacity);
        for (u32 k = 0; k < ne; ++k)
        {
            slot[k] = effect_slot(T, L, T.effects[S.eff_begin + k], lane);
            before[k] = slot[k] != kNone && row_bit(row, slot[k]);
            if (k < S.nadd && slot[k] == kNone)
                atomicOr(status, kStatusNoSlot);
        }
        for (u32 k = S.nadd; k < ne; ++k)
            if (slot[k] != kNone)
                row[slot[k] >> 6] &= ~(u64{1} << (slot[k] & 63));
        for (u32 k = 0; k < S.nadd && k < ne; ++k)
            if (slot[k] != kNone)
                row[slot[k] >> 6] |= u64{1} << (slot[k] & 63);
        for (u32 k = S.nadd; k < ne; ++k)
            if (slot[k] != kNone && before[k] && !row_bit(row, slot[k]))
                view_update(T, L, slot[k], false);
        for (u32 k = 0; k < S.nadd && k < ne; ++k)
            if (slot[k] != kNone && !before[k])
                view_update(T, L, slot[k], true);
    }
    __threadfence_block();
    __syncthreads();
}

__global__ __launch_bounds__(kEB) void k_env_step(EnvArgs A)
{
    extern __shared__ u64 smem[];
    const TaskDev& T = *A.T;
    const Lds L = lds_layout(smem, T);
    const u32 lane = threadIdx.x;
    const u32 Lw = A.label_width;
    for (u64 i = blockIdx.x; i < A.rows; i += gridDim.x)
    {
        u64* row = A.states + i * A.words;
        build_view(T, L, row, lane);
        const bool already_goal = A.at_goal[i] != 0;
        const u32 c = count_all(T, L, row, lane);
        // 2. the choice (env.cpp:416-440)
        enum
        {
            kOk = 0,
            kStuck = 1,
            kInvalid = 2,
            kGoal = 3
        };
        u32 st = already_goal ? kGoal : kOk;
        u32 a = 0;
        if (!already_goal && c == 0)
            st = kStuck;
        else if (!already_goal && A.actions)
        {
            const i64 act = A.actions[i];
            if (act < 0 || static_cast<u64>(act) >= c)
                st = kInvalid;
            else
                a = static_cast<u32>(act);
        }
        else if (!already_goal)
            a = successor_index(A.cfg.seed, A.first_env + i, A.draws[i], c);
        u32 schema = kNone, rank = 0;
        if (st == kOk)
        {
            select_schema(T, L, row, a, lane, &schema, &rank);
            if (schema == kNone || !pick(T, L, row, schema, rank, lane))
            {
                if (lane == 0)
                    atomicOr(A.status, kStatusPickFailed);
                st = kStuck;
            }
        }
        if (lane == 0)
        {
            if (A.draws)
                A.draws[i] += 1;
            if (A.schema)
                A.schema[i] = st == kOk ? static_cast<i32>(schema) : -1;
            if (A.invalid)
                A.invalid[i] = st == kInvalid ? 1 : 0;
        }
        if (A.binding)
        {
            const u32 arity = st == kOk ? T.schemas[schema].arity : 0;
            for (u32 k = lane; k < Lw; k += kWave)
                A.binding[i * Lw + k] = (st == kOk && k < arity) ? static_cast<i32>(L.bind[k * 64 + lane]) : -1;
        }
        // 3. the move, goal and successor count of the reached state
        bool g = already_goal;
        u32 c2 = c;
        if (st == kOk)
        {
            apply_effects(T, L, row, schema, lane, A.status);
            g = goal_test(T, row, lane);
            c2 = count_all(T, L, row, lane);
        }
        // 4. rewards, termination, truncation (env.cpp:466-485)
        const bool dead = !A.cfg.dead_end_none && !g && ((st == kOk && c2 == 0) || st == kStuck);
        const bool term = g || (dead && A.cfg.dead_end_terminal);
        const bool absorbed = already_goal || (st == kStuck && dead && A.cfg.dead_end_terminal);
        const i32 steps0 = A.steps ? A.steps[i] : 0;
        const i32 t2 = A.steps ? steps0 + (absorbed ? 0 : 1) : 0;
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
        if (A.final_states)
        {
            const u32 FW = A.final_words;
            u64* f = A.final_states + i * FW;
            for (u32 k = lane; k < FW; k += kWave)
                f[k] = k < T.W ? row[k] : 0;
        }
        // 5. the autoreset, or the bookkeeping of the move (the row already holds s')
        const bool reset = A.cfg.autoreset && (term || trunc);
        if (reset)
        {
            for (u32 k = lane; k < A.words; k += kWave)
                row[k] = k < T.W ? T.initial[k] : 0;
            if (lane == 0)
            {
                if (A.count)
                    A.count[i] = static_cast<i32>(A.init_count);
                A.at_goal[i] = A.init_goal ? 1 : 0;
                if (A.steps)
                    A.steps[i] = 0;
            }
        }
        else if (lane == 0)
        {
            A.at_goal[i] = g ? 1 : 0;
            if (A.steps)
                A.steps[i] = t2;
            if (A.count)
                A.count[i] = static_cast<i32>(c2);
        }
        // 6. the observation's encoding: true-atom slots and applicable-schema masks (LDS holds the per-schema counts
        // of the state the row holds unless the row was reset)
        if (A.atoms || A.masks)
        {
            __threadfence_block();
            __syncthreads();
            if (A.atoms)
                encode_row(row, T.W, A.atoms + i * A.max_atoms, A.max_atoms, lane, A.status);
            if (A.masks)
                for (u32 s = lane; s < T.num_schemas; s += kWave)
                {
                    u8 m;
                    if (reset)
                        m = A.init_masks[s];
                    else
                        m = (s < kCountCache ? L.counts[s] : 1u) > 0 ? 1 : 0;
                    A.masks[i * T.num_schemas + s] = m;
                }
            if (A.masks && !reset && T.num_schemas > kCountCache)
                for (u32 s = kCountCache; s < T.num_schemas; ++s)
                {
                    const u32 c = schema_count(T, L, row, s, lane);
                    if (lane == 0)
                        A.masks[i * T.num_schemas + s] = c > 0 ? 1 : 0;
                }
        }
        __syncthreads();
    }
}

__global__ __launch_bounds__(kEB) void k_encode(const u64* states, u64 rows, u32 words, u32 W, i32* out, u32 max_atoms, u32* status)
{
    const u32 lane = threadIdx.x;
    for (u64 i = blockIdx.x; i < rows; i += gridDim.x)
        encode_row(states + i * words, W, out + i * max_atoms, max_atoms, lane, status);
}

__global__ __launch_bounds__(kEB) void k_env_count(const TaskDev* __restrict__ Tp, const u64* states, u64 rows, u32 words, i32* count,
                                                   u8* goal, u8* masks)
{
    extern __shared__ u64 smem[];
    const TaskDev& T = *Tp;
    const Lds L = lds_layout(smem, T);
    const u32 lane = threadIdx.x;
    for (u64 i = blockIdx.x; i < rows; i += gridDim.x)
    {
        const u64* row = states + i * words;
        build_view(T, L, row, lane);
        const u32 c = count_all(T, L, row, lane);
        const bool g = goal_test(T, row, lane);
        if (lane == 0)
        {
            if (count)
                count[i] = static_cast<i32>(c);
            if (goal)
                goal[i] = g ? 1 : 0;
        }
        if (masks)
            for (u32 s = 0; s < T.num_schemas; ++s)
            {
                const u32 cs = s < kCountCache ? L.counts[s] : schema_count(T, L, row, s, lane);
                if (lane == 0)
                    masks[i * T.num_schemas + s] = cs > 0 ? 1 : 0;
            }
        __syncthreads();
    }
}

__global__ void k_env_reset(const TaskDev* __restrict__ Tp, u64* states, u64 rows, u32 words, const u8* mask, i32* steps, u8* at_goal,
                            i32* count, u32 init_count, u32 init_goal)
{
    const TaskDev& T = *Tp;
    const u64 total = rows * words;
    for (u64 k = static_cast<u64>(blockIdx.x) * blockDim.x + threadIdx.x; k < total; k += static_cast<u64>(gridDim.x) * blockDim.x)
    {
        const u64 i = k / words;
        const u32 w = static_cast<u32>(k - i * words);
        if (mask && !mask[i])
            continue;
        states[k] = w < T.W ? T.initial[w] : 0;
        if (w == 0)
        {
            if (steps)
                steps[i] = 0;
            if (at_goal)
                at_goal[i] = init_goal ? 1 : 0;
            if (count)
                count[i] = static_cast<i32>(init_count);
        }
    }
}

// Successor listing: successor k of row i is pick(k) applied to a copy of the row.
__global__ __launch_bounds__(kEB) void k_successors(const TaskDev* __restrict__ Tp, const u64* states, u64 rows, u32 words, u32 cap,
                                                   i32* count, i32* schema, i32* binding, u64* succ, u32* status)
{
    extern __shared__ u64 smem[];
    const TaskDev& T = *Tp;
    const Lds L = lds_layout(smem, T);
    const u32 lane = threadIdx.x;
    const u32 Lw = T.label_width;
    for (u64 i = blockIdx.x; i < rows; i += gridDim.x)
    {
        const u64* row = states + i * words;
        build_view(T, L, row, lane);
        const u32 c = count_all(T, L, row, lane);
        if (lane == 0 && count)
            count[i] = static_cast<i32>(c);
        for (u32 k = 0; k < c && k < cap; ++k)
        {
            u32 s = kNone, rank = 0;
            select_schema(T, L, row, k, lane, &s, &rank);
            const bool ok = s != kNone && pick(T, L, row, s, rank, lane);
            if (!ok)
            {
                if (lane == 0)
                    atomicOr(status, kStatusPickFailed);
                break;
            }
            const u64 o = i * cap + k;
            if (lane == 0 && schema)
                schema[o] = static_cast<i32>(s);
            const DevSchema& S = T.schemas[s];
            if (binding)
                for (u32 q = lane; q < Lw; q += kWave)
                    binding[o * Lw + q] = q < S.arity ? static_cast<i32>(L.bind[q * 64 + lane]) : -1;
            if (succ)
            {
                u64* dst = succ + o * words;
                for (u32 q = lane; q < words; q += kWave)
                    dst[q] = q < T.W ? row[q] : 0;
                __threadfence_block();
                __syncthreads();
                if (lane == 0)
                {
                    // delete, then add, on the copy
                    for (u32 e = S.eff_begin + S.nadd; e < S.eff_end; ++e)
                    {
                        const u32 sl = effect_slot(T, L, T.effects[e], lane);
                        if (sl != kNone)
                            dst[sl >> 6] &= ~(u64{1} << (sl & 63));
                    }
                    for (u32 e = S.eff_begin; e < S.eff_begin + S.nadd; ++e)
                    {
                        const u32 sl = effect_slot(T, L, T.effects[e], lane);
                        if (sl != kNone)
                            dst[sl >> 6] |= u64{1} << (sl & 63);
                    }
                }
            }
            __syncthreads();
        }
        __syncthreads();
    }
}

unsigned grid_for(u64 rows) { return static_cast<unsigned>(std::min<u64>(rows, u64{1} << 20)); }
}  // namespace

static void set_lds(const void* fn, size_t bytes)
{
    if (bytes > 64 * 1024)
        hip_check(hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, static_cast<int>(bytes)), "LDS size");
}

void launch_env_step(const EnvArgs& a, hipStream_t stream)
{
    if (a.rows == 0)
        return;
    const size_t lds = static_cast<size_t>(a.view_words + kLdsExtraWords) * sizeof(u64);
    set_lds(reinterpret_cast<const void*>(&k_env_step), lds);
    hipLaunchKernelGGL(k_env_step, dim3(grid_for(a.rows)), dim3(kEB), lds, stream, a);
    launch_check("env step");
}

void launch_env_count(const TaskDev* Td, const TaskDev& Th, const u64* states, u64 rows, u32 words, i32* count, u8* goal, u8* masks,
                      hipStream_t stream)
{
    if (rows == 0)
        return;
    const size_t lds = static_cast<size_t>(Th.view_words + kLdsExtraWords) * sizeof(u64);
    set_lds(reinterpret_cast<const void*>(&k_env_count), lds);
    hipLaunchKernelGGL(k_env_count, dim3(grid_for(rows)), dim3(kEB), lds, stream, Td, states, rows, words, count, goal, masks);
    launch_check("env count");
}

void launch_encode_atoms(const u64* states, u64 rows, u32 words, u32 W, i32* out, u32 max_atoms, u32* status, hipStream_t stream)
{
    if (rows == 0)
        return;
    hipLaunchKernelGGL(k_encode, dim3(grid_for(rows)), dim3(kEB), 0, stream, states, rows, words, W, out, max_atoms, status);
    launch_check("encode atoms");
}

void launch_env_reset(const TaskDev* Td, u64* states, u64 rows, u32 words, const u8* mask, i32* steps, u8* at_goal, i32* count,
                      u32 init_count, u32 init_goal, hipStream_t stream)
{
    if (rows == 0)
        return;
    const u64 total = rows * words;
    hipLaunchKernelGGL(k_env_reset, dim3(static_cast<unsigned>(std::min<u64>(blocks_for(total, 256), 65536))), dim3(256), 0, stream, Td,
                       states, rows, words, mask, steps, at_goal, count, init_count, init_goal);
    launch_check("env reset");
}

void launch_successors(const TaskDev* Td, const TaskDev& Th, const u64* states, u64 rows, u32 words, u32 cap, i32* count, i32* schema,
                       i32* binding, u64* succ, u32* status, hipStream_t stream)
{
    if (rows == 0)
        return;
    const size_t lds = static_cast<size_t>(Th.view_words + kLdsExtraWords) * sizeof(u64);
    set_lds(reinterpret_cast<const void*>(&k_successors), lds);
    hipLaunchKernelGGL(k_successors, dim3(grid_for(rows)), dim3(kEB), lds, stream, Td, states, rows, words, cap, count, schema, binding,
                       succ, status);
    launch_check("successors");
}
}  // namespace mya
