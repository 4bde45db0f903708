// Task text reader and task compiler (host C++). See task.hpp for the reference semantics each part follows.

#include "task.hpp"

#include <algorithm>
#include <bit>
#include <charconv>
#include <cstring>
#include <numeric>
#include <set>
#include <functional>
#include <unordered_set>

namespace mya
{
/// The goal's slot lists and goal_unsat from goal_fluent under the current slots.
void resolve_goal(CompiledTask& C);

namespace
{
// ------------------------------------------------------------------------------------------------- text reader
// Token grammar of the reference reader (src/mymyr/formalism/text_format.cpp:22-197): O, P, SI, FI, G, A, then the
// optional X, C and EG sections. Numeric tasks (the N section) are refused.
class Reader
{
public:
    explicit Reader(std::string_view s) : m_s(s) {}

    TaskText read()
    {
        TaskText t;
        expect("O");
        t.objects = u();
        expect("P");
        const u32 np = u();
        for (u32 i = 0; i < np; ++i)
        {
            const std::string_view k = word();
            PredicateText p;
            if (k == "S")
                p.kind = 'S';
            else if (k == "F")
                p.kind = 'F';
            else if (k == "D" || k == "C" || k == "P")
                p.kind = 'D';
            else
                fail("bad predicate kind " + std::string(k));
            p.arity = u();
            p.name = std::string(word());
            t.preds.push_back(std::move(p));
        }
        std::string_view tag = word();
        if (tag == "N")
            fail("numeric tasks are not supported by the device path");
        if (tag != "SI")
            fail("expected SI, got " + std::string(tag));
        atoms(t, t.static_init);
        expect("FI");
        atoms(t, t.fluent_init);
        expect("G");
        const u32 ng = u();
        for (u32 i = 0; i < ng; ++i)
            t.goal.push_back(literal(t, true));
        expect("A");
        const u32 ns = u();
        for (u32 i = 0; i < ns; ++i)
            t.schemas.push_back(schema(t));
        // the optional sections, in the reference's order: X, C, EG (text_format.cpp:122-187)
        tag = at_end() ? std::string_view{} : word();
        if (tag == "X")
        {
            if (u() != 0)
                fail("axioms (derived predicates) are not supported by the device path");
            tag = at_end() ? std::string_view{} : word();
        }
        if (tag == "C")
        {
            // collapsed parameters: "C <k>", then k lines "<schema> <position> <written> <representative or -1>"
            t.unused_parameters_collapsed = true;
            const u32 k = u();
            for (u32 i = 0; i < k; ++i)
            {
                CollapsedText c;
                c.schema = u();
                if (c.schema >= t.schemas.size())
                    fail("collapsed parameter of an unknown schema");
                c.position = u();
                c.written = u() != 0;
                c.representative = i32v();
                t.collapsed.push_back(c);
            }
            // the reference's checks (task_data.cpp:136-147): per schema, positions ascend and lie among the parameters
            // before collapsing; a representative is an object
            std::stable_sort(t.collapsed.begin(), t.collapsed.end(), [](const CollapsedText& a, const CollapsedText& b) { return a.schema < b.schema; });
            for (size_t a = 0; a < t.collapsed.size();)
            {
                size_t b = a;
                while (b < t.collapsed.size() && t.collapsed[b].schema == t.collapsed[a].schema)
                    ++b;
                const u32 before = t.schemas[t.collapsed[a].schema].arity + static_cast<u32>(b - a);
                for (size_t j = a; j < b; ++j)
                {
                    const CollapsedText& c = t.collapsed[j];
                    if (c.position >= before || (j > a && t.collapsed[j - 1].position >= c.position))
                        fail("collapsed parameter positions must ascend within the schema's parameters before collapsing");
                    if (c.representative >= 0 && static_cast<u32>(c.representative) >= t.objects)
                        fail("collapsed parameter representative out of range");
                    if (c.representative < -1)
                        fail("collapsed parameter representative out of range");
                }
                a = b;
            }
            tag = at_end() ? std::string_view{} : word();
        }
        if (tag == "EG")
        {
            // the encoding goal: "EG <complete> <k>", then k ground literals "<pred> <positive> <objects...>"
            t.encoding_goal_recorded = true;
            t.encoding_goal_complete = u() != 0;
            const u32 k = u();
            for (u32 i = 0; i < k; ++i)
            {
                GroundLiteralText g;
                g.pred = u();
                if (g.pred >= t.preds.size())
                    fail("encoding goal: predicate out of range");
                g.positive = u() != 0;
                for (u32 j = 0; j < t.preds[g.pred].arity; ++j)
                {
                    const u32 o = u();
                    if (o >= t.objects)
                        fail("encoding goal: object out of range");
                    g.objects.push_back(o);
                }
                t.encoding_goal.push_back(std::move(g));
            }
            std::sort(t.encoding_goal.begin(), t.encoding_goal.end());
            t.encoding_goal.erase(std::unique(t.encoding_goal.begin(), t.encoding_goal.end()), t.encoding_goal.end());
            // the reference's reader stops after the encoding goal: what follows it is not read
        }
        else if (!tag.empty())
            fail("unexpected section " + std::string(tag));
        for (const auto& p : t.preds)
            if (p.kind == 'D')
                fail("derived predicates are not supported by the device path");
        return t;
    }

private:
    [[noreturn]] void fail(const std::string& m) { throw Error("task text: " + m); }
    void skip_ws()
    {
        while (m_pos < m_s.size() && (m_s[m_pos] == ' ' || m_s[m_pos] == '\n' || m_s[m_pos] == '\t' || m_s[m_pos] == '\r'))
            ++m_pos;
    }
    bool at_end()
    {
        skip_ws();
        return m_pos >= m_s.size();
    }
    std::string_view word()
    {
        skip_ws();
        if (m_pos >= m_s.size())
            fail("unexpected end of input");
        const size_t b = m_pos;
        while (m_pos < m_s.size() && !(m_s[m_pos] == ' ' || m_s[m_pos] == '\n' || m_s[m_pos] == '\t' || m_s[m_pos] == '\r'))
            ++m_pos;
        return m_s.substr(b, m_pos - b);
    }
    void expect(const char* s)
    {
        const std::string_view w = word();
        if (w != s)
            fail(std::string("expected ") + s + ", got '" + std::string(w) + "'");
    }
    u32 u()
    {
        const std::string_view w = word();
        u32 v = 0;
        auto [p, ec] = std::from_chars(w.data(), w.data() + w.size(), v);
        if (ec != std::errc{} || p != w.data() + w.size())
            fail("expected unsigned integer, got '" + std::string(w) + "'");
        return v;
    }
    i32 i32v()
    {
        const std::string_view w = word();
        i32 v = 0;
        auto [p, ec] = std::from_chars(w.data(), w.data() + w.size(), v);
        if (ec != std::errc{} || p != w.data() + w.size())
            fail("expected integer, got '" + std::string(w) + "'");
        return v;
    }
    u32 pred(const TaskText& t)
    {
        const u32 p = u();
        if (p >= t.preds.size())
            fail("unknown predicate " + std::to_string(p));
        return p;
    }
    void atoms(const TaskText& t, std::vector<std::vector<u32>>& out)
    {
        const u32 k = u();
        for (u32 i = 0; i < k; ++i)
        {
            std::vector<u32> a{pred(t)};
            for (u32 j = 0; j < t.preds[a[0]].arity; ++j)
            {
                const u32 o = u();
                if (o >= t.objects)
                    fail("object out of range");
                a.push_back(o);
            }
            out.push_back(std::move(a));
        }
    }
    Literal literal(const TaskText& t, bool ground, u32 params = 0)
    {
        Literal l;
        l.pred = pred(t);
        l.positive = u() != 0;
        for (u32 j = 0; j < t.preds[l.pred].arity; ++j)
        {
            i32 x;
            if (ground)
            {
                const u32 o = u();
                if (o >= t.objects)
                    fail("object out of range");
                x = -static_cast<i32>(o) - 1;
            }
            else
            {
                x = i32v();
                if (x >= 0 && static_cast<u32>(x) >= params)
                    fail("parameter out of range");
                if (x < 0 && static_cast<u32>(-(x + 1)) >= t.objects)
                    fail("object out of range");
            }
            l.terms.push_back(x);
        }
        return l;
    }
    SchemaText schema(const TaskText& t)
    {
        SchemaText s;
        s.name = std::string(word());
        s.arity = u();
        expect("L");
        const u32 np = u();
        for (u32 i = 0; i < np; ++i)
            s.pre.push_back(literal(t, false, s.arity));
        expect("E");
        const u32 ne = u();
        for (u32 i = 0; i < ne; ++i)
        {
            // an effect without forall parameters and condition is unconditional (text_format.cpp's schema(), and
            // compile.cpp's split of them from the conditional ones)
            CondEffectText ce;
            ce.extra = u();
            if (ce.extra > 1024)
                fail("more than 1024 forall parameters");
            const u32 total = s.arity + ce.extra;
            expect("L");
            const u32 nc = u();
            for (u32 j = 0; j < nc; ++j)
            {
                Literal l = literal(t, false, total);
                if (t.preds[l.pred].kind == 'D')
                    fail("derived literals in effect conditions are not supported (schema " + s.name + ")");
                ce.cond.push_back(std::move(l));
            }
            expect("F");
            const u32 nf = u();
            for (u32 j = 0; j < nf; ++j)
            {
                Literal l = literal(t, false, total);
                if (t.preds[l.pred].kind != 'F')
                    fail("effect on a non-fluent predicate");
                ce.eff.push_back(std::move(l));
            }
            if (ce.extra == 0 && ce.cond.empty())
                for (Literal& l : ce.eff)
                    s.eff.push_back(std::move(l));
            else
                s.ces.push_back(std::move(ce));
        }
        return s;
    }

    std::string_view m_s;
    size_t m_pos = 0;
};

u64 sat_mul(u64 a, u64 b)
{
    constexpr u64 cap = u64{1} << 62;
    if (a == 0 || b == 0)
        return 0;
    if (a > cap / b)
        return cap;
    return std::min(cap, a * b);
}

using Bits = std::vector<u64>;
inline void set_bit(Bits& b, u32 i) { b[i >> 6] |= u64{1} << (i & 63); }
inline bool test_bit(const Bits& b, u32 i) { return (b[i >> 6] >> (i & 63)) & 1; }
inline bool any_bit(const Bits& b)
{
    for (u64 w : b)
        if (w)
            return true;
    return false;
}
inline u32 popcount(const Bits& b)
{
    u32 c = 0;
    for (u64 w : b)
        c += static_cast<u32>(std::popcount(w));
    return c;
}

bool is_object(i32 t) { return t < 0; }
u32 term_object(i32 t) { return static_cast<u32>(-(t + 1)); }

std::vector<u32> distinct_params(const std::vector<i32>& terms)
{
    std::vector<u32> v;
    for (i32 x : terms)
        if (x >= 0 && std::find(v.begin(), v.end(), static_cast<u32>(x)) == v.end())
            v.push_back(static_cast<u32>(x));
    return v;
}

// Packed static key: sum obj_i * n^(ar-1-i).
u64 static_key(const u32* objs, u32 ar, u32 n)
{
    u64 k = 0;
    for (u32 i = 0; i < ar; ++i)
        k = k * n + objs[i];
    return k;
}

class Compiler
{
public:
    Compiler(TaskText text, AtomsOption atoms) : m_opt(atoms)
    {
        C = std::make_unique<CompiledTask>();
        C->text = std::move(text);
    }

    std::unique_ptr<CompiledTask> run()
    {
        T = &C->text;
        n = T->objects;
        if (n == 0)
            n = 0;
        ow = std::max<u32>(1, words_for(n));
        C->n = n;
        C->ow = ow;
        const u32 m = static_cast<u32>(T->preds.size());
        for (const auto& p : T->preds)
            if (p.arity > 6)
                throw Error("predicate " + p.name + " has arity above 6 (unsupported by the device path)");
        // static key packing must fit 64 bits
        for (u32 p = 0; p < m; ++p)
            if (T->preds[p].kind == 'S')
            {
                long double sp = 1;
                for (u32 i = 0; i < T->preds[p].arity; ++i)
                    sp *= std::max<u32>(n, 1);
                if (sp >= 1.8e19L)
                    throw Error("static predicate " + T->preds[p].name + " has a key space beyond 64 bits");
            }
        setup_statics();
        compute_dom0();
        build_layout();
        choose_mode();
        build_state_tables();
        build_image();
        C->static_keys.assign(T->preds.size(), {});
        for (u32 p = 0; p < T->preds.size(); ++p)
        {
            C->static_keys[p].assign(static_keys[p].begin(), static_keys[p].end());
            std::sort(C->static_keys[p].begin(), C->static_keys[p].end());
        }
        return std::move(C);
    }

private:
    // --------------------------------------------------------------------------------------------- statics
    void setup_statics()
    {
        const u32 m = static_cast<u32>(T->preds.size());
        static_atoms.assign(m, {});
        static_keys.assign(m, {});
        s_unary.assign(m, Bits(ow, 0));
        for (const auto& a : T->static_init)
        {
            if (T->preds[a[0]].kind != 'S')
                throw Error("static initial atom of a non-static predicate");
            static_atoms[a[0]].push_back(&a);
            static_keys[a[0]].insert(static_key(a.data() + 1, T->preds[a[0]].arity, std::max<u32>(n, 1)));
            if (T->preds[a[0]].arity == 1)
                set_bit(s_unary[a[0]], a[1]);
        }
        for (const auto& a : T->fluent_init)
            if (T->preds[a[0]].kind != 'F')
                throw Error("fluent initial atom of a non-fluent predicate");
    }

    bool static_holds(u32 p, const u32* objs) const
    {
        return static_keys[p].count(static_key(objs, T->preds[p].arity, std::max<u32>(n, 1))) != 0;
    }
    bool static_ground_holds(const Literal& l) const
    {
        std::vector<u32> objs;
        for (i32 x : l.terms)
            objs.push_back(term_object(x));
        return static_holds(l.pred, objs.data());
    }

    /// Row table of static `pred`: row(a[from]) has bit a[to] (n rows of ow words, object space).
    u32 static_rows(u32 pred, u32 from, u32 to)
    {
        const auto key = std::make_tuple(pred, from, to);
        if (auto it = m_row_tables.find(key); it != m_row_tables.end())
            return it->second;
        const u32 id = static_cast<u32>(m_row_data.size());
        Bits rows(static_cast<size_t>(std::max<u32>(n, 1)) * ow, 0);
        for (const auto* a : static_atoms[pred])
        {
            const u32 f = (*a)[1 + from], t = (*a)[1 + to];
            rows[static_cast<size_t>(f) * ow + (t >> 6)] |= u64{1} << (t & 63);
        }
        m_row_data.push_back(std::move(rows));
        m_row_tables.emplace(key, id);
        return id;
    }

    // --------------------------------------------------------------------------------------------- dom0
    // The static domain of each schema parameter: every object, AND static unary literals, AND static binary
    // literals with one constant, AND projections of positive static k-ary literals (compile.cpp:803-915).
    /// Static domains of the variables [0, total) of a literal list: every object, AND static unary literals, AND static
    /// binary literals with one constant, AND projections of positive static k-ary literals (compile.cpp:803-915).
    /// *never: a ground static literal fails or a domain is empty.
    std::vector<Bits> static_domains(const std::vector<Literal>& lits, u32 total, bool* never)
    {
        std::vector<Bits> dom(total, Bits(ow, 0));
        for (u32 v = 0; v < total; ++v)
            for (u32 o = 0; o < n; ++o)
                set_bit(dom[v], o);
        for (const Literal& l : lits)
        {
            const PredicateText& P = T->preds[l.pred];
            if (P.kind == 'D')
                throw Error("derived precondition literals are not supported");
            const bool fluent = P.kind != 'S';
            const auto vars = distinct_params(l.terms);
            if (vars.empty())
            {
                if (!fluent && static_ground_holds(l) != l.positive)
                    *never = true;
                continue;
            }
            if (P.arity == 1)
            {
                if (!fluent)
                    and_bits(dom[vars[0]], s_unary[l.pred], !l.positive);
                continue;
            }
            if (P.arity == 2 && l.terms[0] != l.terms[1])
            {
                const bool f0 = l.terms[0] >= 0, f1 = l.terms[1] >= 0;
                if (f0 && f1)
                    continue;
                const u32 fpos = f0 ? 0 : 1, opos = 1 - fpos;
                const u32 v = static_cast<u32>(l.terms[fpos]);
                const u32 cobj = term_object(l.terms[opos]);
                if (!fluent)
                {
                    const u32 tab = static_rows(l.pred, opos, fpos);
                    Bits row(m_row_data[tab].begin() + static_cast<size_t>(cobj) * ow,
                             m_row_data[tab].begin() + static_cast<size_t>(cobj + 1) * ow);
                    and_bits(dom[v], row, !l.positive);
                }
                continue;
            }
            if (!fluent && l.positive && P.arity >= 3)
            {
                for (u32 i = 0; i < P.arity; ++i)
                    if (l.terms[i] >= 0)
                    {
                        Bits proj(ow, 0);
                        for (const auto* a : static_atoms[l.pred])
                        {
                            bool ok = true;
                            for (u32 j = 0; j < P.arity && ok; ++j)
                                if (l.terms[j] < 0 && (*a)[1 + j] != term_object(l.terms[j]))
                                    ok = false;
                            if (ok)
                                set_bit(proj, (*a)[1 + i]);
                        }
                        and_bits(dom[static_cast<u32>(l.terms[i])], proj, false);
                    }
            }
        }
        for (u32 v = 0; v < total; ++v)
            if (!any_bit(dom[v]))
                *never = true;
        return dom;
    }

    void compute_dom0()
    {
        C->dom0.resize(T->schemas.size());
        C->never.assign(T->schemas.size(), 0);
        C->ce_dom0.assign(T->schemas.size(), {});
        for (u32 si = 0; si < T->schemas.size(); ++si)
        {
            const SchemaText& s = T->schemas[si];
            if (s.arity > kMaxParams)
                throw Error("schema " + s.name + " has " + std::to_string(s.arity) + " parameters; the device path supports at most " +
                            std::to_string(kMaxParams));
            bool never = false;
            C->dom0[si] = static_domains(s.pre, s.arity, &never);
            // a collapsed parameter without a representative (no object of its type): the schema has no action
            // (src/mymyr/task/compile.cpp:1171-1181)
            for (const CollapsedText& c : T->collapsed)
                if (c.schema == si && c.representative < 0)
                    never = true;
            C->never[si] = never ? 1 : 0;
            // the forall parameters of its conditional effects: the static domains their conditions give them (the
            // condition's matcher, compile.cpp:1208-1216)
            for (const CondEffectText& ce : s.ces)
            {
                bool ce_never = false;
                std::vector<Bits> d = static_domains(ce.cond, s.arity + ce.extra, &ce_never);
                C->ce_dom0[si].emplace_back(d.begin() + s.arity, d.end());
                C->has_ce = true;
            }
        }
    }
    void and_bits(Bits& d, const Bits& s, bool neg)
    {
        for (u32 w = 0; w < ow; ++w)
            d[w] &= neg ? ~s[w] : s[w];
    }

    // --------------------------------------------------------------------------------------------- layout
    // Position domains: the objects the add effects can put there (a constant, or the dom0 of the parameter) plus
    // the initial atoms' objects; ranks in object order; the last position has stride 1 (compile.cpp:1363-1455).
    void build_layout()
    {
        const u32 m = static_cast<u32>(T->preds.size());
        std::vector<std::vector<Bits>> bits(m);
        for (u32 p = 0; p < m; ++p)
            if (T->preds[p].kind == 'F')
                bits[p].assign(T->preds[p].arity, Bits(ow, 0));
        for (u32 si = 0; si < T->schemas.size(); ++si)
        {
            const SchemaText& s = T->schemas[si];
            // a term's objects: a constant, a schema parameter's dom0, or a forall parameter's conditional dom0
            auto add_term = [&](u32 p, u32 i, i32 t, const std::vector<Bits>* ce_dom) {
                if (t < 0)
                    set_bit(bits[p][i], term_object(t));
                else
                {
                    const Bits& d = static_cast<u32>(t) < s.arity ? C->dom0[si][static_cast<u32>(t)] : (*ce_dom)[static_cast<u32>(t) - s.arity];
                    for (u32 w = 0; w < ow; ++w)
                        bits[p][i][w] |= d[w];
                }
            };
            for (const Literal& l : s.eff)
                if (l.positive)
                    for (u32 i = 0; i < l.terms.size(); ++i)
                        add_term(l.pred, i, l.terms[i], nullptr);
            for (u32 k = 0; k < s.ces.size(); ++k)
                for (const Literal& l : s.ces[k].eff)
                    if (l.positive)
                        for (u32 i = 0; i < l.terms.size(); ++i)
                            add_term(l.pred, i, l.terms[i], &C->ce_dom0[si][k]);
        }
        for (const auto& a : T->fluent_init)
            for (u32 i = 0; i + 1 < a.size(); ++i)
                set_bit(bits[a[0]][i], a[1 + i]);

        Layout& L = C->layout;
        L.offset.assign(m, kNone64);
        L.size.assign(m, 0);
        L.pos_begin.assign(m, 0);
        u32 positions = 0;
        for (u32 p = 0; p < m; ++p)
            if (T->preds[p].kind == 'F')
            {
                L.pos_begin[p] = positions;
                positions += T->preds[p].arity;
            }
        L.rs.assign(positions, std::vector<u64>(n, Layout::kOutside));
        L.domain.assign(positions, {});
        u64 running = 0;
        for (u32 p = 0; p < m; ++p)
        {
            if (T->preds[p].kind != 'F')
                continue;
            const u32 ar = T->preds[p].arity;
            u64 size = 1;
            for (u32 i = 0; i < ar; ++i)
            {
                const u32 pos = L.pos_begin[p] + i;
                for (u32 o = 0; o < n; ++o)
                    if (test_bit(bits[p][i], o))
                        L.domain[pos].push_back(o);
                size = sat_mul(size, L.domain[pos].size());
            }
            u64 st = 1;
            for (u32 i = ar; i-- > 0;)
            {
                const u32 pos = L.pos_begin[p] + i;
                for (u32 r = 0; r < L.domain[pos].size(); ++r)
                    L.rs[pos][L.domain[pos][r]] = r * st;
                st = sat_mul(st, std::max<u64>(1, L.domain[pos].size()));
            }
            L.size[p] = size;
            L.offset[p] = running;
            running = std::min<u64>(running + size, u64{1} << 62);
        }
        L.fluent_count = running;
    }

    u64 cid_of(u32 p, const u32* args) const { return C->layout.encode(p, args, T->preds[p].arity); }

    // --------------------------------------------------------------------------------------------- reachability
    // The delete-relaxed fixpoint: one rule per (schema, add literal) with the positive fluent preconditions and every
    // static precondition as its body; negative fluent literals dropped; "=" by object identity; a variable no
    // positive literal binds ranges over every object (relaxed_reachability.hpp:3-12). Evaluated by naive rounds of
    // a bitset join until no new atom appears.
    std::vector<u64> reachable_fluents(u64 stop_at = ~u64{0})
    {
        const u32 m = static_cast<u32>(T->preds.size());
        std::vector<u8> reached(C->layout.fluent_count, 0);
        std::vector<u64> list;
        // per fluent predicate: unary bits, binary fwd/bwd rows (object space)
        std::vector<Bits> unary(m);
        std::vector<Bits> fwd(m), bwd(m);
        for (u32 p = 0; p < m; ++p)
            if (T->preds[p].kind == 'F')
            {
                if (T->preds[p].arity == 1)
                    unary[p].assign(ow, 0);
                if (T->preds[p].arity == 2)
                {
                    fwd[p].assign(static_cast<size_t>(std::max<u32>(n, 1)) * ow, 0);
                    bwd[p].assign(static_cast<size_t>(std::max<u32>(n, 1)) * ow, 0);
                }
            }
        auto add_atom = [&](u32 p, const u32* args) -> bool
        {
            const u64 c = cid_of(p, args);
            if (c >= C->layout.fluent_count)
                return false;  // outside every position domain: no canonical id
            if (reached[c])
                return false;
            reached[c] = 1;
            list.push_back(c);
            const u32 ar = T->preds[p].arity;
            if (ar == 1)
                set_bit(unary[p], args[0]);
            else if (ar == 2)
            {
                fwd[p][static_cast<size_t>(args[0]) * ow + (args[1] >> 6)] |= u64{1} << (args[1] & 63);
                bwd[p][static_cast<size_t>(args[1]) * ow + (args[0] >> 6)] |= u64{1} << (args[0] & 63);
            }
            return true;
        };
        auto holds = [&](u32 p, const u32* args) -> bool
        {
            const u64 c = cid_of(p, args);
            return c < C->layout.fluent_count && reached[c];
        };
        for (const auto& a : T->fluent_init)
            add_atom(a[0], a.data() + 1);
        if (list.size() >= stop_at)
        {
            std::sort(list.begin(), list.end());
            return list;
        }

        const u32 eq = equality_pred();
        Bits all_objects(ow, 0);
        for (u32 o = 0; o < n; ++o)
            set_bit(all_objects, o);
        // the rules: one per schema (its precondition, its unconditional effects) and one per conditional effect (the
        // schema's precondition and the effect's condition over the schema's and the forall parameters, its effects)
        std::vector<SchemaText> rules;
        for (const SchemaText& sc : T->schemas)
        {
            rules.push_back(SchemaText{sc.name, sc.arity, sc.pre, sc.eff, {}});
            for (const CondEffectText& ce : sc.ces)
            {
                SchemaText r{sc.name, sc.arity + ce.extra, sc.pre, ce.eff, {}};
                r.pre.insert(r.pre.end(), ce.cond.begin(), ce.cond.end());
                rules.push_back(std::move(r));
            }
        }
        for (bool changed = true; changed;)
        {
            changed = false;
            for (u32 ri = 0; ri < rules.size(); ++ri)
            {
                const SchemaText& s = rules[ri];
                std::vector<const Literal*> body;
                bool has_head = false;
                for (const Literal& l : s.eff)
                    has_head |= l.positive;
                if (!has_head)
                    continue;
                for (const Literal& l : s.pre)
                {
                    const bool fluent = T->preds[l.pred].kind != 'S';
                    if (fluent && !l.positive)
                        continue;  // the delete relaxation
                    body.push_back(&l);
                }
                // variables: everything the body or a head mentions
                std::vector<u8> mentioned(s.arity, 0);
                for (const Literal* l : body)
                    for (i32 x : l->terms)
                        if (x >= 0)
                            mentioned[x] = 1;
                for (const Literal& l : s.eff)
                    if (l.positive)
                        for (i32 x : l.terms)
                            if (x >= 0)
                                mentioned[x] = 1;
                std::vector<u32> vars;
                for (u32 v = 0; v < s.arity; ++v)
                    if (mentioned[v])
                        vars.push_back(v);
                // ground body literals
                bool ok = true;
                for (const Literal* l : body)
                    if (distinct_params(l->terms).empty())
                    {
                        std::vector<u32> objs;
                        for (i32 x : l->terms)
                            objs.push_back(term_object(x));
                        const bool fluent = T->preds[l->pred].kind != 'S';
                        bool h;
                        if (fluent)
                            h = holds(l->pred, objs.data());
                        else if (l->pred == eq)
                            h = objs[0] == objs[1];
                        else
                            h = static_holds(l->pred, objs.data());
                        if (h != l->positive)
                            ok = false;
                    }
                if (!ok)
                    continue;
                // one rule per positive effect literal (its head): the head's variables are enumerated, and each head
                // atom not reached yet is added if some binding of the remaining variables satisfies the body (a
                // search that stops at the first one); schemas with many parameters thus cost one existence search
                // per new head atom instead of an enumeration of all their bindings
                auto greedy = [&](const std::vector<u32>& cand, std::vector<u8>& placed) {
                    std::vector<u32> order;
                    while (order.size() < cand.size())
                    {
                        int best = -1;
                        long best_score = 0;
                        for (u32 v : cand)
                        {
                            if (placed[v])
                                continue;
                            long links = 0, un = 0;
                            for (const Literal* l : body)
                            {
                                const auto ps = distinct_params(l->terms);
                                if (std::find(ps.begin(), ps.end(), v) == ps.end())
                                    continue;
                                if (ps.size() == 1)
                                    ++un;
                                for (u32 q : ps)
                                    if (q != v && placed[q])
                                        ++links;
                            }
                            const long score = links * 1000000 + un * 10000;
                            if (best < 0 || score > best_score)
                                best = static_cast<int>(v), best_score = score;
                        }
                        placed[best] = 1;
                        order.push_back(static_cast<u32>(best));
                    }
                    return order;
                };
                for (const Literal& head : s.eff)
                {
                    if (!head.positive)
                        continue;
                    const std::vector<u32> hv = distinct_params(head.terms);
                    std::vector<u8> placed(s.arity, 0);
                    const std::vector<u32> order_head = greedy(hv, placed);
                    // the remaining variables that the body constrains (a variable only another head mentions does
                    // not change whether this head's body is satisfiable)
                    std::vector<u8> in_body(s.arity, 0);
                    for (const Literal* l : body)
                        for (i32 x : l->terms)
                            if (x >= 0)
                                in_body[x] = 1;
                    std::vector<u32> rest;
                    for (u32 v : vars)
                        if (!placed[v] && in_body[v])
                            rest.push_back(v);
                    const std::vector<u32> order_rest = greedy(rest, placed);
                    std::vector<u32> bind(s.arity, 0);
                    std::vector<u8> bound(s.arity, 0);
                    std::vector<std::vector<u32>> found;
                    std::vector<u32> h;
                    // the variables' domains, arc consistent over the body (a rule whose body cannot hold adds nothing)
                    std::vector<Bits> dom(s.arity, all_objects);
                    if (!arc_consistent(body, dom, unary, fwd, bwd, eq))
                        continue;
                    std::vector<Bits> fixed;
                    enumerate(s, body, order_head, 0, bind, bound, unary, fwd, bwd, reached, eq, dom, [&] {
                        h.assign(1, head.pred);
                        for (i32 x : head.terms)
                            h.push_back(x < 0 ? term_object(x) : bind[x]);
                        if (holds(h[0], h.data() + 1))
                            return true;  // reached already
                        // the head's variables fixed: the remaining domains made arc consistent again, then a search
                        // for one binding of the rest
                        fixed = dom;
                        for (u32 v : hv)
                        {
                            std::fill(fixed[v].begin(), fixed[v].end(), 0);
                            set_bit(fixed[v], bind[v]);
                        }
                        if (!arc_consistent(body, fixed, unary, fwd, bwd, eq))
                            return true;
                        const bool stopped = !enumerate(s, body, order_rest, 0, bind, bound, unary, fwd, bwd, reached, eq, fixed,
                                                        [] { return false; });
                        if (stopped)
                            found.push_back(h);
                        return true;
                    });
                    for (const auto& a : found)
                        if (add_atom(a[0], a.data() + 1))
                            changed = true;
                    if (list.size() >= stop_at)
                    {
                        std::sort(list.begin(), list.end());
                        return list;
                    }
                }
            }
        }
        std::sort(list.begin(), list.end());
        return list;
    }

    u32 equality_pred() const
    {
        for (u32 p = 0; p < T->preds.size(); ++p)
            if (T->preds[p].kind == 'S' && T->preds[p].name == "=" && T->preds[p].arity == 2)
                return p;
        return kNone;
    }

    /// Arc consistency over a rule body's variables: D[v] (object bits) keeps only the objects that satisfy v's unary
    /// literals and have support in every positive binary literal with another variable (the fluent relation as
    /// reached so far, or the static one), repeated until nothing changes. Only objects that no binding of the body
    /// can use are removed, so a search over the domains finds the same bindings. Returns false if a domain emptied
    /// (the body cannot hold).
    bool arc_consistent(const std::vector<const Literal*>& body, std::vector<Bits>& D, const std::vector<Bits>& unary,
                        const std::vector<Bits>& fwd, const std::vector<Bits>& bwd, u32 eq)
    {
        auto empty = [&](const Bits& b) { return std::all_of(b.begin(), b.end(), [](u64 w) { return w == 0; }); };
        for (const Literal* l : body)
        {
            const auto ps = distinct_params(l->terms);
            const bool fluent = T->preds[l->pred].kind != 'S';
            if (ps.size() == 1 && T->preds[l->pred].arity == 1 && l->pred != eq)
                and_bits(D[ps[0]], fluent ? unary[l->pred] : s_unary[l->pred], !l->positive);
        }
        for (bool changed = true; changed;)
        {
            changed = false;
            for (const Literal* l : body)
            {
                if (!l->positive || T->preds[l->pred].arity != 2 || l->terms[0] < 0 || l->terms[1] < 0 || l->terms[0] == l->terms[1])
                    continue;
                const u32 x = static_cast<u32>(l->terms[0]), y = static_cast<u32>(l->terms[1]);
                for (int dir = 0; dir < 2; ++dir)
                {
                    // revise: the objects of `to` with support in some object of `from`
                    const u32 from = dir == 0 ? x : y, to = dir == 0 ? y : x;
                    Bits sup(ow, 0);
                    if (l->pred == eq)
                        sup = D[from];
                    else
                    {
                        const bool fluent = T->preds[l->pred].kind != 'S';
                        const Bits* tab = fluent ? (dir == 0 ? &fwd[l->pred] : &bwd[l->pred])
                                                 : &m_row_data[static_rows(l->pred, dir == 0 ? 0 : 1, dir == 0 ? 1 : 0)];
                        for (u32 w = 0; w < ow; ++w)
                            for (u64 bits = D[from][w]; bits; bits &= bits - 1)
                            {
                                const u32 o = w * 64 + static_cast<u32>(std::countr_zero(bits));
                                for (u32 k = 0; k < ow; ++k)
                                    sup[k] |= (*tab)[static_cast<size_t>(o) * ow + k];
                            }
                    }
                    for (u32 k = 0; k < ow; ++k)
                    {
                        const u64 nv = D[to][k] & sup[k];
                        if (nv != D[to][k])
                        {
                            D[to][k] = nv;
                            changed = true;
                        }
                    }
                    if (empty(D[to]))
                        return false;
                }
            }
        }
        return std::none_of(D.begin(), D.end(), empty);
    }

    /// Binds the variables order[d..] (the earlier ones bound in `bind` / `bound`) in every way the body literals whose
    /// variables are then bound allow, calling leaf() per complete binding; leaf returning false stops the search, and
    /// then so does this (returns false; true: the search ran to its end).
    template<class Leaf>
    bool enumerate(const SchemaText& s, const std::vector<const Literal*>& body, const std::vector<u32>& order, u32 d,
                   std::vector<u32>& bind, std::vector<u8>& bound, const std::vector<Bits>& unary,
                   const std::vector<Bits>& fwd, const std::vector<Bits>& bwd, const std::vector<u8>& reached, u32 eq,
                   const std::vector<Bits>& dom, Leaf&& leaf)
    {
        if (d == order.size())
            return leaf();
        const u32 v = order[d];
        Bits cand = dom[v];
        std::vector<const Literal*> checks;
        for (const Literal* l : body)
        {
            const auto ps = distinct_params(l->terms);
            if (std::find(ps.begin(), ps.end(), v) == ps.end())
                continue;
            bool rest_bound = true;
            for (u32 q : ps)
                if (q != v && !bound[q])
                    rest_bound = false;
            if (!rest_bound)
                continue;
            const bool fluent = T->preds[l->pred].kind != 'S';
            const u32 ar = T->preds[l->pred].arity;
            if (ar == 1 && l->pred != eq)
            {
                and_bits(cand, fluent ? unary[l->pred] : s_unary[l->pred], !l->positive);
                continue;
            }
            if (ar == 2 && l->terms[0] != l->terms[1] && l->pred != eq)
            {
                const u32 vpos = l->terms[0] == static_cast<i32>(v) ? 0 : 1, opos = 1 - vpos;
                const i32 ot = l->terms[opos];
                const u32 oobj = ot < 0 ? term_object(ot) : bind[ot];
                Bits row(ow, 0);
                if (fluent)
                {
                    const Bits& tab = opos == 0 ? fwd[l->pred] : bwd[l->pred];
                    std::copy(tab.begin() + static_cast<size_t>(oobj) * ow, tab.begin() + static_cast<size_t>(oobj + 1) * ow, row.begin());
                }
                else
                {
                    const u32 t = static_rows(l->pred, opos, vpos);
                    std::copy(m_row_data[t].begin() + static_cast<size_t>(oobj) * ow,
                              m_row_data[t].begin() + static_cast<size_t>(oobj + 1) * ow, row.begin());
                }
                and_bits(cand, row, !l->positive);
                continue;
            }
            checks.push_back(l);
        }
        bound[v] = 1;
        for (u32 w = 0; w < ow; ++w)
        {
            u64 word = cand[w];
            while (word)
            {
                const u32 o = w * 64 + static_cast<u32>(std::countr_zero(word));
                word &= word - 1;
                bind[v] = o;
                bool ok = true;
                for (const Literal* l : checks)
                {
                    std::vector<u32> objs;
                    for (i32 x : l->terms)
                        objs.push_back(x < 0 ? term_object(x) : bind[x]);
                    bool h;
                    if (T->preds[l->pred].kind != 'S')
                    {
                        const u64 c = cid_of(l->pred, objs.data());
                        h = c < C->layout.fluent_count && reached[c];
                    }
                    else if (l->pred == eq)
                        h = objs[0] == objs[1];
                    else
                        h = static_holds(l->pred, objs.data());
                    if (h != l->positive)
                    {
                        ok = false;
                        break;
                    }
                }
                if (!ok)
                    continue;
                if (!enumerate(s, body, order, d + 1, bind, bound, unary, fwd, bwd, reached, eq, dom, leaf))
                {
                    bound[v] = 0;
                    return false;
                }
            }
        }
        bound[v] = 0;
        return true;
    }

    // --------------------------------------------------------------------------------------------- atom mode
    // Dense where it is not wider than the reachable slots (task.cpp:106-143).
    void choose_mode()
    {
        const Layout& L = C->layout;
        if (L.fluent_count > (u64{1} << 28))
            throw Error("the typed-dense canonical space of " + std::to_string(L.fluent_count) + " atoms exceeds 2^28");
        u32 max_arity = 0;
        for (const auto& p : T->preds)
            if (p.kind == 'F')
                max_arity = std::max(max_arity, p.arity);
        auto frozen_bytes = [&](u64 atoms)
        {
            const u64 per = (1 + std::max<u64>(1, max_arity)) * 4 + 16 + 8;
            return atoms * per + (L.fluent_count + 1) * 4;
        };
        constexpr u64 kMaxBytes = u64{4} << 30;
        if (m_opt == AtomsOption::Lazy && C->has_ce)
            throw Error("conditional effects are supported by the ground search over frozen atom slots, not with lazy slots");
        if (m_opt == AtomsOption::Lazy)
        {
            // no slots yet: the initial state's atoms take the first ones (build_state_tables); the tables are sized for
            // every canonical atom, as the reference's lazy index is (atom_index.cpp:60-70)
            if (frozen_bytes(L.fluent_count) + L.fluent_count * 8 > kMaxBytes)
                throw Error("lazy atom slots over " + std::to_string(L.fluent_count) + " canonical atoms need more than 4 GiB of records");
            C->mode = AtomMode::Lazy;
            C->slot_of.assign(L.fluent_count, kNone);
            C->fluent_slots = 0;
            C->slot_cid.clear();
            C->words = 1;
            return;
        }
        std::vector<u64> reach;
        AtomMode mode = AtomMode::Dense;
        if (m_opt != AtomsOption::Dense)
        {
            // under auto, the fixpoint stops once the reachable atoms fill as many words as the dense layout: the
            // dense layout is then not wider (its other conditions aside), which is all the choice needs
            const u64 decided = m_opt == AtomsOption::Auto ? u64{64} * (words_for(L.fluent_count) - 1) + 1 : ~u64{0};
            reach = reachable_fluents(decided);
            C->reachable_fluent = reach.size();
            const bool dense_fits = words_for(L.fluent_count) <= words_for(reach.size()) && frozen_bytes(L.fluent_count) <= kMaxBytes;
            mode = m_opt == AtomsOption::Auto && dense_fits ? AtomMode::Dense : AtomMode::Reachable;
        }
        if (frozen_bytes(mode == AtomMode::Dense ? L.fluent_count : reach.size()) > kMaxBytes)
            throw Error("atom slots need more than 4 GiB of records");
        C->mode = mode;
        C->slot_of.assign(L.fluent_count, kNone);
        if (mode == AtomMode::Dense)
        {
            C->fluent_slots = static_cast<u32>(L.fluent_count);
            C->slot_cid.resize(L.fluent_count);
            for (u64 c = 0; c < L.fluent_count; ++c)
            {
                C->slot_of[c] = static_cast<u32>(c);
                C->slot_cid[c] = c;
            }
        }
        else
        {
            C->fluent_slots = static_cast<u32>(reach.size());
            C->slot_cid = reach;
            for (u32 s = 0; s < reach.size(); ++s)
                C->slot_of[reach[s]] = s;
        }
        C->words = std::max<u32>(1, words_for(C->fluent_slots));
    }

    u32 slot_of_cid(u64 c) const { return c < C->layout.fluent_count ? C->slot_of[c] : kNone; }

    void build_state_tables()
    {
        if (C->mode == AtomMode::Lazy)
        {
            // the initial state's atoms intern first, in the order of its atom list (task.cpp:214-224)
            for (const auto& a : T->fluent_init)
            {
                const u64 c = cid_of(a[0], a.data() + 1);
                if (c >= C->layout.fluent_count)
                    throw Error("an initial atom lies outside the typed-dense domains");
                if (C->slot_of[c] == kNone)
                {
                    C->slot_of[c] = C->fluent_slots++;
                    C->slot_cid.push_back(c);
                }
            }
            C->words = std::max<u32>(1, words_for(C->fluent_slots));
        }
        C->initial.assign(C->words, 0);
        for (const auto& a : T->fluent_init)
        {
            const u32 s = slot_of_cid(cid_of(a[0], a.data() + 1));
            if (s == kNone)
                throw Error("an initial atom has no slot");
            C->initial[s >> 6] |= u64{1} << (s & 63);
        }
        // goal: static literals folded, fluent ones kept by canonical id and resolved to slot lists (a positive atom
        // without a slot holds in no state)
        std::set<std::vector<u32>> pos_atoms;
        for (const Literal& l : T->goal)
        {
            std::vector<u32> objs;
            for (i32 x : l.terms)
                objs.push_back(term_object(x));
            if (T->preds[l.pred].kind == 'S')
            {
                if (static_holds(l.pred, objs.data()) != l.positive)
                    C->goal_fixed_unsat = true;
                continue;
            }
            std::vector<u32> key{l.pred};
            key.insert(key.end(), objs.begin(), objs.end());
            if (l.positive)
                pos_atoms.insert(key);
            const u64 c = cid_of(l.pred, objs.data());
            C->goal_fluent.emplace_back(l.positive, c < C->layout.fluent_count ? c : C->layout.fluent_count);
        }
        for (const Literal& l : T->goal)
            if (!l.positive && T->preds[l.pred].kind != 'S')
            {
                std::vector<u32> key{l.pred};
                for (i32 x : l.terms)
                    key.push_back(term_object(x));
                if (pos_atoms.count(key))
                    C->goal_fixed_unsat = true;
            }
        resolve_goal(*C);
        C->label_width = 0;
        for (const auto& s : T->schemas)
            C->label_width = std::max(C->label_width, s.arity);
    }

    // --------------------------------------------------------------------------------------------- device image
    struct PairKey
    {
        u32 pred, dir;
        bool operator<(const PairKey& o) const { return pred != o.pred ? pred < o.pred : dir < o.dir; }
    };

    u32 pair_of(u32 pred, u32 dir)
    {
        const PairKey k{pred, dir};
        if (auto it = m_pairs.find(k); it != m_pairs.end())
            return it->second;
        const u32 id = static_cast<u32>(m_pair_list.size());
        m_pairs.emplace(k, id);
        m_pair_list.push_back(k);
        return id;
    }

    // object window [lo, hi] of a layout position's domain (empty domain: lo = hi + 1)
    std::pair<u32, u32> position_window(u32 pos) const
    {
        const auto& d = C->layout.domain[pos];
        if (d.empty())
            return {0, 0};
        return {d.front(), d.back() - d.front() + 1};
    }

    // every position of predicate p has a domain that is a contiguous object range (rank = object - first)
    bool pred_contiguous(u32 p) const
    {
        const u32 pb = C->layout.pos_begin[p];
        for (u32 i = 0; i < T->preds[p].arity; ++i)
        {
            const auto& d = C->layout.domain[pb + i];
            if (d.empty() || d.back() - d.front() + 1 != d.size())
                return false;
        }
        return true;
    }

    void build_image()
    {
        const u32 m = static_cast<u32>(T->preds.size());
        const u32 eq = equality_pred();
        (void)eq;
        std::vector<DevSchema> schemas;
        std::vector<DevWitness> witness;  // per schema
        bool any_witness = false;
        std::vector<DevStep> steps;
        std::vector<DevCons> cons;
        std::vector<DevCheck> checks;
        std::vector<DevEffect> effects;
        std::vector<u64> dom0_words;
        // static k-ary relations used by checks
        std::map<u32, u32> static_rel;  // pred -> index
        std::vector<DevStaticMeta> static_meta;
        std::vector<u64> static_key_words;
        auto rel_of = [&](u32 p) -> u32
        {
            if (auto it = static_rel.find(p); it != static_rel.end())
                return it->second;
            const u32 id = static_cast<u32>(static_meta.size());
            DevStaticMeta meta{};
            meta.arity = T->preds[p].arity;
            std::vector<u64> keys(static_keys[p].begin(), static_keys[p].end());
            std::sort(keys.begin(), keys.end());
            meta.keys = static_key_words.size();  // relative; fixed up below
            meta.count = keys.size();
            static_key_words.insert(static_key_words.end(), keys.begin(), keys.end());
            static_meta.push_back(meta);
            static_rel.emplace(p, id);
            return id;
        };

        for (u32 si = 0; si < T->schemas.size(); ++si)
        {
            const SchemaText& s = T->schemas[si];
            DevSchema ds{};
            ds.arity = s.arity;
            ds.never = C->never[si];
            // windows and dom0 (window-aligned)
            std::vector<u32> lo(s.arity, 0), wwords(s.arity, 1), dom_off(s.arity, 0);
            for (u32 v = 0; v < s.arity; ++v)
            {
                const Bits& d = C->dom0[si][v];
                u32 first = kNone, last = 0;
                for (u32 o = 0; o < n; ++o)
                    if (test_bit(d, o))
                    {
                        if (first == kNone)
                            first = o;
                        last = o;
                    }
                if (first == kNone)
                    first = last = 0;
                lo[v] = first;
                wwords[v] = words_for(last - first + 1);
                dom_off[v] = static_cast<u32>(dom0_words.size());
                Bits wbits(wwords[v], 0);
                for (u32 o = first; o <= last && o < n; ++o)
                    if (test_bit(d, o))
                        wbits[(o - first) >> 6] |= u64{1} << ((o - first) & 63);
                dom0_words.insert(dom0_words.end(), wbits.begin(), wbits.end());
            }
            // ground fluent checks
            ds.ground_begin = static_cast<u32>(checks.size());
            for (const Literal& l : s.pre)
                if (distinct_params(l.terms).empty() && T->preds[l.pred].kind == 'F')
                    checks.push_back(make_check(l, rel_of));
            ds.ground_end = static_cast<u32>(checks.size());

            // a step binding `v` after the parameters marked in `bound`
            auto make_step = [&](u32 v, const std::vector<u8>& bound)
            {
                DevStep st{};
                st.param = v;
                st.lo = lo[v];
                st.words = wwords[v];
                st.cons_begin = static_cast<u32>(cons.size());
                cons.push_back(DevCons{static_cast<u32>(ConsKind::Dom0), 0, kNone, 0, dom_off[v], 0});
                st.check_begin = kNone;
                std::vector<DevCheck> mine;
                for (const Literal& l : s.pre)
                {
                    const PredicateText& P = T->preds[l.pred];
                    const auto ps = distinct_params(l.terms);
                    if (std::find(ps.begin(), ps.end(), v) == ps.end())
                        continue;
                    bool rest = true;
                    for (u32 q : ps)
                        if (q != v && !bound[q])
                            rest = false;
                    if (!rest)
                        continue;
                    const bool fluent = P.kind == 'F';
                    if (P.arity == 1)
                    {
                        if (fluent)
                            cons.push_back(DevCons{static_cast<u32>(ConsKind::ViewUnary), l.positive ? 0u : 1u, kNone, 0,
                                                   pair_of(l.pred, 0), 0});
                        continue;  // static unary: in dom0
                    }
                    if (P.arity == 2 && l.terms[0] != l.terms[1])
                    {
                        const u32 vpos = l.terms[0] == static_cast<i32>(v) ? 0 : 1, opos = 1 - vpos;
                        const i32 ot = l.terms[opos];
                        if (ot < 0)
                        {
                            if (fluent)  // the row of the constant: forward if the constant is at position 0
                                cons.push_back(DevCons{static_cast<u32>(ConsKind::ViewRow), l.positive ? 0u : 1u, kNone,
                                                       term_object(ot), pair_of(l.pred, opos == 0 ? 0 : 1), 0});
                            continue;  // static with a constant: in dom0
                        }
                        if (fluent)
                            cons.push_back(DevCons{static_cast<u32>(ConsKind::ViewRow), l.positive ? 0u : 1u,
                                                   static_cast<u32>(ot), 0, pair_of(l.pred, opos == 0 ? 0 : 1), 0});
                        else
                            cons.push_back(DevCons{static_cast<u32>(ConsKind::StaticRow), l.positive ? 0u : 1u,
                                                   static_cast<u32>(ot), 0, static_rows(l.pred, opos, vpos), 0});
                        continue;
                    }
                    mine.push_back(make_check(l, rel_of));
                }
                st.cons_end = static_cast<u32>(cons.size());
                st.check_begin = static_cast<u32>(checks.size());
                checks.insert(checks.end(), mine.begin(), mine.end());
                st.check_end = static_cast<u32>(checks.size());
                return st;
            };

            // plans P_j: parameters [0, j) bound, the rest in greedy order
            for (u32 j = 0; j <= s.arity; ++j)
            {
                ds.plan_begin[j] = static_cast<u32>(steps.size());
                std::vector<u8> bound(s.arity, 0);
                for (u32 v = 0; v < j; ++v)
                    bound[v] = 1;
                for (u32 placed = j; placed < s.arity; ++placed)
                {
                    int best = -1;
                    long best_score = 0;
                    for (u32 v = 0; v < s.arity; ++v)
                    {
                        if (bound[v])
                            continue;
                        long links = 0, un = 0;
                        for (const Literal& l : s.pre)
                        {
                            const auto ps = distinct_params(l.terms);
                            if (std::find(ps.begin(), ps.end(), v) == ps.end())
                                continue;
                            if (T->preds[l.pred].kind == 'F' && ps.size() == 1)
                                ++un;
                            if (ps.size() == 2)
                                for (u32 q : ps)
                                    if (q != v && bound[q])
                                        ++links;
                        }
                        const long score = links * 1000000 + un * 10000 - static_cast<long>(popcount(C->dom0[si][v]));
                        if (best < 0 || score > best_score)
                            best = static_cast<int>(v), best_score = score;
                    }
                    steps.push_back(make_step(static_cast<u32>(best), bound));
                    bound[best] = 1;
                }
            }
            ds.plan_begin[s.arity + 1] = static_cast<u32>(steps.size());
            for (u32 j = s.arity + 2; j < kMaxParams + 2; ++j)
                ds.plan_begin[j] = ds.plan_begin[s.arity + 1];
            // filters F_i
            for (u32 i = 0; i < s.arity; ++i)
            {
                std::vector<u8> bound(s.arity, 0);
                for (u32 v = 0; v < i; ++v)
                    bound[v] = 1;
                ds.filter_step[i] = static_cast<u32>(steps.size());
                steps.push_back(make_step(i, bound));
            }
            // witness pruning: the witnesses in the matcher's order, each one's filter with the effect-relevant
            // parameters and the earlier witnesses bound, and the count plan of the later witnesses
            {
                DevWitness wd{};
                const std::vector<u8> rel = effect_relevant(s);
                const std::vector<u32> wit = witness_order(*C, si, rel);
                wd.n = static_cast<u32>(wit.size());
                std::vector<u8> bound = rel;
                for (u32 t = 0; t < wd.n; ++t)
                {
                    wd.param[t] = wit[t];
                    wd.filter[t] = static_cast<u32>(steps.size());
                    steps.push_back(make_step(wit[t], bound));
                    bound[wit[t]] = 1;
                    std::vector<u8> b2 = bound;
                    wd.plan_lo[t] = static_cast<u32>(steps.size());
                    for (u32 t2 = t + 1; t2 < wd.n; ++t2)
                    {
                        steps.push_back(make_step(wit[t2], b2));
                        b2[wit[t2]] = 1;
                    }
                    wd.plan_hi[t] = static_cast<u32>(steps.size());
                }
                witness.push_back(wd);
                any_witness = any_witness || wd.n > 0;
            }
            // effects: adds first, then deletes
            ds.eff_begin = static_cast<u32>(effects.size());
            for (int pass = 0; pass < 2; ++pass)
                for (const Literal& l : s.eff)
                {
                    if (l.positive != (pass == 0))
                        continue;
                    DevEffect e{};
                    e.pred = l.pred;
                    e.base = C->layout.offset[l.pred];
                    if (l.terms.size() > 4)
                        throw Error("effect literals of arity above 4 are not supported by the device path");
                    for (u32 i = 0; i < l.terms.size(); ++i)
                    {
                        const u32 pos = C->layout.pos_begin[l.pred] + i;
                        if (l.terms[i] < 0)
                            e.base += C->layout.rs[pos][term_object(l.terms[i])];
                        else
                        {
                            e.var_param[e.nvar] = static_cast<u32>(l.terms[i]);
                            e.var_pos[e.nvar] = pos;
                            ++e.nvar;
                        }
                    }
                    effects.push_back(e);
                }
            ds.eff_end = static_cast<u32>(effects.size());
            ds.nadd = 0;
            for (const Literal& l : s.eff)
                ds.nadd += l.positive ? 1 : 0;
            schemas.push_back(ds);
        }
        // which schemas' successor counts an action of schema a can change: an add or delete effect of a that can be an
        // atom of a fluent precondition literal of s (the same predicate, and at every position the two terms can take
        // a common object: a constant, or a parameter's static domain); a schema no action of a can touch keeps its
        // count across the move. With more than 32 schemas every schema counts as changed.
        {
            const u32 S = static_cast<u32>(schemas.size());
            auto dom_of = [&](u32 si, i32 t) {
                Bits b(ow, 0);
                if (t < 0)
                    set_bit(b, term_object(t));
                else
                    b = C->dom0[si][static_cast<u32>(t)];
                return b;
            };
            auto meet = [](const Bits& x, const Bits& y) {
                for (size_t w = 0; w < x.size() && w < y.size(); ++w)
                    if (x[w] & y[w])
                        return true;
                return false;
            };
            for (u32 a = 0; a < S; ++a)
            {
                u32 mask = S > 32 ? ~0u : 0u;
                for (u32 s2 = 0; s2 < S && S <= 32; ++s2)
                {
                    bool hit = false;
                    for (const Literal& e : T->schemas[a].eff)
                        for (const Literal& l : T->schemas[s2].pre)
                        {
                            if (hit || l.pred != e.pred || T->preds[l.pred].kind != 'F' || l.terms.size() != e.terms.size())
                                continue;
                            bool all = true;
                            for (size_t i = 0; i < l.terms.size() && all; ++i)
                                all = meet(dom_of(a, e.terms[i]), dom_of(s2, l.terms[i]));
                            hit = all;
                        }
                    if (hit)
                        mask |= 1u << s2;
                }
                schemas[a].affects = mask;
            }
        }

        // view pairs: windows and offsets
        std::vector<DevPair> pairs;
        u32 view_words = 0;
        for (const PairKey& k : m_pair_list)
        {
            DevPair p{};
            p.pred = k.pred;
            p.dir = k.dir;
            const u32 pb = C->layout.pos_begin[k.pred];
            if (T->preds[k.pred].arity == 1)
            {
                p.src_lo = 0;
                p.src_n = 1;
                const auto [dl, dn] = position_window(pb);
                p.dst_lo = dl;
                p.dst_words = std::max<u32>(1, words_for(dn));
            }
            else
            {
                const u32 spos = pb + (k.dir == 0 ? 0 : 1), dpos = pb + (k.dir == 0 ? 1 : 0);
                const auto [sl, sn] = position_window(spos);
                const auto [dl, dn] = position_window(dpos);
                p.src_lo = sl;
                p.src_n = std::max<u32>(1, sn);
                p.dst_lo = dl;
                p.dst_words = std::max<u32>(1, words_for(dn));
            }
            // forward rows (and unary rows) of a dense predicate over contiguous domains are slices of the state
            if (C->mode == AtomMode::Dense && k.dir == 0 && pred_contiguous(k.pred) && C->layout.size[k.pred] > 0)
            {
                p.bulk = 1;
                p.bit0 = C->layout.offset[k.pred];
                const u32 last = pb + T->preds[k.pred].arity - 1;
                p.row_bits = static_cast<u32>(C->layout.domain[last].size());
            }
            // bulk rows are read from the state itself: only the other pairs take view words
            p.offset = view_words;
            if (!p.bulk)
                view_words += p.src_n * p.dst_words;
            pairs.push_back(p);
        }
        // slot decoding per fluent predicate (ascending offset)
        std::vector<DevPredDecode> decode;
        bool decode_arith = C->mode == AtomMode::Dense;
        for (u32 p = 0; p < m; ++p)
        {
            if (T->preds[p].kind != 'F' || C->layout.size[p] == 0)
                continue;
            DevPredDecode d{};
            d.offset = C->layout.offset[p];
            d.size = C->layout.size[p];
            d.pred = p;
            d.arity = T->preds[p].arity;
            const u32 pb = C->layout.pos_begin[p];
            d.d1 = d.arity >= 2 ? static_cast<u32>(C->layout.domain[pb + 1].size()) : 1;
            d.lo0 = d.arity >= 1 ? C->layout.domain[pb][0] : 0;
            d.lo1 = d.arity >= 2 ? C->layout.domain[pb + 1][0] : 0;
            d.contiguous = pred_contiguous(p) ? 1 : 0;
            if (d.arity > 2 || !d.contiguous)
                decode_arith = false;
            for (const DevPair& q : pairs)
                if (q.pred == p && !q.bulk)
                    d.has_scatter = 1;
            decode.push_back(d);
        }

        // slot records (pred | a0 << 16 | a1 << 32 | a2 << 48) for the view build and the atom listing; lazy slots
        // reserve one per canonical atom
        const bool lazy = C->mode == AtomMode::Lazy;
        std::vector<u64> records(lazy ? C->layout.fluent_count : C->fluent_slots, 0);
        for (u32 s = 0; s < C->fluent_slots; ++s)
            records[s] = atom_record(*C, C->slot_cid[s]);

        // per predicate: its view pairs (unary/forward, backward) for the view build
        std::vector<u64> pred_pairs(m, ~u64{0});
        for (u32 i = 0; i < pairs.size(); ++i)
        {
            u64& e = pred_pairs[pairs[i].pred];
            if (pairs[i].dir == 0)
                e = (e & 0xFFFFFFFF00000000ull) | i;
            else
                e = (e & 0x00000000FFFFFFFFull) | (static_cast<u64>(i) << 32);
        }

        // assemble the image
        std::vector<u64> img;
        auto reserve_words = [&](size_t w)
        {
            const u64 off = img.size();
            img.resize(img.size() + w, 0);
            return off;
        };
        auto put = [&](const void* src, size_t bytes) -> u64
        {
            const u64 off = reserve_words((bytes + 7) / 8);
            if (bytes)
                std::memcpy(img.data() + off, src, bytes);
            return off;
        };
        reserve_words((sizeof(DevTaskHeader) + 7) / 8);
        DevTaskHeader h{};
        h.num_objects = n;
        h.ow = ow;
        h.words = C->words;
        h.fluent_slots = C->fluent_slots;
        h.dense = C->mode == AtomMode::Dense ? 1 : 0;
        h.num_schemas = static_cast<u32>(schemas.size());
        h.label_width = C->label_width;
        h.num_pairs = static_cast<u32>(pairs.size());
        h.view_words = view_words;
        h.num_goal_pos = static_cast<u32>(C->goal_pos.size());
        h.num_goal_neg = static_cast<u32>(C->goal_neg.size());
        h.goal_unsat = C->goal_unsat ? 1 : 0;
        h.fluent_count = C->layout.fluent_count;
        // hot sections first: everything read per state by the step and count kernels
        h.off_schemas = put(schemas.data(), schemas.size() * sizeof(DevSchema));
        h.off_steps = put(steps.data(), steps.size() * sizeof(DevStep));
        h.off_cons = put(cons.data(), cons.size() * sizeof(DevCons));
        h.off_checks = put(checks.data(), checks.size() * sizeof(DevCheck));
        h.off_effects = put(effects.data(), effects.size() * sizeof(DevEffect));
        h.off_pairs = put(pairs.data(), pairs.size() * sizeof(DevPair));
        h.num_decode = static_cast<u32>(decode.size());
        h.decode_arith = decode_arith ? 1 : 0;
        h.off_decode = put(decode.data(), decode.size() * sizeof(DevPredDecode));
        h.off_dom0 = put(dom0_words.data(), dom0_words.size() * sizeof(u64));
        {
            // lazy slots: room for every fluent goal literal (the lists grow as their atoms intern)
            std::vector<u32> gp = C->goal_pos, gn = C->goal_neg;
            if (lazy)
            {
                u32 np = 0, nn = 0;
                for (const auto& [pos, c] : C->goal_fluent)
                    ++(pos ? np : nn);
                gp.resize(np, 0);
                gn.resize(nn, 0);
            }
            h.off_goal_pos = put(gp.data(), gp.size() * sizeof(u32));
            h.off_goal_neg = put(gn.data(), gn.size() * sizeof(u32));
        }
        {
            std::vector<u32> ar(m);
            for (u32 p = 0; p < m; ++p)
                ar[p] = T->preds[p].arity;
            h.off_pred_arity = put(ar.data(), ar.size() * sizeof(u32));
            h.off_pos_begin = put(C->layout.pos_begin.data(), C->layout.pos_begin.size() * sizeof(u32));
        }
        h.off_pred_pairs = put(pred_pairs.data(), pred_pairs.size() * sizeof(u64));
        {
            std::vector<u64> offs(m, 0);
            for (u32 p = 0; p < m; ++p)
                offs[p] = C->layout.offset[p] == kNone64 ? 0 : C->layout.offset[p];
            h.off_pred_offset = put(offs.data(), offs.size() * sizeof(u64));
        }
        h.hot_words = img.size();
        for (const DevStep& st : steps)
            h.max_step_words = std::max(h.max_step_words, st.words);
        // rs tables: per position n entries (u64)
        h.num_positions = static_cast<u32>(C->layout.rs.size());
        h.off_rs = reserve_words(static_cast<size_t>(h.num_positions) * n);
        for (u32 pos = 0; pos < h.num_positions; ++pos)
            std::copy(C->layout.rs[pos].begin(), C->layout.rs[pos].end(), img.begin() + h.off_rs + static_cast<size_t>(pos) * n);
        {
            std::vector<u32> so(C->mode == AtomMode::Dense ? 0 : C->layout.fluent_count);
            for (size_t c = 0; c < so.size(); ++c)
                so[c] = C->slot_of[c];
            h.off_slot_of = put(so.data(), so.size() * sizeof(u32));
        }
        h.off_records = put(records.data(), records.size() * sizeof(u64));
        {
            // static row tables back to back (n * ow words each); DevCons.table holds the table index, the kernel
            // multiplies by n * ow
            h.off_static_rows = img.size();
            for (const auto& t : m_row_data)
                img.insert(img.end(), t.begin(), t.end());
        }
        h.off_static_keys = put(static_key_words.data(), static_key_words.size() * sizeof(u64));
        for (auto& meta : static_meta)
            meta.keys += h.off_static_keys;
        h.off_static_meta = put(static_meta.data(), static_meta.size() * sizeof(DevStaticMeta));
        {
            std::vector<u64> init = C->initial;
            if (lazy)
                init.resize(std::max<u32>(1, words_for(C->layout.fluent_count)), 0);
            h.off_initial = put(init.data(), init.size() * sizeof(u64));
        }
        h.off_witness = any_witness ? put(witness.data(), witness.size() * sizeof(DevWitness)) : 0;
        h.lazy = lazy ? 1 : 0;
        std::memcpy(img.data(), &h, sizeof(h));
        C->image = std::move(img);
    }

    template<class RelOf>
    DevCheck make_check(const Literal& l, RelOf&& rel_of)
    {
        DevCheck c{};
        c.pos = l.positive ? 1 : 0;
        c.nterms = static_cast<u32>(l.terms.size());
        if (c.nterms > 6)
            throw Error("literal arity above 6");
        for (u32 i = 0; i < c.nterms; ++i)
            c.terms[i] = l.terms[i];
        if (T->preds[l.pred].kind == 'F')
        {
            c.kind = static_cast<u32>(CheckKind::Fluent);
            c.pred = l.pred;
        }
        else
        {
            c.kind = static_cast<u32>(CheckKind::Static);
            c.pred = rel_of(l.pred);
        }
        return c;
    }

    AtomsOption m_opt;
    std::unique_ptr<CompiledTask> C;
    const TaskText* T = nullptr;
    u32 n = 0, ow = 1;
    std::vector<std::vector<const std::vector<u32>*>> static_atoms;
    std::vector<std::unordered_set<u64>> static_keys;
    std::vector<Bits> s_unary;
    std::map<std::tuple<u32, u32, u32>, u32> m_row_tables;
    std::vector<Bits> m_row_data;
    std::map<PairKey, u32> m_pairs;
    std::vector<PairKey> m_pair_list;
};
}  // namespace

TaskText parse_task_text(std::string_view text) { return Reader(text).read(); }

bool CompiledTask::static_holds(u32 pred, const u32* objs) const
{
    const u64 k = static_key(objs, text.preds[pred].arity, std::max<u32>(n, 1));
    return std::binary_search(static_keys[pred].begin(), static_keys[pred].end(), k);
}

u32 CompiledTask::slot_of_atom(u32 pred, const u32* objs) const
{
    const u64 c = layout.encode(pred, objs, text.preds[pred].arity);
    return c < layout.fluent_count ? slot_of[c] : kNone;
}

std::vector<u8> effect_relevant(const SchemaText& s)
{
    std::vector<u8> rel(s.arity, 0);
    auto mark = [&](const std::vector<Literal>& ls) {
        for (const Literal& l : ls)
            for (i32 x : l.terms)
                if (x >= 0 && static_cast<u32>(x) < s.arity)
                    rel[static_cast<u32>(x)] = 1;
    };
    mark(s.eff);
    for (const CondEffectText& ce : s.ces)
    {
        mark(ce.cond);
        mark(ce.eff);
    }
    return rel;
}

/// The witness parameters of schema si (those no effect mentions) in the order the reference's successor matcher binds
/// them (src/mymyr/task/compile.cpp:916-946): after every effect-relevant parameter, greedily the one with the most
/// binary constraints to placed parameters, then the most fluent unary constraints, then the fewest dom0 objects, ties
/// to the smallest parameter. The constraints are counted as the matcher builds them with every parameter free
/// (compile.cpp:826-907): a binary per arity-2 literal over two distinct parameters, and per pair i < j of distinct
/// parameters of a positive static literal of arity 3 or more; a fluent unary per arity-1 fluent literal and per
/// arity-2 fluent literal of one parameter and one constant.
std::vector<u32> witness_order(const CompiledTask& task, u32 si, const std::vector<u8>& relevant)
{
    const TaskText& T = task.text;
    const SchemaText& s = T.schemas[si];
    std::vector<std::pair<u32, u32>> bin;
    std::vector<long> unary(s.arity, 0);
    for (const Literal& l : s.pre)
    {
        const PredicateText& P = T.preds[l.pred];
        const bool fluent = P.kind != 'S';
        const auto& t = l.terms;
        if (std::none_of(t.begin(), t.end(), [](i32 x) { return x >= 0; }))
            continue;
        if (P.arity == 1)
        {
            if (fluent)
                ++unary[static_cast<u32>(t[0])];
            continue;
        }
        if (P.arity == 2 && t[0] != t[1])
        {
            if (t[0] >= 0 && t[1] >= 0)
                bin.push_back({static_cast<u32>(t[0]), static_cast<u32>(t[1])});
            else if (fluent)
                ++unary[static_cast<u32>(t[0] >= 0 ? t[0] : t[1])];
            continue;
        }
        if (!fluent && l.positive && P.arity >= 3)
            for (u32 i = 0; i < P.arity; ++i)
                for (u32 j = i + 1; j < P.arity; ++j)
                    if (t[i] >= 0 && t[j] >= 0 && t[i] != t[j])
                        bin.push_back({static_cast<u32>(t[i]), static_cast<u32>(t[j])});
    }
    std::vector<u8> placed(relevant.begin(), relevant.end());
    std::vector<u32> order;
    for (;;)
    {
        int best = -1;
        long best_score = 0;
        for (u32 v = 0; v < s.arity; ++v)
        {
            if (placed[v])
                continue;
            long links = 0;
            for (const auto& [a, b] : bin)
                links += (a == v && placed[b]) || (b == v && placed[a]);
            long pc = 0;
            for (u64 w : task.dom0[si][v])
                pc += std::popcount(w);
            const long score = links * 1000000 + unary[v] * 10000 - pc;
            if (best < 0 || score > best_score)
                best = static_cast<int>(v), best_score = score;
        }
        if (best < 0)
            break;
        placed[static_cast<u32>(best)] = 1;
        order.push_back(static_cast<u32>(best));
    }
    return order;
}

namespace
{
/// The ground instances of schema si's conditional effects for the action with parameters `bind` into g (the
/// reference's collect_literals, include/mymyr/successor/successors.hpp:321-385): per effect, every binding of its
/// forall parameters over their static domains whose static condition literals hold; the fluent condition literals
/// become slots (a positive one without a slot never holds: the instance is dropped; a negative one always holds), the
/// effects slots (an add without a slot belongs to an instance that never fires in a reachable state: dropped; a
/// delete without one changes nothing).
void ground_ces(const CompiledTask& task, u32 si, const std::vector<u32>& bind, GroundActions& g)
{
    const TaskText& T = task.text;
    const SchemaText& s = T.schemas[si];
    for (u32 k = 0; k < s.ces.size(); ++k)
    {
        const CondEffectText& ce = s.ces[k];
        const auto& dom = task.ce_dom0[si][k];
        std::vector<u32> ext(ce.extra, 0);
        auto obj = [&](i32 x) { return x < 0 ? term_object(x) : static_cast<u32>(x) < s.arity ? bind[x] : ext[x - s.arity]; };
        std::function<void(u32)> rec = [&](u32 d) {
            if (d < ce.extra)
            {
                for (u32 o = 0; o < task.n; ++o)
                    if ((dom[d][o >> 6] >> (o & 63)) & 1)
                    {
                        ext[d] = o;
                        rec(d + 1);
                    }
                return;
            }
            std::vector<u32> pos, neg, add, del;
            std::vector<u32> objs;
            for (const Literal& l : ce.cond)
            {
                objs.clear();
                for (i32 x : l.terms)
                    objs.push_back(obj(x));
                if (T.preds[l.pred].kind == 'S')
                {
                    if (task.static_holds(l.pred, objs.data()) != l.positive)
                        return;
                    continue;
                }
                const u32 slot = task.slot_of_atom(l.pred, objs.data());
                if (slot == kNone)
                {
                    if (l.positive)
                        return;
                    continue;
                }
                (l.positive ? pos : neg).push_back(slot);
            }
            for (const Literal& l : ce.eff)
            {
                objs.clear();
                for (i32 x : l.terms)
                    objs.push_back(obj(x));
                const u32 slot = task.slot_of_atom(l.pred, objs.data());
                if (slot == kNone)
                {
                    if (l.positive)
                        return;
                    continue;
                }
                (l.positive ? add : del).push_back(slot);
            }
            if (add.empty() && del.empty())
                return;  // changes nothing where it fires
            if (pos.size() > 255 || neg.size() > 255 || add.size() > 255 || del.size() > 255)
                throw Error("ground conditional effect with more than 255 atoms in one list");
            g.ce_meta.push_back(static_cast<u32>(pos.size()) | static_cast<u32>(neg.size()) << 8 | static_cast<u32>(add.size()) << 16 |
                                static_cast<u32>(del.size()) << 24);
            g.ce_soff.push_back(static_cast<u32>(g.ce_slots.size()));
            for (auto* v : {&pos, &neg, &add, &del})
                g.ce_slots.insert(g.ce_slots.end(), v->begin(), v->end());
            if (g.ce_slots.size() > (u64{1} << 31))
                throw Error("the ground conditional effects hold more than 2^31 atoms");
        };
        rec(0);
    }
}
}  // namespace

GroundActions ground_actions(const CompiledTask& task, bool witness_pruning, u64 limit)
{
    const TaskText& T = task.text;
    GroundActions g;
    g.label_width = task.label_width;
    const u32 eq = [&] {
        for (u32 p = 0; p < T.preds.size(); ++p)
            if (T.preds[p].kind == 'S' && T.preds[p].name == "=" && T.preds[p].arity == 2)
                return p;
        return kNone;
    }();
    (void)eq;  // the successor engine reads "=" as a static relation over its initial atoms, as the reference does
    // (schema, effect-relevant objects) -> members with their witness objects in the matcher's witness order
    std::map<std::vector<u32>, std::vector<std::pair<std::vector<u32>, u32>>> groups;
    for (u32 si = 0; si < T.schemas.size(); ++si)
    {
        const SchemaText& s = T.schemas[si];
        const std::vector<u8> rel = effect_relevant(s);
        std::vector<u32> wit;  // witness parameters in the matcher's order
        if (witness_pruning)
            wit = witness_order(task, si, rel);
        if (task.never[si])
            continue;
        const u32 first_action = static_cast<u32>(g.meta.size());
        // lexicographic enumeration over dom0, static literals checked once their parameters are bound
        std::vector<u32> bind(s.arity, 0);
        std::vector<std::vector<const Literal*>> statics_at(s.arity + 1);
        for (const Literal& l : s.pre)
        {
            if (T.preds[l.pred].kind != 'S')
                continue;
            i32 last = -1;
            for (i32 x : l.terms)
                last = std::max(last, x);
            statics_at[static_cast<u32>(last + 1)].push_back(&l);
        }
        auto lit_objs = [&](const Literal& l) {
            std::vector<u32> o;
            for (i32 x : l.terms)
                o.push_back(x < 0 ? term_object(x) : bind[x]);
            return o;
        };
        auto statics_ok = [&](u32 level) {
            for (const Literal* l : statics_at[level])
            {
                const auto o = lit_objs(*l);
                if (task.static_holds(l->pred, o.data()) != l->positive)
                    return false;
            }
            return true;
        };
        if (!statics_ok(0))
            continue;
        std::function<void(u32)> rec = [&](u32 d) {
            if (d == s.arity)
            {
                std::vector<u32> pos, neg, add, del;
                for (const Literal& l : s.pre)
                {
                    if (T.preds[l.pred].kind == 'S')
                        continue;
                    const auto o = lit_objs(l);
                    const u32 slot = task.slot_of_atom(l.pred, o.data());
                    if (slot == kNone)
                    {
                        if (l.positive)
                            return;  // never applicable
                        continue;
                    }
                    (l.positive ? pos : neg).push_back(slot);
                }
                for (const Literal& l : s.eff)
                {
                    const auto o = lit_objs(l);
                    const u32 slot = task.slot_of_atom(l.pred, o.data());
                    if (slot == kNone)
                    {
                        if (l.positive)
                            throw Error("an add effect of " + s.name + " has no atom slot");
                        continue;
                    }
                    (l.positive ? add : del).push_back(slot);
                }
                if (pos.size() > 255 || neg.size() > 255 || add.size() > 255 || del.size() > 255)
                    throw Error("ground action with more than 255 atoms in one list");
                if (g.meta.size() >= limit)
                    throw Error("more than " + std::to_string(limit) + " ground actions");
                g.meta.push_back(static_cast<u32>(pos.size()) | static_cast<u32>(neg.size()) << 8 | static_cast<u32>(add.size()) << 16 |
                                 static_cast<u32>(del.size()) << 24);
                g.off.push_back(static_cast<u32>(g.slots.size()));
                for (auto* v : {&pos, &neg, &add, &del})
                    g.slots.insert(g.slots.end(), v->begin(), v->end());
                g.schema.push_back(si);
                for (u32 k = 0; k < g.label_width; ++k)
                    g.binding.push_back(k < s.arity ? bind[k] : kNone);
                if (task.has_ce)
                {
                    g.ce_off.push_back(static_cast<u32>(g.ce_meta.size()));
                    ground_ces(task, si, bind, g);
                }
                return;
            }
            const auto& dom = task.dom0[si][d];
            for (u32 o = 0; o < task.n; ++o)
            {
                if (!((dom[o >> 6] >> (o & 63)) & 1))
                    continue;
                bind[d] = o;
                if (statics_ok(d + 1))
                    rec(d + 1);
            }
        };
        rec(0);
        if (!wit.empty())
            for (u32 a = first_action; a < g.meta.size(); ++a)
            {
                const u32* b = g.binding.data() + static_cast<size_t>(a) * g.label_width;
                std::vector<u32> key{si};
                for (u32 v = 0; v < s.arity; ++v)
                    if (rel[v])
                        key.push_back(b[v]);
                std::vector<u32> w;
                for (u32 v : wit)
                    w.push_back(b[v]);
                groups[key].push_back({std::move(w), a});
            }
    }
    if (task.has_ce)
        g.ce_off.push_back(static_cast<u32>(g.ce_meta.size()));
    if (witness_pruning)
    {
        // dominators: the group's members (fixed effect-relevant objects) whose witness objects come first in the
        // matcher's witness order; an action is a successor only if none of them applies (the matcher emits the first
        // witness binding it finds, include/mymyr/successor/detail/engine.hpp:345-356)
        std::vector<std::vector<u32>> doms(g.meta.size());
        for (auto& [key, members] : groups)
        {
            std::sort(members.begin(), members.end());
            for (size_t i = 1; i < members.size(); ++i)
                for (size_t k = 0; k < i; ++k)
                    doms[members[i].second].push_back(members[k].second);
        }
        g.dom_off.assign(g.meta.size() + 1, 0);
        for (u32 a = 0; a < g.meta.size(); ++a)
        {
            g.dom_off[a] = static_cast<u32>(g.dom.size());
            g.dom.insert(g.dom.end(), doms[a].begin(), doms[a].end());
        }
        g.dom_off[g.meta.size()] = static_cast<u32>(g.dom.size());
    }
    return g;
}

std::unique_ptr<CompiledTask> compile_task(TaskText text, AtomsOption atoms) { return Compiler(std::move(text), atoms).run(); }

u64 atom_record(const CompiledTask& C, u64 c)
{
    // the predicate whose canonical block holds c, then its mixed-radix ranks (the last position has stride 1)
    u32 p = kNone;
    for (u32 q = 0; q < C.text.preds.size(); ++q)
        if (C.text.preds[q].kind == 'F' && C.layout.size[q] > 0 && C.layout.offset[q] <= c && c < C.layout.offset[q] + C.layout.size[q])
            p = q;
    if (p == kNone)
        throw std::logic_error("mymyr_amd: canonical atom " + std::to_string(c) + " outside the fluent predicates' blocks");
    u64 rem = c - C.layout.offset[p];
    const u32 ar = C.text.preds[p].arity;
    u32 args[8] = {};
    for (u32 i = ar; i-- > 0;)
    {
        const auto& dom = C.layout.domain[C.layout.pos_begin[p] + i];
        const u64 dsz = std::max<u64>(1, dom.size());
        args[i] = dom[rem % dsz];
        rem /= dsz;
    }
    u64 rec = p;
    for (u32 i = 0; i < ar && i < 3; ++i)
    {
        if (args[i] >= 65536)
            throw Error("objects beyond 65535 are not supported by the device path");
        rec |= static_cast<u64>(args[i]) << (16 * (i + 1));
    }
    return rec;
}

void resolve_goal(CompiledTask& C)
{
    C.goal_pos.clear();
    C.goal_neg.clear();
    C.goal_unsat = C.goal_fixed_unsat;
    for (const auto& [pos, c] : C.goal_fluent)
    {
        const u32 s = c < C.layout.fluent_count ? C.slot_of[c] : kNone;
        if (s == kNone)
        {
            if (pos)
                C.goal_unsat = true;
            continue;
        }
        (pos ? C.goal_pos : C.goal_neg).push_back(s);
    }
}

std::vector<std::pair<u64, u64>> intern_atoms(CompiledTask& C, const std::vector<u64>& cids)
{
    if (C.mode != AtomMode::Lazy)
        throw std::logic_error("mymyr_amd: atoms interned into a task with frozen slots");
    std::vector<std::pair<u64, u64>> ranges;
    DevTaskHeader h;
    std::memcpy(&h, C.image.data(), sizeof(h));
    const u32 first = C.fluent_slots;
    u64 lo = ~u64{0}, hi = 0;
    u32* slot_img = reinterpret_cast<u32*>(C.image.data() + h.off_slot_of);
    for (const u64 c : cids)
    {
        if (c >= C.layout.fluent_count)
            throw std::logic_error("mymyr_amd: an atom outside the typed-dense domains met without a slot");
        if (C.slot_of[c] != kNone)
            continue;
        const u32 s = C.fluent_slots++;
        C.slot_of[c] = s;
        C.slot_cid.push_back(c);
        C.image[h.off_records + s] = atom_record(C, c);
        slot_img[c] = s;
        lo = std::min(lo, c);
        hi = std::max(hi, c);
    }
    if (C.fluent_slots == first)
        return ranges;
    C.words = std::max<u32>(1, words_for(C.fluent_slots));
    C.initial.resize(C.words, 0);
    resolve_goal(C);
    if (!C.goal_pos.empty())
        std::memcpy(reinterpret_cast<u32*>(C.image.data() + h.off_goal_pos), C.goal_pos.data(), C.goal_pos.size() * sizeof(u32));
    if (!C.goal_neg.empty())
        std::memcpy(reinterpret_cast<u32*>(C.image.data() + h.off_goal_neg), C.goal_neg.data(), C.goal_neg.size() * sizeof(u32));
    h.words = C.words;
    h.fluent_slots = C.fluent_slots;
    h.num_goal_pos = static_cast<u32>(C.goal_pos.size());
    h.num_goal_neg = static_cast<u32>(C.goal_neg.size());
    h.goal_unsat = C.goal_unsat ? 1 : 0;
    std::memcpy(C.image.data(), &h, sizeof(h));
    // the header and the goal lists (hot section), the slot table's changed words, the new records
    ranges.emplace_back(0, h.hot_words);
    ranges.emplace_back(h.off_slot_of + lo / 2, h.off_slot_of + hi / 2 + 1);
    ranges.emplace_back(h.off_records + first, h.off_records + C.fluent_slots);
    return ranges;
}
}  // namespace mya
