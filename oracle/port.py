"""Test infrastructure, not product code: a CPU restatement of the reference algorithm of the state-expansion path
(maichmueller/mymyr), written from the reference's semantics in plain Python with numpy for row arithmetic. Only
tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it, to check results; the product never imports it.

Every function cites the reference file:line it restates. How each part is pinned (tests/test_oracle.py):
  hash_words / hash_state / mix64   closed form (include/mymyr/core/hash.hpp:12-60) + the compiled reference
                                    (oracle/_ref) on random rows + golden vectors in tests/golden/hash.json
  philox / successor_index          Random123 known-answer vectors (tests/cpp/rl/test_env.cpp:167-194) + the
                                    compiled reference
  read_task / compile (layout)      slot tables of the compiled reference for 18 suite tasks and the 5 workloads
                                    (tests/golden/slots.json)
  successors                        the compiled reference's canonical successor lists on random-walk states
  env_step                          the compiled reference's HostEnv trajectories (tests/golden/env_*.json)
  brfs                              the reference suite's exhaustive counts (tests/cpp/support/suite.hpp:33-56)
                                    and layer counts / fingerprints of the compiled reference
  dedup unique count                closed form: the number of fresh rows of the generator
  encode_atoms / schema_masks       closed form (ascending set bits; any applicable binding per schema)
Limitation: witness pruning is restated only where it is vacuous (every parameter in some effect); a task with
witness parameters raises NotImplementedError ("parity unpinned" for that case).
"""

from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
M32 = (1 << 32) - 1
HASH_SEED = 0x2D358DCCAA6C78A5
HASH_P1 = 0x8BB84B93962EACC9
HASH_P2 = 0x4B33A62ED433D4A3
OUTSIDE = 1 << 40


# ------------------------------------------------------------------------------------------------- hashing
def mix64(x: int) -> int:
    """splitmix64 finalizer (include/mymyr/core/hash.hpp:12-20)."""
    x &= M64
    x ^= x >> 30
    x = (x * 0xBF58476D1CE4E5B9) & M64
    x ^= x >> 27
    x = (x * 0x94D049BB133111EB) & M64
    x ^= x >> 31
    return x


def mulfold(a: int, b: int) -> int:
    """64x64->128 product folded to 64 bits (hash.hpp:23-31)."""
    r = (a & M64) * (b & M64)
    return (r & M64) ^ (r >> 64)


def hash_words(w, seed: int = HASH_SEED) -> int:
    """Hash of n words (hash.hpp:37-47)."""
    w = [int(x) for x in w]
    n = len(w)
    h = (seed ^ (n * HASH_P1)) & M64
    i = 0
    while i + 1 < n:
        h = mulfold(h ^ w[i] ^ HASH_P1, w[i + 1] ^ HASH_P2)
        i += 2
    if i < n:
        h = mulfold(h ^ w[i] ^ HASH_P1, HASH_P2)
    return mix64(h)


def trimmed(w) -> int:
    """bits::trimmed_size (include/mymyr/core/bitset.hpp:49-55)."""
    n = len(w)
    while n > 0 and int(w[n - 1]) == 0:
        n -= 1
    return n


def hash_state(w) -> int:
    """hash::state_words: hash over the trimmed words (hash.hpp:49-53)."""
    return hash_words(list(w)[: trimmed(w)])


# ------------------------------------------------------------------------------------------------- Philox
def philox4x32_10(c, k0: int, k1: int):
    """Philox-4x32-10 (include/mymyr/rl/rng.hpp:45-57)."""
    c = [x & M32 for x in c]
    k0 &= M32
    k1 &= M32
    for _ in range(10):
        p0 = 0xD2511F53 * c[0]
        p1 = 0xCD9E8D57 * c[2]
        c = [((p1 >> 32) ^ c[1] ^ k0) & M32, p1 & M32, ((p0 >> 32) ^ c[3] ^ k1) & M32, p0 & M32]
        k0 = (k0 + 0x9E3779B9) & M32
        k1 = (k1 + 0xBB67AE85) & M32
    return c


def philox_block(seed: int, env: int, draw: int, purpose: int):
    """rng::block: counter (draw lo, draw hi, env, purpose), key = seed (rng.hpp:59-64)."""
    return philox4x32_10([draw & M32, (draw >> 32) & M32, env & M32, purpose], seed & M32, (seed >> 32) & M32)


def below(x: int, n: int) -> int:
    """high64(x * n) from 32x32 partial products (rng.hpp:73-78)."""
    hi = (x >> 32) * n
    lo = (x & M32) * n
    return ((hi + (lo >> 32)) >> 32) & M32


def successor_index(seed: int, env: int, draw: int, count: int) -> int:
    """rng::successor_index (rng.hpp:80-84)."""
    b = philox_block(seed, env, draw, 0)
    return below(b[0] | (b[1] << 32), count)


# ------------------------------------------------------------------------------------------------- task text
def fmix32(x: int) -> int:
    """MurmurHash3's 32-bit finalizer (rl::rng::fmix32, include/mymyr/rl/rng.hpp:86-92)."""
    x &= M32
    x = ((x ^ (x >> 16)) * 0x85EBCA6B) & M32
    x = ((x ^ (x >> 13)) * 0xC2B2AE35) & M32
    return x ^ (x >> 16)


def instance_draw(seed: int, env: int, reset_count: int, instances: int, thresholds=(), indices=()) -> int:
    """The instance of env's draw number reset_count (rl::rng::instance_draw, include/mymyr/rl/rng.hpp:94-115): uniform
    over `instances` without indices, else indices[k] with k the number of thresholds at most the draw's 32 bits."""
    value = fmix32((seed & M32) ^ fmix32(((seed >> 32) & M32) ^ 0x53414D50))
    bits = fmix32(value ^ fmix32(env & M32) ^ fmix32((reset_count & M32) ^ 0x9E3779B9))
    if len(indices) == 0:
        return (bits * instances) >> 32
    return int(indices[sum(1 for t in thresholds if int(t) <= bits)])


class Task:
    """A classical task read from the text format (src/mymyr/formalism/text_format.cpp:22-197) and compiled to atom
    slots (src/mymyr/task/compile.cpp:803-915, 1363-1455; src/mymyr/task/task.cpp:106-143, 216-232)."""

    def __init__(self, text: str, atoms: str = "auto"):
        self._read(text)
        self._compile(atoms)

    # ---------------------------------------------------------------------------- reader
    def _read(self, text: str) -> None:
        tok = text.split()
        pos = 0

        def word():
            nonlocal pos
            pos += 1
            return tok[pos - 1]

        def num():
            return int(word())

        assert word() == "O"
        self.n = num()
        assert word() == "P"
        self.preds = []  # (kind, arity, name)
        for _ in range(num()):
            k = word()
            a = num()
            nm = word()
            if k not in ("S", "F"):
                raise NotImplementedError("derived predicates")
            self.preds.append((k, a, nm))
        tag = word()
        if tag != "SI":
            raise NotImplementedError("numeric tasks")

        def atoms():
            out = []
            for _ in range(num()):
                p = num()
                out.append((p, tuple(num() for _ in range(self.preds[p][1]))))
            return out

        self.static_init = atoms()
        assert word() == "FI"
        self.fluent_init = atoms()
        assert word() == "G"
        self.goal = []
        for _ in range(num()):
            p = num()
            s = num() != 0
            self.goal.append((p, s, tuple(num() for _ in range(self.preds[p][1]))))
        assert word() == "A"
        self.schemas = []  # (name, arity, pre [(p, pos, terms)], eff [(p, pos, terms)])
        for _ in range(num()):
            name = word()
            ar = num()
            assert word() == "L"
            pre = []
            for _ in range(num()):
                p = num()
                s = num() != 0
                pre.append((p, s, tuple(int(word()) for _ in range(self.preds[p][1]))))
            assert word() == "E"
            eff = []
            for _ in range(num()):
                extra = num()
                assert word() == "L"
                nc = num()
                if extra or nc:
                    raise NotImplementedError("conditional effects")
                assert word() == "F"
                for _ in range(num()):
                    p = num()
                    s = num() != 0
                    eff.append((p, s, tuple(int(word()) for _ in range(self.preds[p][1]))))
            self.schemas.append((name, ar, pre, eff))
        while pos < len(tok):
            t = word()
            if t == "X":
                if num():
                    raise NotImplementedError("axioms")
            elif t == "C":
                for _ in range(num()):
                    num(); num(); num(); int(word())
            elif t == "EG":
                num()
                for _ in range(num()):
                    p = num(); num()
                    for _ in range(self.preds[p][1]):
                        num()
            else:
                raise ValueError("unexpected section " + t)
        self.statics = {}
        for p, args in self.static_init:
            self.statics.setdefault(p, set()).add(args)
        self.label_width = max([s[1] for s in self.schemas] + [0])

    def pred_info(self) -> list:
        """The predicates as (name, arity, kind) in declaration order."""
        return [(nm, a, k) for k, a, nm in self.preds]

    # ---------------------------------------------------------------------------- compile
    def _static(self, p: int, args) -> bool:
        return tuple(args) in self.statics.get(p, ())

    def _dom0(self, s):
        """The matcher's static domain of every parameter (compile.cpp:803-915)."""
        name, ar, pre, eff = s
        dom = [set(range(self.n)) for _ in range(ar)]
        never = False
        for p, pos, terms in pre:
            kind, arity, _ = self.preds[p]
            params = sorted({t for t in terms if t >= 0})
            if not params:
                if kind == "S" and self._static(p, [-(t + 1) for t in terms]) != pos:
                    never = True
                continue
            if arity == 1:
                if kind == "S":
                    sat = {a[0] for a in self.statics.get(p, ())}
                    dom[params[0]] = dom[params[0]] & sat if pos else dom[params[0]] - sat
                continue
            if arity == 2 and terms[0] != terms[1]:
                f0, f1 = terms[0] >= 0, terms[1] >= 0
                if f0 and f1:
                    continue
                fpos = 0 if f0 else 1
                opos = 1 - fpos
                v = terms[fpos]
                c = -(terms[opos] + 1)
                if kind == "S":
                    row = {a[fpos] for a in self.statics.get(p, ()) if a[opos] == c}
                    dom[v] = dom[v] & row if pos else dom[v] - row
                continue
            if kind == "S" and pos and arity >= 3:
                for i in range(arity):
                    if terms[i] >= 0:
                        proj = {a[i] for a in self.statics.get(p, ())
                                if all(terms[j] >= 0 or a[j] == -(terms[j] + 1) for j in range(arity))}
                        dom[terms[i]] &= proj
        if any(not d for d in dom):
            never = True
        return dom, never

    def _compile(self, atoms: str) -> None:
        self.dom0 = []
        self.never = []
        for s in self.schemas:
            d, nv = self._dom0(s)
            self.dom0.append(d)
            self.never.append(nv)
        # canonical layout (compile.cpp:1363-1455)
        pos_dom = {}
        for p, (k, a, _) in enumerate(self.preds):
            if k == "F":
                pos_dom[p] = [set() for _ in range(a)]
        for si, (_, _, _, eff) in enumerate(self.schemas):
            for p, positive, terms in eff:
                if positive:
                    for i, t in enumerate(terms):
                        pos_dom[p][i] |= {-(t + 1)} if t < 0 else self.dom0[si][t]
        for p, args in self.fluent_init:
            for i, o in enumerate(args):
                pos_dom[p][i].add(o)
        self.offset, self.rank, self.stride, self.domain = {}, {}, {}, {}
        running = 0
        for p, (k, a, _) in enumerate(self.preds):
            if k != "F":
                continue
            doms = [sorted(d) for d in pos_dom[p]]
            self.domain[p] = doms
            self.rank[p] = [{o: r for r, o in enumerate(d)} for d in doms]
            st = [0] * a
            acc = 1
            for i in range(a - 1, -1, -1):
                st[i] = acc
                acc *= max(1, len(doms[i]))
            self.stride[p] = st
            size = 1
            for d in doms:
                size *= len(d)
            self.offset[p] = running
            running += size
        self.fluent_count = running
        # atom mode (task.cpp:106-143)
        words_for = lambda x: (x + 63) // 64
        if atoms == "dense":
            self.mode = "dense"
        else:
            reach = sorted(self._reachable())
            self.reachable = reach
            dense_fits = words_for(self.fluent_count) <= words_for(len(reach))
            self.mode = "dense" if atoms == "auto" and dense_fits else "reachable"
        if self.mode == "dense":
            self.slot_cid = list(range(self.fluent_count))
        else:
            self.slot_cid = self.reachable
        self.slot_of = {c: s for s, c in enumerate(self.slot_cid)}
        self.slots = len(self.slot_cid)
        self.words = max(1, words_for(self.slots))
        self.initial = self.row_of([(p, a) for p, a in self.fluent_init])
        self.goal_unsat = False
        self.goal_pos, self.goal_neg = [], []
        posset = set()
        for p, pos, args in self.goal:
            if self.preds[p][0] == "S":
                if self._static(p, args) != pos:
                    self.goal_unsat = True
                continue
            if pos:
                posset.add((p, args))
            s = self.slot(p, args)
            if s is None:
                if pos:
                    self.goal_unsat = True
                continue
            (self.goal_pos if pos else self.goal_neg).append(s)
        for p, pos, args in self.goal:
            if not pos and self.preds[p][0] == "F" and (p, args) in posset:
                self.goal_unsat = True

    def cid(self, p: int, args) -> int | None:
        """CanonicalLayout::encode (include/mymyr/task/atom_index.hpp:89-95); None outside the position domains."""
        c = self.offset[p]
        for i, o in enumerate(args):
            r = self.rank[p][i].get(o)
            if r is None:
                return None
            c += r * self.stride[p][i]
        return c

    def slot(self, p: int, args) -> int | None:
        c = self.cid(p, args)
        return None if c is None else self.slot_of.get(c)

    def record(self, s: int):
        """(predicate, args) of slot s (AtomIndex::record)."""
        c = self.slot_cid[s]
        p = next(q for q in self.offset if self.offset[q] <= c < self.offset[q] + self._size(q))
        rem = c - self.offset[p]
        args = []
        for i, d in enumerate(self.domain[p]):
            args.append(d[rem // self.stride[p][i]])
            rem %= self.stride[p][i]
        return p, tuple(args)

    def _size(self, p: int) -> int:
        s = 1
        for d in self.domain[p]:
            s *= len(d)
        return s

    def row_of(self, atoms, words: int | None = None) -> np.ndarray:
        w = self.words if words is None else words
        row = np.zeros(w, dtype=np.uint64)
        for p, args in atoms:
            s = self.slot(p, args)
            row[s >> 6] |= np.uint64(1 << (s & 63))
        return row

    def true_atoms(self, row) -> list:
        out = []
        for wi, x in enumerate(row):
            x = int(x)
            while x:
                b = (x & -x).bit_length() - 1
                x &= x - 1
                s = wi * 64 + b
                if s < self.slots:
                    out.append(self.record(s))
        return out

    # ---------------------------------------------------------------------------- reachability
    def _reachable(self) -> set:
        """The delete-relaxed fixpoint (include/mymyr/reachability/relaxed_reachability.hpp:3-12): rules per add
        effect, bodies of positive fluent and all static literals, '=' by identity; naive rounds."""
        eq = next((p for p, (k, a, nm) in enumerate(self.preds) if k == "S" and nm == "=" and a == 2), None)
        reached = set()
        for p, args in self.fluent_init:
            c = self.cid(p, args)
            if c is not None:
                reached.add((p, args))
        changed = True
        while changed:
            changed = False
            state = Index(reached)
            for si, (name, ar, pre, eff) in enumerate(self.schemas):
                heads = [e for e in eff if e[1]]
                if not heads:
                    continue
                body = [(p, pos, t) for p, pos, t in pre if not (self.preds[p][0] == "F" and not pos)]
                for b in self._bindings(ar, body, state, eq, dom=self.dom0[si]):
                    for p, _, terms in heads:
                        args = tuple(-(t + 1) if t < 0 else b[t] for t in terms)
                        if self.cid(p, args) is not None and (p, args) not in reached:
                            reached.add((p, args))
                            changed = True
        return {self.cid(p, a) for p, a in reached}

    # ---------------------------------------------------------------------------- bindings
    def _holds(self, p, args, state, eq) -> bool:
        if self.preds[p][0] == "S":
            return args[0] == args[1] if (eq is not None and p == eq) else tuple(args) in self.statics.get(p, ())
        return (p, tuple(args)) in state.atoms

    def _bindings(self, ar, lits, state, eq, dom):
        """Every binding (parameters in index order, so lexicographic) under which all `lits` hold: brute force over
        the parameters' domains, where a positive literal whose other parameters are already bound narrows the
        candidates of its last parameter to the objects that make it true (an index lookup), and every literal is
        checked once its last parameter is bound."""
        b = [0] * ar
        filters = [[] for _ in range(ar)]
        checks = [[] for _ in range(ar)]
        for p, pos, terms in lits:
            ps = [t for t in terms if t >= 0]
            if not ps:
                if self._holds(p, tuple(-(t + 1) for t in terms), state, eq) != pos:
                    return
                continue
            last = max(ps)
            checks[last].append((p, pos, terms))
            if pos and terms.count(last) == 1 and not (eq is not None and p == eq):
                filters[last].append((p, terms.index(last), terms))

        def rec(i):
            if i == ar:
                yield list(b)
                return
            cands = set(dom[i]) if dom is not None else set(range(self.n))
            for p, at, terms in filters[i]:
                key = tuple(-(t + 1) if t < 0 else b[t] for j, t in enumerate(terms) if j != at)
                cands &= state.objects(self, p, at, key)
            for o in sorted(cands):
                b[i] = o
                if all(self._holds(p, tuple(-(t + 1) if t < 0 else b[t] for t in terms), state, eq) == pos
                       for p, pos, terms in checks[i]):
                    yield from rec(i + 1)

        yield from rec(0)


class Index:
    """A set of fluent atoms with per-(predicate, position) lookups; static predicates read the task's atoms."""

    def __init__(self, atoms):
        self.atoms = set(atoms)
        self._idx = {}

    def objects(self, task: Task, p: int, at: int, key) -> set:
        k = (p, at)
        if k not in self._idx:
            d = {}
            src = [(p, a) for a in task.statics.get(p, ())] if task.preds[p][0] == "S" else [x for x in self.atoms if x[0] == p]
            for _, args in src:
                d.setdefault(args[:at] + args[at + 1:], set()).add(args[at])
            self._idx[k] = d
        return self._idx[k].get(key, set())


def successors(task: Task, row, witness: bool = False):
    """Successors in canonical order: schemas in id order, bindings lexicographic over the parameter list; effects as
    delete, then add (include/mymyr/successor/successors.hpp:154-248, 423-451). Returns [(schema, binding, row)]."""
    state = Index(task.true_atoms(row))
    out = []
    for si, (name, ar, pre, eff) in enumerate(task.schemas):
        if task.never[si]:
            continue
        rel = sorted({t for _, _, terms in eff for t in terms if t >= 0})
        if witness and len(rel) < ar - 1:
            raise NotImplementedError("witness pruning with several witness parameters (parity unpinned)")
        seen = set()
        for b in task._bindings(ar, pre, state, None, task.dom0[si]):
            if witness and len(rel) < ar:
                # one witness: the matcher's first witness is the smallest object, which is the lexicographically
                # first binding of the effect-relevant values (engine.hpp:345-356)
                key = tuple(b[v] for v in rel)
                if key in seen:
                    continue
                seen.add(key)
            nxt = np.array(row, dtype=np.uint64, copy=True)
            for p, pos, terms in eff:
                if not pos:
                    s = task.slot(p, tuple(-(t + 1) if t < 0 else b[t] for t in terms))
                    if s is not None:
                        nxt[s >> 6] &= np.uint64(~(1 << (s & 63)) & M64)
            for p, pos, terms in eff:
                if pos:
                    s = task.slot(p, tuple(-(t + 1) if t < 0 else b[t] for t in terms))
                    nxt[s >> 6] |= np.uint64(1 << (s & 63))
            out.append((si, b, nxt))
    return out


def expand(task: Task, rows, capacity: int | None = None, drop_noops: bool = False) -> dict:
    """The flat expansion of rows (rl::expand over one task, expand_impl: src/mymyr/rl/expand.cpp:560-620, the
    no-op filter of DirectSink::compact: 340-377): per state its successors in canonical order, each with its parent,
    schema, binding, goal flag, hash_state, no-op flag (the successor equals the parent) and index (its position in
    the parent's full order). With drop_noops a state keeps its non-no-op successors, or all of them when every one is
    a no-op. generated counts every successor; an overflow with drop_noops (generated > capacity) reports the counts
    before dropping in offsets and total."""
    out = {k: [] for k in ("succ", "parent", "schema", "binding", "goal", "succ_hash", "noop", "index")}
    offsets, per_state = [0], []
    for i, row in enumerate(rows):
        entries = []
        for k, (si, b, nxt) in enumerate(successors(task, row)):
            entries.append((k, si, b, nxt, bool(np.array_equal(nxt, row))))
        per_state.append(len(entries))
        kept = [e for e in entries if not e[4]] if drop_noops else entries
        if drop_noops and not kept:
            kept = entries
        for k, si, b, nxt, noop in kept:
            out["succ"].append(nxt)
            out["parent"].append(i)
            out["schema"].append(si)
            out["binding"].append(list(b))
            out["goal"].append(is_goal(task, nxt))
            out["succ_hash"].append(hash_state(nxt))
            out["noop"].append(noop)
            out["index"].append(k)
        offsets.append(len(out["parent"]))
    generated = sum(per_state)
    total = offsets[-1]
    if drop_noops and capacity is not None and generated > capacity:
        offsets = [0] + list(np.cumsum(per_state))
        total = generated
    out.update(offsets=offsets, generated=generated, total=total)
    return out


def table_expand(tasks: list, rows, task_ids, drop_noops: bool = False) -> dict:
    """rl::expand over a task table (include/mymyr/rl/expand.hpp:5-10, 133-150): row i is a state of instance
    task_ids[i]; its successors are that instance's, in its canonical order, as rows of the batch's width (zeros past
    the instance's words) with bindings padded to the table's label width (-1)."""
    rows = np.asarray(rows, np.uint64)
    W = rows.shape[1]
    L = max(1, max(t.label_width for t in tasks))
    out = {k: [] for k in ("succ", "parent", "schema", "binding", "goal", "succ_hash", "noop", "index")}
    offsets, generated = [0], 0
    for i, row in enumerate(rows):
        t = tasks[int(task_ids[i])]
        x = expand(t, [row[: t.words]], drop_noops=drop_noops)
        generated += x["generated"]
        for j in range(len(x["parent"])):
            succ = np.zeros(W, np.uint64)
            succ[: t.words] = x["succ"][j]
            out["succ"].append(succ)
            out["parent"].append(i)
            out["binding"].append(list(x["binding"][j]) + [-1] * (L - len(x["binding"][j])))
            for k in ("schema", "goal", "succ_hash", "noop", "index"):
                out[k].append(x[k][j])
        offsets.append(len(out["parent"]))
    out["succ"] = np.array(out["succ"], np.uint64).reshape(-1, W)
    out["binding"] = np.array(out["binding"], np.int32).reshape(-1, L)
    out.update(offsets=offsets, generated=generated, total=offsets[-1])
    return out


def pad(flat: dict, rows: int, k: int, words: int | None = None, label_width: int | None = None, capacity: int | None = None) -> dict:
    """rl::pad (src/mymyr/rl/expand.cpp:799-873) of a flat expansion (offsets required) into [rows, k] arrays: slot k of
    row i is flat row j = offsets[i] + k when k < count and j < capacity (index j, mask 1, the flat row's fields, and
    canonical = flat index[j]); other slots hold the padding (-1 for index, schema, binding, canonical; 0 otherwise).
    Overflow: the flat expansion's own, a count above k, or a successor past capacity."""
    off = np.asarray(flat["offsets"], np.int64)
    succ = np.asarray(flat["succ"], np.uint64)
    FW, FL = succ.shape[1], np.asarray(flat["binding"]).shape[1]
    W = FW if words is None else words
    L = FL if label_width is None else label_width
    cap = len(succ) if capacity is None else capacity
    c = off[1:rows + 1] - off[:rows]
    kk = np.arange(k)
    j = off[:rows, None] + kk[None, :]
    listed = kk[None, :] < c[:, None]
    valid = listed & (j < cap)
    flat_over = flat.get("generated", 0) > cap or flat.get("total", 0) > cap or flat.get("words_needed", 0) > FW
    out = {"count": c.astype(np.int32), "index": np.where(valid, j, -1).astype(np.int32), "mask": valid.astype(np.uint8),
           "overflow": bool(flat_over or (c > k).any() or (listed & ~valid).any())}
    jv = j[valid]
    out["succ"] = np.zeros((rows, k, W), np.uint64)
    out["succ"][valid, :FW] = succ[jv]
    out["binding"] = np.full((rows, k, L), -1, np.int32)
    out["binding"][valid, :FL] = np.asarray(flat["binding"], np.int32)[jv]
    for name, fill, dt in (("schema", -1, np.int32), ("goal", 0, np.uint8), ("succ_hash", 0, np.uint64), ("noop", 0, np.uint8),
                           ("index", -1, np.int32)):
        dst = "canonical" if name == "index" else name
        out[dst] = np.full((rows, k), fill, dt)
        if flat.get(name) is not None:
            out[dst][valid] = np.asarray(flat[name], dt)[jv]
    return out


def mask_goal(row, gp, gn) -> bool:
    """The per-env goal test over the words of the masks (mask_goal, src/mymyr/rl/env.cpp:55-61)."""
    row, gp, gn = (np.asarray(x, np.uint64) for x in (row, gp, gn))
    return bool(np.all((row & gp) == gp) and np.all((row & gn) == 0))


def is_goal(task: Task, row) -> bool:
    """Successors::goal_holds over the compiled goal (successors.hpp:129-141)."""
    if task.goal_unsat:
        return False
    bit = lambda s: (int(row[s >> 6]) >> (s & 63)) & 1
    return all(bit(s) for s in task.goal_pos) and not any(bit(s) for s in task.goal_neg)


# ------------------------------------------------------------------------------------------------- env
class Env:
    """HostEnv over one task, index action space (src/mymyr/rl/env.cpp:351-528): per-row state, steps, draws, at_goal."""

    def __init__(self, task: Task, seed=0, max_steps=0, step_reward=0.0, goal_reward=1.0, dead_end_reward=0.0,
                 dead_end="no_successors", dead_end_terminal=True, autoreset=True):
        self.t = task
        self.seed, self.max_steps = seed, max_steps
        self.step_reward = np.float32(step_reward)
        self.goal_reward = np.float32(goal_reward)
        self.dead_end_reward = np.float32(dead_end_reward)
        self.dead_end, self.dead_end_terminal, self.autoreset = dead_end, dead_end_terminal, autoreset
        self.init_count = len(successors(task, task.initial))
        self.init_goal = is_goal(task, task.initial)

    def goal_masks(self, words: int):
        """The task's goal as masks over `words` words (TaskTable::Instance::goal_pos / goal_neg)."""
        gp, gn = np.zeros(words, np.uint64), np.zeros(words, np.uint64)
        for s in self.t.goal_pos:
            gp[s >> 6] |= np.uint64(1 << (s & 63))
        for s in self.t.goal_neg:
            gn[s >> 6] |= np.uint64(1 << (s & 63))
        return gp, gn

    def reset(self, n: int, words: int | None = None, goals: bool = False) -> dict:
        """HostEnv::reset (env.cpp:223-255): every row to the initial state, steps 0, draws 0; with per-env goals the
        task's goal masks in every row (reset_row, env.cpp:179-200)."""
        w = self.t.words if words is None else words
        states = np.zeros((n, w), dtype=np.uint64)
        states[:, : self.t.words] = self.t.initial
        b = {"states": states, "steps": np.zeros(n, np.int32), "draws": np.zeros(n, np.uint64),
             "at_goal": np.full(n, 1 if self.init_goal else 0, np.uint8), "count": np.full(n, self.init_count, np.int32)}
        if goals:
            gp, gn = self.goal_masks(w)
            b["goal_pos"] = np.tile(gp, (n, 1))
            b["goal_neg"] = np.tile(gn, (n, 1))
        return b

    def keep_goals_reset(self, b: dict) -> None:
        """reset(keep_goals=True) of every row: the initial state, the given masks kept, at_goal their test on it."""
        n = b["states"].shape[0]
        W = self.t.words
        b["states"][:] = 0
        b["states"][:, :W] = self.t.initial
        b["steps"][:] = 0
        b["count"][:] = self.init_count
        for i in range(n):
            b["at_goal"][i] = 1 if mask_goal(self.t.initial, b["goal_pos"][i, :W], b["goal_neg"][i, :W]) else 0

    def step(self, b: dict, first_env: int = 0, actions=None) -> dict:
        n = b["states"].shape[0]
        L = max(1, self.t.label_width)
        out = {"reward": np.zeros(n, np.float32), "terminated": np.zeros(n, np.uint8), "truncated": np.zeros(n, np.uint8),
               "count": np.zeros(n, np.int32), "schema": np.full(n, -1, np.int32), "binding": np.full((n, L), -1, np.int32),
               "goal": np.zeros(n, np.uint8), "invalid": np.zeros(n, np.uint8),
               "final_states": np.zeros_like(b["states"])}
        W = self.t.words
        for i in range(n):
            row = b["states"][i, :W].copy()
            already = bool(b["at_goal"][i])
            succ = successors(self.t, row)
            c = len(succ)
            st = "goal" if already else "ok"
            a = 0
            if not already and c == 0:
                st = "stuck"
            elif not already and actions is not None:
                if actions[i] < 0 or actions[i] >= c:
                    st = "invalid"
                else:
                    a = int(actions[i])
            elif not already:
                a = successor_index(self.seed, first_env + i, int(b["draws"][i]), c)
            b["draws"][i] += np.uint64(1)
            if st == "ok":
                out["schema"][i] = succ[a][0]
                for k, o in enumerate(succ[a][1]):
                    out["binding"][i, k] = o
            out["invalid"][i] = 1 if st == "invalid" else 0
            s2 = succ[a][2] if st == "ok" else row
            g = already
            c2 = c
            if st == "ok":
                g = (mask_goal(s2, b["goal_pos"][i, :W], b["goal_neg"][i, :W]) if "goal_pos" in b else is_goal(self.t, s2))
                c2 = len(successors(self.t, s2))
            dead = self.dead_end == "no_successors" and not g and ((st == "ok" and c2 == 0) or st == "stuck")
            term = g or (dead and self.dead_end_terminal)
            absorbed = already or (st == "stuck" and dead and self.dead_end_terminal)
            t2 = int(b["steps"][i]) + (0 if absorbed else 1)
            trunc = (not term) and self.max_steps and t2 >= self.max_steps
            if absorbed:
                r = np.float32(0.0)
            else:
                r = np.float32(self.step_reward + (self.goal_reward if g else np.float32(0.0)))
                r = np.float32(r + (self.dead_end_reward if dead else np.float32(0.0)))
            out["reward"][i] = r
            out["terminated"][i] = 1 if term else 0
            out["truncated"][i] = 1 if trunc else 0
            out["goal"][i] = 1 if g else 0
            out["final_states"][i, :W] = s2
            if self.autoreset and (term or trunc):
                b["states"][i, :] = 0
                b["states"][i, :W] = self.t.initial
                b["steps"][i] = 0
                b["at_goal"][i] = 1 if self.init_goal else 0
                if "goal_pos" in b:  # an autoreset writes the task's goal (reset_row with keep_goals off)
                    gp, gn = self.goal_masks(b["goal_pos"].shape[1])
                    b["goal_pos"][i], b["goal_neg"][i] = gp, gn
                out["count"][i] = self.init_count
                continue
            b["at_goal"][i] = 1 if g else 0
            b["states"][i, :W] = s2
            b["steps"][i] = t2
            out["count"][i] = c2
        return out


class TableEnv:
    """HostEnv over a task table: several instances of one domain, each row in the instance task_ids[i] names
    (TaskTable, include/mymyr/rl/task_table.hpp:1-28; src/mymyr/rl/env.cpp:179-255, 351-528). Rows are `words` wide
    (at least the widest instance); a row's words past its own instance's are padding that a step neither reads nor
    writes, and a reset zeroes only what it may have dirtied (TaskSuite::initial_row, src/mymyr/rl/task_suite.cpp:130-138)."""

    def __init__(self, tasks: list, seed=0, max_steps=0, step_reward=0.0, goal_reward=1.0, dead_end_reward=0.0,
                 dead_end="no_successors", dead_end_terminal=True, autoreset=True, sampler=None, suite=False):
        """sampler: (instances, thresholds, indices) of an instance sampler (rl/sampling.hpp; empty arrays: uniform).
        suite: instances of several domains (TaskSuite::group, include/mymyr/rl/task_suite.hpp:62-64): no domain check;
        each row steps in its own instance's domain."""
        if not tasks:
            raise ValueError("mymyr: TaskTable: no instances")
        for i, t in enumerate([] if suite else tasks[1:], 1):
            why = domain_mismatch(tasks[0], t)
            if why:
                raise ValueError(f"mymyr: TaskTable: instance {i} is not of the domain of instance 0: {why}")
        self.envs = [Env(t, seed, max_steps, step_reward, goal_reward, dead_end_reward, dead_end, dead_end_terminal, autoreset)
                     for t in tasks]
        self.tasks = tasks
        self.words = max(t.words for t in tasks)
        self.label_width = max(1, max(t.label_width for t in tasks))
        e = self.envs[0]
        self.seed, self.max_steps, self.autoreset = seed, max_steps, autoreset
        self.step_reward, self.goal_reward, self.dead_end_reward = e.step_reward, e.goal_reward, e.dead_end_reward
        self.dead_end, self.dead_end_terminal = dead_end, dead_end_terminal
        self.sampler = sampler
        if sampler is not None:
            n, thr, idx = sampler
            if n != len(tasks):
                raise ValueError(f"mymyr: env: a sampler over {n} instances for {len(tasks)}")

    def sample_row(self, b: dict, i: int) -> int:
        """Row i's next sampled instance (HostEnv::sample_row, include/mymyr/rl/env.hpp:255-260)."""
        n, thr, idx = self.sampler
        key = int(b["sampling_seeds"][i]) if "sampling_seeds" in b else self.seed
        env = int(b["env_ids"][i]) if "env_ids" in b else b.get("first_env", 0) + i
        return instance_draw(key, env, int(b["reset_counts"][i]), n, thr, idx)

    def _check_ids(self, ids) -> None:
        bad = [(r, int(x)) for r, x in enumerate(ids) if x < 0 or x >= len(self.tasks)]
        if bad:
            r, x = bad[0]
            raise ValueError(f"mymyr: task id {x} of row {r} is outside the table's {len(self.tasks)} instances")

    def _reset_row(self, b: dict, i: int, inst: int, keep_goals: bool, dirty: int) -> None:
        """reset_row (env.cpp:179-205) with TaskSuite::initial_row: the instance's initial state in its own words,
        zeros up to the words the row may have dirtied."""
        t = self.tasks[inst]
        W = b["states"].shape[1]
        w = t.words
        z = min(W, max(w, dirty))
        b["states"][i, :w] = t.initial
        b["states"][i, w:z] = 0
        b["task_ids"][i] = inst
        b["steps"][i] = 0
        if "goal_pos" in b and not keep_goals:
            gp, gn = self.envs[inst].goal_masks(w)
            b["goal_pos"][i, :w], b["goal_neg"][i, :w] = gp, gn
            b["goal_pos"][i, w:z] = 0
            b["goal_neg"][i, w:z] = 0
        if b.get("visited") is not None:
            b["visited_count"][i] = visited_restart(b["visited"][i], hash_state(t.initial))

    def clear_visited(self, b: dict, mask=None) -> None:
        """HostEnv::clear_visited (env.cpp:207-221): the masked rows' tables hold their current states' keys only."""
        for i in range(b["states"].shape[0]):
            if mask is None or mask[i]:
                t = self.tasks[int(b["task_ids"][i])]
                b["visited_count"][i] = visited_restart(b["visited"][i], hash_state(b["states"][i, : t.words]))

    def _goal_row(self, b: dict, i: int) -> bool:
        t = self.tasks[int(b["task_ids"][i])]
        w = min(b["states"].shape[1], t.words)
        if "goal_pos" in b:
            return mask_goal(b["states"][i, :w], b["goal_pos"][i, :w], b["goal_neg"][i, :w])
        return is_goal(t, b["states"][i, :w])

    def reset(self, b: dict, mask=None, keep_goals: bool = False, sample: bool = False, first_env: int = 0) -> None:
        """HostEnv::reset (env.cpp:223-255) of the rows with mask[i] != 0 into their instances task_ids[i] (with
        `sample`, first drawn from the sampler): count receives the initial states' successor counts; with keep_goals
        the rows' goal masks stay (checked against the instance's fluent slots) and at_goal is their test on the
        initial state; reset counters advance for every reset row."""
        n = b["states"].shape[0]
        if sample and self.sampler is None:
            raise ValueError("mymyr: env: a sampling reset needs an instance sampler")
        if sample and n and "reset_counts" not in b:
            raise ValueError("mymyr: env: a sampling reset needs the reset counters")
        if sample:
            for i in range(n):
                if mask is None or mask[i]:
                    b["task_ids"][i] = self.sample_row(dict(b, first_env=first_env), i)
        self._check_ids(b["task_ids"])
        if keep_goals and "goal_pos" in b:
            for i in range(n):
                if mask is None or mask[i]:
                    t = self.tasks[int(b["task_ids"][i])]
                    if not goal_masks_fit(b["goal_pos"][i], b["goal_neg"][i], t.slots):
                        raise ValueError(f"mymyr: env: goal masks in row {i} set fluent slots its instance does not have; "
                                         "supply goals for the written instance")
        W = b["states"].shape[1]
        for i in range(n):
            if mask is not None and not mask[i]:
                continue
            inst = int(b["task_ids"][i])
            self._reset_row(b, i, inst, keep_goals, W)
            if "reset_counts" in b:
                b["reset_counts"][i] += np.uint32(1)
            b["count"][i] = self.envs[inst].init_count
            b["at_goal"][i] = 1 if (self._goal_row(b, i) if "goal_pos" in b else self.envs[inst].init_goal) else 0

    def step(self, b: dict, first_env: int = 0, actions=None, next_task_ids=None, final_words: int | None = None) -> dict:
        """HostEnv::step (env.cpp:351-528) of every row in its own instance; an autoreset restarts a row in
        next_task_ids[i] when given, else in its instance."""
        n, W = b["states"].shape
        self._check_ids(b["task_ids"])
        if next_task_ids is not None:
            self._check_ids(next_task_ids)
        L = self.label_width
        FW = W if final_words is None else final_words
        out = {"reward": np.zeros(n, np.float32), "terminated": np.zeros(n, np.uint8), "truncated": np.zeros(n, np.uint8),
               "count": np.zeros(n, np.int32), "schema": np.full(n, -1, np.int32), "binding": np.full((n, L), -1, np.int32),
               "goal": np.zeros(n, np.uint8), "invalid": np.zeros(n, np.uint8),
               "final_states": np.zeros((n, FW), np.uint64), "revisited": np.zeros(n, np.uint8)}
        goals = "goal_pos" in b
        for i in range(n):
            inst = int(b["task_ids"][i])
            t = self.tasks[inst]
            w = min(W, t.words)
            row = b["states"][i, :w].copy()
            already = bool(b["at_goal"][i])
            succ = successors(t, row)
            c = len(succ)
            st = "goal" if already else "ok"
            a = 0
            if not already and c == 0:
                st = "stuck"
            elif not already and actions is not None:
                if actions[i] < 0 or actions[i] >= c:
                    st = "invalid"
                else:
                    a = int(actions[i])
            elif not already:
                key = int(b["seeds"][i]) if "seeds" in b else self.seed
                env = int(b["env_ids"][i]) if "env_ids" in b else first_env + i
                a = successor_index(key, env, int(b["draws"][i]), c)
            b["draws"][i] += np.uint64(1)
            if st == "ok":
                out["schema"][i] = succ[a][0]
                for k, o in enumerate(succ[a][1]):
                    out["binding"][i, k] = o
            out["invalid"][i] = 1 if st == "invalid" else 0
            s2 = succ[a][2] if st == "ok" else row
            g, c2 = already, c
            if st == "ok":
                g = mask_goal(s2, b["goal_pos"][i, :w], b["goal_neg"][i, :w]) if goals else is_goal(t, s2)
                c2 = len(successors(t, s2))
            dead = self.dead_end == "no_successors" and not g and ((st == "ok" and c2 == 0) or st == "stuck")
            term = g or (dead and self.dead_end_terminal)
            absorbed = already or (st == "stuck" and dead and self.dead_end_terminal)
            t2 = int(b["steps"][i]) + (0 if absorbed else 1)
            trunc = (not term) and self.max_steps and t2 >= self.max_steps
            if absorbed:
                r = np.float32(0.0)
            else:
                r = np.float32(self.step_reward + (self.goal_reward if g else np.float32(0.0)))
                r = np.float32(r + (self.dead_end_reward if dead else np.float32(0.0)))
            out["reward"][i] = r
            out["terminated"][i] = 1 if term else 0
            out["truncated"][i] = 1 if trunc else 0
            out["goal"][i] = 1 if g else 0
            out["final_states"][i, :w] = s2
            if b.get("visited") is not None:
                # the reached state's key (env.cpp:487-499), unless the episode is over without autoreset
                over = (not self.autoreset) and (absorbed or (self.max_steps and int(b["steps"][i]) >= self.max_steps))
                rv = False
                if not over:
                    rv, b["visited_count"][i] = visited_insert(b["visited"][i], int(b["visited_count"][i]), hash_state(s2))
                    if b["visited_count"][i] == b["visited"].shape[1]:
                        b["visited_status"][0] |= 1
                out["revisited"][i] = 1 if rv else 0
            if self.autoreset and (term or trunc):
                if next_task_ids is not None:
                    nxt = int(next_task_ids[i])
                elif "reset_counts" in b and self.sampler is not None:
                    nxt = self.sample_row(dict(b, first_env=first_env), i)
                else:
                    nxt = inst
                if "reset_counts" in b:
                    b["reset_counts"][i] += np.uint32(1)
                self._reset_row(b, i, nxt, False, w)
                out["count"][i] = self.envs[nxt].init_count
                b["at_goal"][i] = 1 if (self._goal_row(b, i) if goals else self.envs[nxt].init_goal) else 0
                continue
            b["at_goal"][i] = 1 if g else 0
            b["states"][i, :w] = s2
            b["steps"][i] = t2
            out["count"][i] = c2
        return out


VISITED_ZERO = 0x9E3779B97F4A7C15


def visited_insert(table, count: int, h: int) -> tuple[bool, int]:
    """The visited table's insert (include/mymyr/rl/visited.hpp:31-52): linear probing over H slots from key & (H - 1),
    key = the hash (0 maps to a reserved key); a new key above floor(3H/4) entries is skipped and the count saturates
    at H. Returns (whether the key was present, the new count); writes `table` in place."""
    H = len(table)
    key = h if h else VISITED_ZERO
    at = key & (H - 1)
    for _ in range(H):
        if int(table[at]) == key:
            return True, count
        if int(table[at]) == 0:
            if count >= (H * 3) // 4:
                return False, H
            table[at] = np.uint64(key)
            return False, count + 1
        at = (at + 1) & (H - 1)
    return False, H


def visited_restart(table, h: int) -> int:
    """visited_clear then visited_insert of one hash (visited.hpp:55-61): returns the count, 1."""
    table[:] = 0
    _, c = visited_insert(table, 0, h)
    return c


def visited_contains(table, count: int, h: int) -> bool:
    """visited_contains (include/mymyr/rl/visited.hpp:12-28): an empty table (count 0) holds nothing; otherwise probe
    from key & (H - 1) until the key or an empty slot, at most H slots."""
    if not count:
        return False
    H = len(table)
    key = h if h else VISITED_ZERO
    at = key & (H - 1)
    for _ in range(H):
        if int(table[at]) == key:
            return True
        if int(table[at]) == 0:
            return False
        at = (at + 1) & (H - 1)
    return False


def visited_mask(table, count, succ_hash, parent, rows=None) -> np.ndarray:
    """rl::visited_mask (include/mymyr/rl/visited.hpp:63-74): out[j] = succ_hash[j] is in the table of row parent[j]
    (or rows[parent[j]]); -1 is padding. Parents or mapped rows outside the tables read as not visited (the device
    contract of the reference's launch_visited_mask, include/mymyr/cuda/rl_ops.hpp:53-58)."""
    table = np.asarray(table, np.uint64)
    n = len(table)
    out = np.zeros(len(succ_hash), np.uint8)
    for j, (h, p) in enumerate(zip(np.asarray(succ_hash, np.uint64), np.asarray(parent, np.int64))):
        if p < 0 or (rows is not None and p >= len(rows)) or (rows is None and p >= n):
            continue
        row = int(rows[p]) if rows is not None else int(p)
        if 0 <= row < n:
            out[j] = visited_contains(table[row], int(count[row]), int(h))
    return out


def goal_masks_fit(gp, gn, fluent_slots: int) -> bool:
    """Whether goal masks set no bit at or past fluent_slots (rl::goal_masks_fit, include/mymyr/rl/goal_masks.hpp:8-21)."""
    for wi, (p, q) in enumerate(zip(np.asarray(gp, np.uint64), np.asarray(gn, np.uint64))):
        x = int(p) | int(q)
        lo = 64 * wi
        if x and (x.bit_length() - 1 + lo) >= fluent_slots:
            return False
    return True


def domain_mismatch(ref: Task, task: Task) -> str:
    """Empty if `task` is of the domain of `ref`: the same action schemas (names, arities) and predicates (names,
    arities, kinds) in the same order (TaskTable::domain_mismatch, src/mymyr/rl/task_table.cpp:75-100; text tasks
    have no problem-local predicates)."""
    if len(task.schemas) != len(ref.schemas):
        return f"{len(task.schemas)} action schemas, instance 0 has {len(ref.schemas)}"
    for s, (a, b) in enumerate(zip(task.schemas, ref.schemas)):
        if a[0] != b[0] or a[1] != b[1]:
            return f"action schema {s} is {a[0]}/{a[1]}, instance 0 has {b[0]}/{b[1]}"
    kinds = {"S": "static", "F": "fluent", "D": "derived"}
    rp, dp = ref.pred_info(), task.pred_info()
    for d, (name, ar, kind) in enumerate(dp):
        if d >= len(rp) or rp[d] != (name, ar, kind):
            have = f"{rp[d][0]}/{rp[d][1]} ({kinds[rp[d][2]]})" if d < len(rp) else "no more"
            return f"domain predicate {d} is {name}/{ar} ({kinds[kind]}), instance 0 has {have}"
    if len(dp) != len(rp):
        return f"{len(dp)} domain predicates, instance 0 has {len(rp)}"
    return ""


# ------------------------------------------------------------------------------------------------- BrFS
def brfs(task: Task, max_depth=None, max_states=None, max_expanded=None, stop_at_goal=True, fingerprint=True) -> dict:
    """run_flat (src/mymyr/search/brfs.cpp:274-404) with Control::finish (brfs.cpp:194-203): ids by first discovery,
    layer_counts {expanded, generated, new}, fingerprint = XOR mix64(id * phi ^ canonical_hash) (brfs.cpp:34-37,
    task.cpp:387-404)."""
    INF = float("inf")
    md = INF if max_depth is None else max_depth
    ms = INF if max_states is None else max_states
    me = INF if max_expanded is None else max_expanded
    rows = [task.initial.copy()]
    ids = {task.initial.tobytes(): 0}
    expanded = generated = goals = 0
    layers = 0
    layer_end = 0
    pos = 0
    first_goal = None
    lc = []
    cur = None
    stopped_budget = False
    full = False
    while pos < len(rows) and len(rows) < ms:
        if expanded >= me:
            stopped_budget = True
            break
        if pos == layer_end:
            if cur is not None:
                lc.append([expanded - cur[0], generated - cur[1], len(rows) - cur[2]])
                cur = None
            if layers == md:
                break
            layers += 1
            layer_end = len(rows)
            cur = (expanded, generated, len(rows))
        row = rows[pos]
        g = is_goal(task, row)
        goals += g
        if g and first_goal is None:
            first_goal = pos
        if g and stop_at_goal:
            break
        expanded += 1
        for _, _, nxt in successors(task, row, witness=True):
            generated += 1
            key = nxt.tobytes()
            if key not in ids:
                ids[key] = len(rows)
                rows.append(nxt)
                if len(rows) >= ms:
                    full = True
                    break
        if full:
            break
        pos += 1
    if cur is not None:
        lc.append([expanded - cur[0], generated - cur[1], len(rows) - cur[2]])
    exhausted = pos == len(rows)
    fp = 0
    if fingerprint:
        for i, r in enumerate(rows):
            fp ^= mix64((i * 0x9E3779B97F4A7C15 & M64) ^ canonical_hash(task, r))
    solved = first_goal is not None
    status = 0 if solved else (2 if stopped_budget else (1 if exhausted or layers >= md else 2))
    return {"states": len(rows), "expanded": expanded, "generated": generated, "goal_states": goals, "layers": layers,
            "layer_counts": lc, "exhausted": exhausted, "solved": solved, "status": status, "fingerprint": fp}


def canonical_hash(task: Task, row) -> int:
    """Task::canonical_hash (src/mymyr/task/task.cpp:387-404), classical part."""
    x = 0
    for wi, w in enumerate(row):
        w = int(w)
        while w:
            b = (w & -w).bit_length() - 1
            w &= w - 1
            x ^= mix64(task.slot_cid[wi * 64 + b] + 0x1234567)
    return x


# ------------------------------------------------------------------------------------------------- encoding
def encode_atoms(row, max_atoms: int) -> np.ndarray:
    """Ascending slot indices of the set bits (State::slots, include/mymyr/state/state.hpp:96-101), -1 padded
    (the padded-array convention, include/mymyr/rl/task_arrays.hpp:4-8)."""
    out = np.full(max_atoms, -1, np.int32)
    k = 0
    for wi, w in enumerate(row):
        w = int(w)
        while w and k < max_atoms:
            b = (w & -w).bit_length() - 1
            w &= w - 1
            out[k] = wi * 64 + b
            k += 1
    return out


def schema_masks(task: Task, row) -> np.ndarray:
    """Per schema, whether some binding is applicable (rl::schema_masks, include/mymyr/rl/masks.hpp:9-11)."""
    m = np.zeros(len(task.schemas), np.uint8)
    for si, _, _ in successors(task, row):
        m[si] = 1
    return m


def dedup_unique(rows: np.ndarray) -> tuple[int, np.ndarray]:
    """Unique count and first-occurrence ids of rows inserted in order (FlatStateStore::insert ids,
    include/mymyr/state/flat_store.hpp:73-115)."""
    seen = {}
    ids = np.zeros(rows.shape[0], np.int64)
    for i in range(rows.shape[0]):
        k = rows[i, : trimmed(rows[i])].tobytes()
        ids[i] = seen.setdefault(k, len(seen))
    return len(seen), ids
