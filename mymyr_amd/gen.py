"""Seeded synthetic workloads, written as tasks in the reference's text format (src/mymyr/formalism/text_format.cpp):

  gridworld(32, 32, 0.2)            one agent on a grid with blocked cells, lifted move(?from ?to)
  random_strips(512, 4096)          a random ground STRIPS task (nullary fluents and schemas)
  transport(64, 16, 128)            typed transport: load / unload / drive over a random connected road graph
  dedup rows                        counter-based rows with injected exact duplicates (``dedup_rows``)

The random draws are SplitMix64 / Xoshiro256** with Lemire's bounded draw exactly as the reference specifies them
(include/mymyr/core/random.hpp:1-158), so a (generator, seed) pair names one task file everywhere.
"""

from __future__ import annotations

import numpy as np

M64 = (1 << 64) - 1
GAMMA = 0x9E3779B97F4A7C15


def mix64(x: int) -> int:
    x &= M64
    x ^= x >> 30
    x = (x * 0xBF58476D1CE4E5B9) & M64
    x ^= x >> 27
    x = (x * 0x94D049BB133111EB) & M64
    x ^= x >> 31
    return x


class SplitMix64:
    def __init__(self, seed: int = 0):
        self.state = seed & M64

    def next(self) -> int:
        self.state = (self.state + GAMMA) & M64
        return mix64(self.state)


class Xoshiro256:
    """xoshiro256** seeded with the first four SplitMix64 outputs (include/mymyr/core/random.hpp:120-158)."""

    def __init__(self, seed: int = 0):
        sm = SplitMix64(seed)
        self.s = [sm.next() for _ in range(4)]

    @staticmethod
    def _rotl(x: int, k: int) -> int:
        return ((x << k) | (x >> (64 - k))) & M64

    def next(self) -> int:
        s = self.s
        result = (self._rotl((s[1] * 5) & M64, 7) * 9) & M64
        t = (s[1] << 17) & M64
        s[2] ^= s[0]
        s[3] ^= s[1]
        s[1] ^= s[2]
        s[0] ^= s[3]
        s[2] ^= t
        s[3] = self._rotl(s[3], 45)
        return result

    def bounded(self, n: int) -> int:
        """Lemire's multiply-shift with rejection (random.hpp:26-40)."""
        m = self.next() * n
        low = m & M64
        if low < n:
            threshold = ((1 << 64) - n) % n
            while low < threshold:
                m = self.next() * n
                low = m & M64
        return m >> 64

    def uniform(self) -> float:
        return (self.next() >> 11) * (2.0 ** -53)

    def sample(self, n: int, k: int) -> list[int]:
        """k distinct values of [0, n) in draw order (rejection of repeats)."""
        seen: set[int] = set()
        out = []
        while len(out) < k:
            v = self.bounded(n)
            if v not in seen:
                seen.add(v)
                out.append(v)
        return out


def _lit(pred: int, positive: bool, terms: list[int]) -> str:
    return " ".join([str(pred), "1" if positive else "0"] + [str(t) for t in terms])


def _obj(o: int) -> int:
    """Object term encoding of the text format: -(o + 1)."""
    return -(o + 1)


def gridworld(width: int = 32, height: int = 32, blocked: float = 0.2, seed: int = 0) -> str:
    """One agent on a width x height grid; each cell blocked with probability `blocked`; static adj(?a ?b) between
    4-neighbour free cells; fluent at(?c); move(?from ?to) with pre at(?from), adj(?from ?to). Start and goal are
    distinct free cells, the goal reachable from the start (redrawn until it is)."""
    rng = Xoshiro256(seed)
    n = width * height
    free = [rng.uniform() >= blocked for _ in range(n)]
    cells = [c for c in range(n) if free[c]]
    if len(cells) < 2:
        raise ValueError("gridworld: fewer than two free cells")
    adj = []
    nbrs: dict[int, list[int]] = {c: [] for c in cells}
    for c in cells:
        x, y = c % width, c // width
        for dx, dy in ((1, 0), (-1, 0), (0, 1), (0, -1)):
            nx, ny = x + dx, y + dy
            if 0 <= nx < width and 0 <= ny < height and free[ny * width + nx]:
                d = ny * width + nx
                adj.append((c, d))
                nbrs[c].append(d)
    while True:
        s = cells[rng.bounded(len(cells))]
        g = cells[rng.bounded(len(cells))]
        if s == g:
            continue
        seen = {s}
        todo = [s]
        while todo:
            c = todo.pop()
            for d in nbrs[c]:
                if d not in seen:
                    seen.add(d)
                    todo.append(d)
        if g in seen:
            break
    lines = [f"O {n}", "P 2", "S 2 adj", "F 1 at", f"SI {len(adj)}"]
    lines += [f"0 {a} {b}" for a, b in adj]
    lines += ["FI 1", f"1 {s}", "G 1", f"1 1 {g}", "A 1", "move 2", "L 2", _lit(1, True, [0]), _lit(0, True, [0, 1]),
              "E 1", "0", "L 0", "F 2", _lit(1, False, [0]), _lit(1, True, [1])]
    return "\n".join(lines) + "\n"


def witness_task(items: int = 6, places: int = 6, seed: int = 0) -> str:
    """A task whose actions have two witness parameters (parameters no effect mentions) that the successor matcher binds
    in an order other than the parameter order: work(?x ?w1 ?w2) with pre todo(?x), link(?w1 ?w2), tool(?w2), effect
    del todo(?x), add done(?x); the fluent unary tool(?w2) makes the matcher bind ?w2 first. toggle(?t ?u) moves a tool
    along static near(?t ?u); relink(?a ?b ?c) moves a link's end along near. Objects: items [0, items), places
    after. Goal: every item done."""
    rng = Xoshiro256(seed)
    P0 = items
    places_ = list(range(P0, P0 + places))
    near = sorted({(a, b) for a in places_ for b in places_ if a != b and rng.uniform() < 0.4})
    links = sorted({(places_[rng.bounded(places)], places_[rng.bounded(places)]) for _ in range(places)})
    tools = sorted({places_[rng.bounded(places)] for _ in range(2)})
    # predicates: 0 S near, 1 S item, 2 F todo, 3 F done, 4 F tool, 5 F link
    lines = [f"O {items + places}", "P 6", "S 2 near", "S 1 item", "F 1 todo", "F 1 done", "F 1 tool", "F 2 link",
             f"SI {len(near) + items}"]
    lines += [f"0 {a} {b}" for a, b in near] + [f"1 {x}" for x in range(items)]
    lines += [f"FI {items + len(tools) + len(links)}"] + [f"2 {x}" for x in range(items)] + [f"4 {t}" for t in tools]
    lines += [f"5 {a} {b}" for a, b in links]
    lines += [f"G {items}"] + [f"3 1 {x}" for x in range(items)]
    lines += ["A 3"]
    lines += ["work 3", "L 4", _lit(2, True, [0]), _lit(1, True, [0]), _lit(5, True, [1, 2]), _lit(4, True, [2]),
              "E 1", "0", "L 0", "F 2", _lit(2, False, [0]), _lit(3, True, [0])]
    lines += ["toggle 2", "L 2", _lit(4, True, [0]), _lit(0, True, [0, 1]),
              "E 1", "0", "L 0", "F 2", _lit(4, False, [0]), _lit(4, True, [1])]
    lines += ["relink 3", "L 2", _lit(5, True, [0, 1]), _lit(0, True, [1, 2]),
              "E 1", "0", "L 0", "F 2", _lit(5, False, [0, 1]), _lit(5, True, [0, 2])]
    return "\n".join(lines) + "\n"


def random_strips(props: int = 512, actions: int = 4096, init_atoms: int = 64, goal_atoms: int = 8, walk: int = 32,
                  seed: int = 0) -> str:
    """A random ground STRIPS task: `props` nullary fluents, `actions` nullary schemas with 1-4 precondition atoms,
    1-3 add and 1-3 delete atoms (add and delete disjoint); `init_atoms` true initially; the goal is `goal_atoms` atoms
    of the state a seeded random walk of `walk` steps reaches."""
    rng = Xoshiro256(seed)
    acts = []
    for _ in range(actions):
        pre = rng.sample(props, 1 + rng.bounded(4))
        na, nd = 1 + rng.bounded(3), 1 + rng.bounded(3)
        eff = rng.sample(props, na + nd)
        acts.append((pre, eff[:na], eff[na:]))
    init = rng.sample(props, init_atoms)
    state = set(init)
    for _ in range(walk):
        app = [a for a in acts if all(p in state for p in a[0])]
        if not app:
            break
        pre, add, dele = app[rng.bounded(len(app))]
        state -= set(dele)
        state |= set(add)
    true = sorted(state)
    goal = sorted(true[i] for i in rng.sample(len(true), min(goal_atoms, len(true))))
    lines = ["O 0", f"P {props}"] + [f"F 0 p{i}" for i in range(props)]
    lines += ["SI 0", f"FI {len(init)}"] + [str(p) for p in sorted(init)]
    lines += [f"G {len(goal)}"] + [f"{p} 1" for p in goal]
    lines += [f"A {actions}"]
    for k, (pre, add, dele) in enumerate(acts):
        lines += [f"a{k} 0", f"L {len(pre)}"] + [f"{p} 1" for p in pre]
        lines += ["E 1", "0", "L 0", f"F {len(add) + len(dele)}"] + [f"{p} 0" for p in dele] + [f"{p} 1" for p in add]
    return "\n".join(lines) + "\n"


def transport(locations: int = 64, trucks: int = 16, packages: int = 128, goals: int = 32, degree: int = 4,
              seed: int = 0) -> str:
    """Typed transport. Objects: locations [0, L), trucks [L, L + T), packages after. A random spanning tree plus
    random extra roads up to L * degree / 2 undirected roads (static road, both directions); trucks and packages start
    at uniform locations; the goal puts `goals` distinct packages at uniform locations.
    load(?p ?t ?l), unload(?p ?t ?l), drive(?t ?from ?to) with type predicates location / truck / package."""
    rng = Xoshiro256(seed)
    L, T, P = locations, trucks, packages
    n = L + T + P
    edges: set[tuple[int, int]] = set()
    for i in range(1, L):
        j = rng.bounded(i)
        edges.add((min(i, j), max(i, j)))
    target = max(L - 1, L * degree // 2)
    while len(edges) < target:
        a, b = rng.bounded(L), rng.bounded(L)
        if a != b:
            edges.add((min(a, b), max(a, b)))
    roads = sorted({(a, b) for a, b in edges} | {(b, a) for a, b in edges})
    truck_at = [rng.bounded(L) for _ in range(T)]
    pkg_at = [rng.bounded(L) for _ in range(P)]
    goal_pkgs = rng.sample(P, min(goals, P))
    goal = sorted((L + T + p, rng.bounded(L)) for p in goal_pkgs)
    # predicates: 0 location, 1 truck, 2 package, 3 road (static); 4 at, 5 in (fluent)
    lines = [f"O {n}", "P 6", "S 1 location", "S 1 truck", "S 1 package", "S 2 road", "F 2 at", "F 2 in"]
    si = [f"0 {l}" for l in range(L)] + [f"1 {L + t}" for t in range(T)] + [f"2 {L + T + p}" for p in range(P)]
    si += [f"3 {a} {b}" for a, b in roads]
    lines += [f"SI {len(si)}"] + si
    fi = [f"4 {L + t} {truck_at[t]}" for t in range(T)] + [f"4 {L + T + p} {pkg_at[p]}" for p in range(P)]
    lines += [f"FI {len(fi)}"] + fi
    lines += [f"G {len(goal)}"] + [f"4 1 {o} {l}" for o, l in goal]
    lines += ["A 3"]
    # load(?p ?t ?l)
    lines += ["load 3", "L 5", _lit(2, True, [0]), _lit(1, True, [1]), _lit(0, True, [2]), _lit(4, True, [0, 2]),
              _lit(4, True, [1, 2]), "E 1", "0", "L 0", "F 2", _lit(4, False, [0, 2]), _lit(5, True, [0, 1])]
    # unload(?p ?t ?l)
    lines += ["unload 3", "L 5", _lit(2, True, [0]), _lit(1, True, [1]), _lit(0, True, [2]), _lit(5, True, [0, 1]),
              _lit(4, True, [1, 2]), "E 1", "0", "L 0", "F 2", _lit(5, False, [0, 1]), _lit(4, True, [0, 2])]
    # drive(?t ?from ?to)
    lines += ["drive 3", "L 5", _lit(1, True, [0]), _lit(0, True, [1]), _lit(0, True, [2]), _lit(4, True, [0, 1]),
              _lit(3, True, [1, 2]), "E 1", "0", "L 0", "F 2", _lit(4, False, [0, 1]), _lit(4, True, [0, 2])]
    return "\n".join(lines) + "\n"


# ------------------------------------------------------------------------------------------------- dedup rows
# Row i of the dedup stream (seed s): with probability `dup` (i > 0) an exact copy of row src(i) < i, else fresh words
# w_k = mix64(s + (16 i + k + 1) * GAMMA). The HIP generator in the library computes the same function.
DEDUP_DUP_KEY = 0xD1B54A32D192ED03
DEDUP_SRC_KEY = 0x8CB92BA72F3D8DD7


def dedup_rows(start: int, count: int, words: int = 16, seed: int = 0, dup: float = 0.3) -> np.ndarray:
    """Rows [start, start + count) of the dedup stream as a [count, words] uint64 array (numpy, vectorized)."""
    idx = np.arange(start, start + count, dtype=np.uint64)
    src = _resolve_sources(idx, seed, dup)
    k = np.arange(words, dtype=np.uint64)
    with np.errstate(over="ignore"):
        x = np.uint64(seed) + (src[:, None] * np.uint64(16) + k[None, :] + np.uint64(1)) * np.uint64(GAMMA)
    return _mix64_np(x)


def dedup_is_fresh(idx: np.ndarray, seed: int = 0, dup: float = 0.3) -> np.ndarray:
    d, _ = _dup_and_src(np.asarray(idx, dtype=np.uint64), seed, dup)
    return ~d


def _mix64_np(x: np.ndarray) -> np.ndarray:
    x = x.astype(np.uint64, copy=True)
    with np.errstate(over="ignore"):
        x ^= x >> np.uint64(30)
        x *= np.uint64(0xBF58476D1CE4E5B9)
        x ^= x >> np.uint64(27)
        x *= np.uint64(0x94D049BB133111EB)
        x ^= x >> np.uint64(31)
    return x


def _dup_and_src(idx: np.ndarray, seed: int, dup: float):
    with np.errstate(over="ignore"):
        a = _mix64_np(np.uint64(seed ^ DEDUP_DUP_KEY) ^ (idx * np.uint64(GAMMA)))
        b = _mix64_np(np.uint64(seed ^ DEDUP_SRC_KEY) ^ (idx * np.uint64(GAMMA)))
    # dup iff the top 32 bits, as a fraction of 2^32, fall below `dup` (rows > 0 only)
    thr = np.uint64(int(dup * 4294967296.0))
    is_dup = ((a >> np.uint64(32)) < thr) & (idx > 0)
    # src = high32(low32(b) * i) in [0, i) (i < 2^32)
    src = ((b & np.uint64(0xFFFFFFFF)) * idx) >> np.uint64(32)
    return is_dup, src


def _resolve_sources(idx: np.ndarray, seed: int, dup: float) -> np.ndarray:
    """The fresh row each row copies (itself when fresh): duplicates' sources followed until a fresh row, only the rows
    still on a duplicate being drawn again."""
    cur = idx.copy()
    live = np.arange(len(idx))
    while live.size:
        d, s = _dup_and_src(cur[live], seed, dup)
        live = live[d]
        cur[live] = s[d]
    return cur


def dedup_sources(start: int, count: int, seed: int = 0, dup: float = 0.3) -> np.ndarray:
    """For rows [start, start + count) of the dedup stream, the index of the fresh row each one equals (uint64)."""
    return _resolve_sources(np.arange(start, start + count, dtype=np.uint64), seed, dup)
