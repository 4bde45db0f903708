"""``search.brfs`` on the device: the drop-in for the reference's ``mymyr.search.brfs`` / ``mymyr.cuda.brfs``
(python/src/search_bindings.cpp:3348, python/src/cuda_bindings.cpp:2716; C++ brfs(), include/mymyr/search/brfs.hpp:140).
"""

from __future__ import annotations

import ctypes
import enum
from dataclasses import dataclass, field
from typing import NamedTuple

import numpy as np

from . import _lib
from ._lib import check, lib
from .task import Task

STATUS = {0: "solved", 1: "exhausted", 2: "out_of_states", 3: "out_of_time", 4: "cancelled", 5: "failed", 6: "unsolvable"}


class Status(str, enum.Enum):
    """The reference's mymyr.search.Status (search::SearchStatus, python/src/search_bindings.cpp:2240-2248): its members
    are the strings a result's status holds, so `result.status == Status.EXHAUSTED` reads as with the reference."""

    SOLVED = "solved"
    EXHAUSTED = "exhausted"
    OUT_OF_STATES = "out_of_states"
    OUT_OF_TIME = "out_of_time"
    CANCELLED = "cancelled"
    FAILED = "failed"
    UNSOLVABLE = "unsolvable"

    def __str__(self) -> str:
        return self.value
UNBOUNDED32 = 0xFFFFFFFF
UNBOUNDED64 = (1 << 64) - 1


class Action(NamedTuple):
    """An action label (include/mymyr/successor/action.hpp:27-44): the schema and the objects of its full parameter list."""

    schema: int
    binding: tuple


@dataclass
class Statistics:
    """search::SearchStatistics (include/mymyr/search/control.hpp:129-139) as the observer's events carry it."""

    expanded: int = 0
    generated: int = 0
    states: int = 0
    pruned: int = 0
    seconds: float = 0.0
    memory_bytes: int = 0


def _default_event(fn):
    # an event a subclass does not override carries this attribute and is not installed (python/mymyr/search/
    # _observer.py:17-20)
    fn._mymyr_default_event = True
    return fn


class Observer:
    """Base class of search observers (the reference's mymyr.search.Observer, python/mymyr/search/_observer.py:23-120):
    pass an instance (or any object with some of these methods) as ``observer=`` to :func:`brfs` and override the
    events of interest; events a subclass does not override are never called. The device search sends ``on_start``,
    ``on_expand`` per expanded state, ``on_generate`` per successor (``on_prune`` after it for a blocked one), ``on_pass``
    after every layer, ``on_progress`` at its batch boundaries once ``progress_interval`` more states were expanded,
    ``on_solution`` and ``on_end``, all on the calling thread and in the reference's order; the per-state events come a
    device batch at a time (with any of them defined, each batch's parents, transitions and successor rows are brought
    to the host). A BrFS sends no ``on_transition``, as the reference's. The first exception an event raises stops the
    search (status "cancelled") at the next batch and is raised when the search returns."""

    @_default_event
    def on_start(self, state: np.ndarray) -> None:
        """The search starts from ``state`` (its words)."""

    @_default_event
    def on_expand(self, id: int, state: np.ndarray) -> None:
        """State ``id`` is expanded."""

    @_default_event
    def on_generate(self, parent: int, action: Action, child, state: np.ndarray, is_new: bool) -> None:
        """``action`` leads from ``parent`` to ``state``; ``child`` is its id (None for a blocked successor); ``is_new``:
        the state was entered by this transition."""

    @_default_event
    def on_prune(self, parent: int, action: Action, state: np.ndarray) -> None:
        """The successor ``state`` of ``parent`` is not entered (a blocked state)."""

    @_default_event
    def on_transition(self, parent: int, action: Action, child, state, outcome) -> None:
        """Not sent by a BrFS (the reference's BrFS does not send it either)."""

    @_default_event
    def on_pass(self, width: int, stats: Statistics) -> None:
        """The brfs layer of this depth ended; ``stats`` are its own counts."""

    @_default_event
    def on_solution(self, plan: list, cost: float) -> None:
        """A plan was found."""

    @_default_event
    def on_progress(self, stats: Statistics) -> bool:
        """The statistics so far; return False to stop the search (status "cancelled")."""
        return True

    @_default_event
    def on_end(self, status: str, stats: Statistics) -> None:
        """The search ended with ``status`` and the total ``stats``."""


def _event(obj, name: str):
    fn = getattr(obj, name, None)
    if fn is None or getattr(fn, "_mymyr_default_event", False):
        return None
    return fn


def _stats(p) -> Statistics:
    v = p.contents
    return Statistics(int(v.expanded), int(v.generated), int(v.states), int(v.pruned), float(v.seconds), int(v.memory_bytes))


class _ObserverBridge:
    """The C observer (mya_search_observer) forwarding to a Python object's events; keeps the ctypes callbacks alive for
    the search and records the first exception an event raised."""

    def __init__(self, obj, interval: int):
        self.error: BaseException | None = None
        ev = {n: _event(obj, n) for n in ("on_start", "on_pass", "on_progress", "on_solution", "on_end", "on_expand", "on_generate",
                                          "on_prune")}
        self.defines_any = any(f is not None for f in ev.values())

        def guard(fn):
            def run(*args):
                if self.error is not None:
                    return None
                try:
                    return fn(*args)
                except BaseException as e:  # noqa: BLE001 - re-raised when the search returns
                    self.error = e
                    return None
            return run

        def on_start(_u, state, words):
            ev["on_start"](np.ctypeslib.as_array(state, shape=(words,)).copy())

        def on_pass(_u, layer, stats):
            ev["on_pass"](int(layer), _stats(stats))

        # the C side asks at every batch boundary (interval 1), so that an exception in any event stops the search at
        # the next batch; the observer's on_progress is called every `interval` expansions
        self.next_progress = max(1, interval)

        def on_progress(_u, stats):
            if self.error is not None:
                return 0
            if ev["on_progress"] is None or stats.contents.expanded < self.next_progress:
                return 1
            self.next_progress = int(stats.contents.expanded) + max(1, interval)
            r = guard(lambda: ev["on_progress"](_stats(stats)))()
            return 0 if self.error is not None or (r is not None and not r) else 1

        def on_solution(_u, schemas, bindings, length, width, cost):
            plan = [Action(int(schemas[i]), tuple(int(bindings[i * width + k]) for k in range(width) if bindings[i * width + k] >= 0))
                    for i in range(length)]
            ev["on_solution"](plan, float(cost))

        def on_end(_u, status, stats):
            ev["on_end"](STATUS.get(int(status), str(int(status))), _stats(stats))

        def row(p, words):
            return np.ctypeslib.as_array(p, shape=(words,)).copy()

        def action(schema, binding, arity):
            return Action(int(schema), tuple(int(binding[k]) for k in range(arity)))

        def on_expand(_u, sid, state, words):
            ev["on_expand"](int(sid), row(state, words))

        def on_generate(_u, parent, schema, binding, arity, child, state, words, is_new):
            ev["on_generate"](int(parent), action(schema, binding, arity), None if child == (1 << 64) - 1 else int(child),
                              row(state, words), bool(is_new))

        def on_prune(_u, parent, schema, binding, arity, state, words):
            ev["on_prune"](int(parent), action(schema, binding, arity), row(state, words))

        # on_progress is always installed: an exception in another event stops the search at the next batch
        self.c = _lib.SearchObserver(
            None,
            _lib.ON_START(guard(on_start)) if ev["on_start"] else _lib.ON_START(),
            _lib.ON_PASS(guard(on_pass)) if ev["on_pass"] else _lib.ON_PASS(),
            _lib.ON_PROGRESS(on_progress),
            _lib.ON_SOLUTION(guard(on_solution)) if ev["on_solution"] else _lib.ON_SOLUTION(),
            _lib.ON_END(guard(on_end)) if ev["on_end"] else _lib.ON_END(),
            _lib.ON_EXPAND(guard(on_expand)) if ev["on_expand"] else _lib.ON_EXPAND(),
            _lib.ON_GENERATE(guard(on_generate)) if ev["on_generate"] else _lib.ON_GENERATE(),
            _lib.ON_PRUNE(guard(on_prune)) if ev["on_prune"] else _lib.ON_PRUNE())


_LAYER_KINDS = {"queue": 0, "in_order": 1, "reverse": 2, "randomized": 3, "goal_count": 4}
_BEAM_NOVELTY = {"all_tested": 0, "survivors_only": 1, "relaxed_survivors_only": 2}


class _Layers:
    """BrfsOptions::layers from search.brfs's arguments (python/src/search_bindings.cpp:1638-1680): the kind, the
    limits (None: none; 0 is refused, as the reference's check_layers refuses it) and, for a scorer, the C callback
    that hands it the layer's rows; the first exception the scorer raises is raised when the search returns."""

    def __init__(self, order, seed, max_next, prefer_more, beam_width, novelty, randomize_ties, beam_chunk):
        self.error: BaseException | None = None
        self.c_scorer = _lib.LAYER_SCORER()
        if isinstance(order, str):
            if order not in _LAYER_KINDS:
                raise ValueError("mymyr: layer_order must be 'queue', 'in_order', 'reverse', 'randomized', 'goal_count' or an "
                                 "evaluator (scores, lower first)")
            self.kind = _LAYER_KINDS[order]
        else:
            score = getattr(order, "evaluate_batch", order)
            if not callable(score):
                raise TypeError("mymyr_amd: layer_order must be a kind name or a scorer")
            self.kind = 5

            def call(_u, rows, n, words, out):
                if self.error is not None:
                    for i in range(n):
                        out[i] = float("nan")
                    return
                try:
                    states = np.ctypeslib.as_array(rows, shape=(n, words)).copy() if n else np.zeros((0, words), np.uint64)
                    v = np.asarray(score(states), dtype=np.float64).reshape(-1)
                    if v.size != n:
                        raise ValueError(f"mymyr_amd: the layer scorer returned {v.size} scores for {n} states")
                    for i in range(n):
                        out[i] = float(v[i])
                except BaseException as e:  # noqa: BLE001 - raised when the search returns
                    self.error = e
                    for i in range(n):
                        out[i] = float("nan")

            self.c_scorer = _lib.LAYER_SCORER(call)
        if not 0 <= int(seed) < (1 << 64):
            raise ValueError("mymyr: seed must be a 64-bit unsigned integer")
        self.seed = int(seed)
        for name, v in (("max_next_layer_states", max_next), ("beam_width", beam_width)):
            if v is not None and not 0 < int(v) < (1 << 32) - 1:
                raise ValueError(f"mymyr brfs: {name} must be positive" if v is not None and int(v) <= 0 else
                                 f"mymyr: {name} must be below 2^32 - 1")
        self.limit = 0 if max_next is None else int(max_next)
        self.beam = 0 if beam_width is None else int(beam_width)
        if novelty not in _BEAM_NOVELTY:
            raise ValueError("mymyr: beam_novelty must be 'all_tested', 'survivors_only' or 'relaxed_survivors_only'")
        self.novelty = _BEAM_NOVELTY[novelty]
        if int(beam_chunk) <= 0:
            raise ValueError("mymyr brfs: beam_chunk must be positive")


@dataclass
class BrfsResult:
    """The fields of the reference's BrfsResult (include/mymyr/search/brfs.hpp:103-138) that the device search fills.
    A solved search has its plan (Actions from the start state to the first goal state tested), its cost (unit action
    costs: the plan's length) and goal_state (the goal state's words, uint64); unsolved: [], 0.0 and None."""

    status: str
    states: int
    expanded: int
    generated: int
    num_goal_states: int
    layers: int
    exhausted: bool
    solved: bool
    fingerprint: int
    first_goal: int
    search_s: float
    device_s: float
    layer_counts: list = field(default_factory=list)
    kernels: dict = field(default_factory=dict)  # class -> {"ms", "bytes", "launches"} (ms with timings=True)
    plan: list = field(default_factory=list)
    cost: float = 0.0
    goal_state: np.ndarray | None = None
    pruned: int = 0
    memory_bytes: int = 0
    words: int = 0          # the task's state words at the end (lazy slots: after interning)
    fluent_slots: int = 0   # assigned fluent atom slots at the end
    threads_used: int = 1   # host threads the search ran on (the calling thread; the work runs on the device)
    store: str = ""         # "device" (the device state set), "none" when nothing was searched
    message: str = ""       # why the search stopped early or ran otherwise than asked ("" if neither)

    @property
    def stats(self) -> Statistics:
        """The search's counts and time as Statistics (the reference's result.stats, brfs_stats in
        python/src/search_bindings.cpp:661-670): expanded, generated, states, pruned, seconds (search_s) and
        memory_bytes."""
        return Statistics(self.expanded, self.generated, self.states, self.pruned, self.search_s, self.memory_bytes)


KERNEL_CLASSES = ["count", "emit", "insert", "unused", "rank", "compact", "other"]


class CancelToken:
    """The reference's mymyr.search.CancelToken (python/src/search_bindings.cpp:2277-2287, search::CancelToken,
    include/mymyr/search/control.hpp:81-90): request() from any thread stops a search that holds the token (status
    "cancelled"). The flag is a 32-bit word the device search reads between batches."""

    def __init__(self):
        self._flag = ctypes.c_int32(0)

    def request(self) -> None:
        self._flag.value = 1

    @property
    def requested(self) -> bool:
        return bool(self._flag.value)

    @property
    def address(self) -> int:
        return ctypes.addressof(self._flag)

    def __repr__(self) -> str:
        return f"CancelToken(requested={self.requested})"


def _rows(task: Task, rows, what: str) -> np.ndarray:
    """States as [k, task.words] uint64 rows (the task's state words)."""
    a = np.ascontiguousarray(np.asarray(rows, dtype=np.uint64))
    if a.ndim == 1:
        a = a.reshape(1, -1)
    if a.ndim != 2 or a.shape[1] != task.words:
        raise ValueError(f"mymyr_amd: brfs: {what} must have {task.words} words per state, got shape {a.shape}")
    return a


class _GoalTest:
    """A callable goal (state words -> bool) as the C goal test: each row of a batch is passed as a uint64 array of the
    task's words (the reference passes its State view); the first exception stops the search and is raised again."""

    def __init__(self, fn):
        self.fn, self.error = fn, None

        def call(_user, rows, n, words, out):
            if self.error is not None:
                return 1
            try:
                a = np.ctypeslib.as_array(rows, shape=(n, words))
                for i in range(n):
                    out[i] = 1 if self.fn(a[i].copy()) else 0
                return 0
            except BaseException as e:  # noqa: BLE001 (raised again after the search)
                self.error = e
                return 1

        self.c = _lib.GOAL_TEST(call)


def _goal_records(task: Task, goal) -> tuple[np.ndarray, np.ndarray]:
    """AnyOf goal conditions as the C ABI's offsets [k + 1] and literal records (predicate, positive, object count,
    objects). A condition is a sequence of (predicate index, positive, objects) literals."""
    if isinstance(goal, (str, bytes)) or not hasattr(goal, "__iter__"):
        raise TypeError("mymyr: goal= takes a sequence of ground conditions (each a sequence of (predicate, positive, objects))")
    offs, recs = [0], []
    for cond in goal:
        for lit in cond:
            pred, pos, objs = lit
            objs = [int(o) for o in objs]
            if len(objs) > _lib.GOAL_LITERAL_INTS - 3:
                raise ValueError("mymyr_amd: brfs: goal literals hold at most 6 objects")
            recs.append([int(pred), int(bool(pos)), len(objs)] + objs + [0] * (_lib.GOAL_LITERAL_INTS - 3 - len(objs)))
        offs.append(len(recs))
    return np.array(offs, np.uint32), np.array(recs, np.int32).reshape(-1, _lib.GOAL_LITERAL_INTS)


def brfs(task: Task, max_depth: int | None = None, max_states: int | None = None, max_expanded: int | None = None,
         witness_pruning: bool = True, stop_at_goal: bool = True, fingerprint: bool = False, layer_stats: bool = True,
         chunk: int = 0, memory_states: int = 0, timings: bool = False, start=None, blocked_states=None,
         max_seconds: float | None = None, cancel: CancelToken | None = None, goal=None, observer=None,
         progress_interval: int | None = None, layer_order="queue", seed: int = 0, max_next_layer_states: int | None = None,
         prefer_more_satisfied_goals: bool = True, beam_width: int | None = None, beam_novelty: str = "all_tested",
         randomize_ties: bool = False, beam_chunk: int = 1024, threads: int = 1, store: str = "auto", canonical_order: bool = True,
         deterministic_ids: bool = True) -> BrfsResult:
    """Breadth-first search on the current HIP device. Defaults follow the reference's BrfsOptions
    (witness_pruning and stop_at_goal on). layer_counts holds [expanded, generated, new] per expanded layer.

    start: the start state's words (default: the task's initial state). blocked_states: states never stored ([k, words]
    or a list of rows); a successor equal to one counts as generated and pruned (the start state is exempt).
    max_seconds (None: unlimited) and cancel (a CancelToken) stop the search between device batches with status
    "out_of_time" or "cancelled" (python/src/search_bindings.cpp:516-538, 2135-2145).
    goal (None: the task's goal): BrfsOptions::goal as GoalSpec::AnyOf, a sequence of ground conditions, each a sequence
    of (predicate index, positive, object indices) literals; a state is a goal iff one of them holds in it (the
    reference's goal= with GroundConditions, python/src/search_bindings.cpp:439-505; conditions that can never hold are
    left out). Or a callable (GoalSpec::Custom, python/src/search_bindings.cpp:444-448; threads=1): goal(words) -> bool
    on a state's uint64 words in the task's slot layout (the reference passes its State view), called on each state
    before it is expanded; an exception in it stops the search and is raised again.
    observer (an :class:`Observer`, or any object with some of its methods) and progress_interval (expansions between
    on_progress calls; None: 2^16): BrfsOptions::observer and progress_interval (include/mymyr/search/brfs.hpp:99-100).
    layer_order, seed, max_next_layer_states, prefer_more_satisfied_goals, beam_width, beam_novelty, randomize_ties and
    beam_chunk: BrfsOptions::layers (include/mymyr/search/layer_ordering.hpp; python/src/search_bindings.cpp:1638-1680,
    2206-2233): 'queue' (the default), 'in_order', 'reverse', 'randomized', 'goal_count', or a scorer (a callable
    taking the layer's states [n, words] uint64 and returning n scores, lower first, or an object with evaluate_batch);
    'relaxed_survivors_only' is refused by the device search.
    threads, store and deterministic_ids are the reference's host-side choices (python/src/search_bindings.cpp:3396-3398):
    they are checked and the device state set is used (its ids are the single-threaded search's, which every thread
    count of the reference's deterministic search gives); canonical_order=False (the matcher's own order) is refused."""
    if max_seconds is not None and not max_seconds >= 0:
        raise ValueError("mymyr_amd: brfs: max_seconds must be >= 0")
    if store not in ("auto", "flat", "chunked", "compact", "concurrent"):
        raise ValueError("mymyr: store must be 'auto', 'flat', 'chunked', 'compact' or 'concurrent'")
    if int(threads) < 0:
        raise ValueError("mymyr: threads must be >= 0")
    if not canonical_order:
        raise ValueError("mymyr_amd: brfs: the device search generates successors in canonical order only "
                         "(canonical_order=False is not supported)")
    if cancel is not None and not isinstance(cancel, CancelToken):
        raise TypeError("mymyr_amd: cancel must be a mymyr_amd.search.CancelToken")
    st = None if start is None else _rows(task, start, "start")
    if st is not None and st.shape[0] != 1:
        raise ValueError("mymyr_amd: brfs: start must be one state")
    bl = None if blocked_states is None else _rows(task, np.zeros((0, task.words), np.uint64) if len(blocked_states) == 0
                                                   else blocked_states, "blocked_states")
    timed = max_seconds is not None and np.isfinite(max_seconds)
    goal_test = None
    if goal is not None and callable(goal) and not isinstance(goal, (str, bytes)):
        # GoalSpec::Custom: the callable decides on each state's words (python/src/search_bindings.cpp:444-448)
        if int(threads) > 1:
            raise ValueError("mymyr brfs: a custom goal test needs threads == 1 and a test function")
        goal_test = _GoalTest(goal)
        go, gl = None, None
    else:
        go, gl = _goal_records(task, goal) if goal is not None else (None, None)
    if progress_interval is not None and not 0 <= int(progress_interval) < (1 << 64):
        raise ValueError("mymyr_amd: brfs: progress_interval must be a non-negative 64-bit count")
    bridge = _ObserverBridge(observer, (1 << 16) if progress_interval is None else int(progress_interval)) if observer is not None else None
    lay = _Layers(layer_order, seed, max_next_layer_states, prefer_more_satisfied_goals, beam_width, beam_novelty, randomize_ties,
                  beam_chunk)
    if bridge is not None and not bridge.defines_any:
        bridge = None  # an observer that defines no event is not installed
    o = _lib.BrfsOptions(UNBOUNDED32 if max_depth is None else max_depth, int(witness_pruning),
                         UNBOUNDED64 if max_states is None else max_states, UNBOUNDED64 if max_expanded is None else max_expanded,
                         int(stop_at_goal), int(fingerprint), chunk, memory_states, int(timings), 0,
                         None if st is None else st.ctypes.data, None if bl is None or bl.shape[0] == 0 else bl.ctypes.data,
                         0 if bl is None else bl.shape[0], task.words, int(timed), float(max_seconds) if timed else 0.0,
                         None if cancel is None else cancel.address, 0 if go is None else 1, 0 if go is None else len(go) - 1,
                         None if go is None else go.ctypes.data, None if gl is None or gl.size == 0 else gl.ctypes.data,
                         None if bridge is None else ctypes.addressof(bridge.c), 1, lay.kind, int(not prefer_more_satisfied_goals),
                         lay.seed, lay.limit, lay.beam, int(bool(randomize_ties)), lay.novelty, lay.c_scorer, None,
                         _lib.GOAL_TEST() if goal_test is None else goal_test.c, None)
    r = _lib.BrfsResult()
    lc = np.zeros((4096, 3), dtype=np.uint64)
    L = max(1, task.label_width)
    cap = 1 << 16
    ps = np.zeros(cap, np.int32)
    pb = np.zeros((cap, L), np.int32)
    # lazy slots: the goal state may be as wide as the task's canonical atoms make it
    gs = np.zeros(max(1, task.words if task.frozen else (task.dense_fluent + 63) // 64), np.uint64)
    plan = _lib.BrfsPlan(ps.ctypes.data, pb.ctypes.data, cap, L, gs.ctypes.data, gs.size, 0, 0, 0, 0.0)
    n = lib.mya_brfs(task.handle, ctypes.byref(o), ctypes.byref(r), lc.ctypes.data, 4096, ctypes.byref(plan))
    if goal_test is not None and goal_test.error is not None:
        raise goal_test.error
    if lay.error is not None:
        raise lay.error
    if n < 0:
        check(-1)
    if bridge is not None and bridge.error is not None:
        raise bridge.error
    kernels = {c: {"ms": r.kernel_ms[i], "bytes": r.kernel_bytes[i], "launches": r.kernel_launches[i]}
               for i, c in enumerate(KERNEL_CLASSES)}
    res = BrfsResult(STATUS.get(r.status, str(r.status)), r.states, r.expanded, r.generated, r.goal_states, r.layers,
                     bool(r.exhausted), bool(r.solved), r.fingerprint, r.first_goal, r.search_s, r.device_s,
                     lc[:n].tolist() if layer_stats else [], kernels, pruned=r.pruned, memory_bytes=r.memory_bytes,
                     words=r.words, fluent_slots=r.fluent_slots, threads_used=r.threads_used, store=r.store.decode(),
                     message=r.message.decode())
    if r.solved:
        if plan.length > cap:
            raise RuntimeError(f"mymyr_amd: brfs: a plan of {plan.length} actions (at most {cap} are read)")
        res.plan = [Action(int(ps[i]), tuple(int(x) for x in pb[i] if x >= 0)) for i in range(plan.length)]
        res.cost = plan.cost
        res.goal_state = gs[: plan.goal_words].copy()
    return res
