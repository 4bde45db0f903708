"""Test infrastructure, not product code: ctypes binding of oracle/_ref/libmymyr_ref.so, the reference CPU core
(maichmueller/mymyr) compiled from its own sources by oracle/Makefile, with the harness oracle/ref_harness.cpp.

Only tests/, __graft_entry__.smoke() and bench.py's CPU-baseline leg use it, to check results or as the timed CPU
baseline; the product never imports it.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_uint32, c_uint64, c_void_p

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "_ref", "libmymyr_ref.so")


class EnvConfig(Structure):
    _fields_ = [
        ("seed", c_uint64),
        ("max_steps", c_uint32),
        ("step_reward", c_float),
        ("goal_reward", c_float),
        ("dead_end_reward", c_float),
        ("dead_end", c_int32),
        ("dead_end_terminal", c_int32),
        ("autoreset", c_int32),
        ("canonical_order", c_int32),
        ("witness_pruning", c_int32),
        ("label_actions", c_int32),
    ]


class BrfsOptions(Structure):
    _fields_ = [
        ("threads", c_uint32),
        ("max_depth", c_uint32),
        ("max_states", c_uint64),
        ("witness_pruning", c_int32),
        ("canonical_order", c_int32),
        ("stop_at_goal", c_int32),
        ("fingerprint", c_int32),
        ("max_expanded", c_uint64),
        ("start", c_void_p),
        ("blocked", c_void_p),
        ("blocked_count", c_uint64),
        ("words", c_uint32),
        ("reserved", c_uint32),
        ("max_seconds", c_double),
        ("goal_kind", c_int32),
        ("goal_count", c_uint32),
        ("goal_offsets", c_void_p),
        ("goal_literals", c_void_p),
        ("layer_kind", c_int32),
        ("prefer_fewer", c_int32),
        ("layer_seed", c_uint64),
        ("max_next_layer_states", c_uint32),
        ("beam_width", c_uint32),
        ("randomize_ties", c_int32),
        ("record_events", c_int32),
        ("scorer", ctypes.CFUNCTYPE(None, c_void_p, ctypes.POINTER(c_uint64), c_uint64, c_uint32, ctypes.POINTER(ctypes.c_double))),
        ("scorer_user", c_void_p),
        ("goal_mod", c_uint64),
        ("goal_res", c_uint64),
    ]


SCORER = dict(BrfsOptions._fields_)["scorer"]
LAYER_KINDS = {"queue": 0, "in_order": 1, "reverse": 2, "randomized": 3, "goal_count": 4}


def goal_records(goal) -> tuple[np.ndarray, np.ndarray]:
    """AnyOf goal conditions (a list of conditions, each a list of (predicate, positive, objects) literals) as the
    harness's offsets [k + 1] and 8-int32 literal records (predicate, positive, objects, zero padded)."""
    offs = [0]
    recs = []
    for cond in goal:
        for pred, pos, objs in cond:
            objs = list(objs)
            if len(objs) > 6:
                raise ValueError("goal literals of more than 6 objects")
            recs.append([int(pred), int(bool(pos))] + [int(o) for o in objs] + [0] * (6 - len(objs)))
        offs.append(len(recs))
    return np.array(offs, np.uint32), np.array(recs if recs else np.zeros((0, 8)), np.int32).reshape(-1, 8)


class PoolOut(Structure):
    _fields_ = [
        ("cap", c_uint64),
        ("words", c_uint32),
        ("label_width", c_uint32),
    ] + [(n, c_void_p) for n in ("env_ids", "states", "task_ids", "count", "steps", "at_goal", "terminated", "goal", "reward", "truncated",
                                  "invalid", "final_states", "schema", "binding")]


class BrfsResult(Structure):
    _fields_ = [
        ("states", c_uint64),
        ("expanded", c_uint64),
        ("generated", c_uint64),
        ("goal_states", c_uint64),
        ("fingerprint", c_uint64),
        ("layers", c_uint32),
        ("status", c_int32),
        ("solved", c_int32),
        ("exhausted", c_int32),
        ("seconds", c_double),
        ("cost", c_double),
        ("pruned", c_uint64),
        ("plan_len", c_uint32),
        ("goal_words", c_uint32),
        ("words", c_uint32),
        ("fluent_slots", c_uint32),
        ("threads_used", c_uint32),
        ("reserved", c_uint32),
        ("store", ctypes.c_char * 16),
        ("message", ctypes.c_char * 256),
    ]


def available() -> bool:
    return os.path.exists(LIB_PATH)


_lib = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not available():
            raise ImportError(f"reference build missing: {LIB_PATH} (make -C oracle)")
        L = ctypes.CDLL(LIB_PATH)
        sig = {
            "mref_last_error": (c_char_p, []),
            "mref_task_load": (c_void_p, [c_char_p, c_int]),
            "mref_task_free": (None, [c_void_p]),
            "mref_task_info": (c_int, [c_void_p, c_void_p]),
            "mref_task_slots": (c_int, [c_void_p, c_void_p, c_void_p]),
            "mref_task_initial": (c_int, [c_void_p, c_void_p, c_uint32]),
            "mref_task_goal": (c_int, [c_void_p, c_void_p, c_uint32]),
            "mref_canonical_hash": (c_uint64, [c_void_p, c_void_p, c_uint32]),
            "mref_successors": (c_int64, [c_void_p, c_void_p, c_uint32, c_int, c_int, c_void_p, c_void_p, c_uint32, c_void_p, c_uint32, c_uint64]),
            "mref_brfs_events": (c_uint64, [c_void_p, c_uint64]),
            "mref_hash_words": (c_uint64, [c_void_p, c_uint32, c_uint64]),
            "mref_hash_state": (c_uint64, [c_void_p, c_uint32]),
            "mref_hash_rows": (None, [c_void_p, c_uint64, c_uint32, c_uint32, c_void_p]),
            "mref_hash_mix64": (c_uint64, [c_uint64]),
            "mref_philox": (None, [c_uint64, c_uint64, c_uint64, c_uint32, c_void_p]),
            "mref_philox_raw": (None, [c_void_p, c_uint32, c_uint32, c_void_p]),
            "mref_successor_index": (c_uint32, [c_uint64, c_uint64, c_uint64, c_uint32]),
            "mref_env_create": (c_void_p, [c_void_p, POINTER(EnvConfig), c_uint32]),
            "mref_env_free": (None, [c_void_p]),
            "mref_env_reset": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p, c_uint64]),
            "mref_env_step": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, c_void_p, c_void_p, c_void_p, c_uint64, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p]),
            "mref_table_env_create": (c_void_p, [c_void_p, c_uint32, POINTER(EnvConfig), c_uint32, c_void_p, c_void_p, c_uint32, c_int]),
            "mref_table_env_reset": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int]),
            "mref_table_env_step": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_void_p]),
            "mref_table_env_step_labels": (c_int, [c_void_p, c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p,
                                                   c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_uint32, c_void_p]),
            "mref_table_env_clear_visited": (c_int, [c_void_p, c_void_p, c_void_p]),
            "mref_table_expand": (c_int64, [c_void_p, c_uint32, c_void_p, c_void_p, c_uint64, c_uint32, c_int, c_uint64, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                            POINTER(c_uint64)]),
            "mref_table_pad": (c_int, [c_void_p, c_uint32, c_void_p, c_void_p, c_uint64, c_uint32, c_int, c_uint32, c_uint32] + [c_void_p] * 10),
            "mref_visited_insert": (None, [c_void_p, c_uint32, c_void_p, c_void_p, c_uint64, c_void_p]),
            "mref_visited_mask": (None, [c_void_p, c_void_p, c_uint32, c_void_p, c_void_p, c_void_p, c_uint64, c_void_p]),
            "mref_instance_draw": (c_int32, [c_uint64, c_uint64, c_uint32, c_uint32, c_void_p, c_void_p, c_uint32]),
            "mref_pool_run": (c_int, [c_void_p, POINTER(EnvConfig), c_uint32, c_uint32, c_uint32, POINTER(c_double), POINTER(c_uint64)]),
            "mref_brfs": (c_int, [c_void_p, POINTER(BrfsOptions), POINTER(BrfsResult), c_void_p, c_uint32, c_void_p, c_void_p,
                                  c_uint32, c_uint32, c_void_p, c_uint32]),
            "mref_pool_create": (c_void_p, [c_void_p, POINTER(EnvConfig), c_uint32, c_uint32, c_uint64]),
            "mref_pool_free": (None, [c_void_p]),
            "mref_pool_reset": (c_int64, [c_void_p, c_void_p, c_uint64, POINTER(PoolOut)]),
            "mref_pool_send": (c_int64, [c_void_p, c_void_p, c_uint64, c_void_p]),
            "mref_pool_recv": (c_int64, [c_void_p, c_uint64, POINTER(PoolOut)]),
            "mref_pool_recv_ticket": (c_int64, [c_void_p, c_uint64, POINTER(PoolOut)]),
            "mref_pool_pending": (c_int64, [c_void_p]),
            "mref_dedup_flat": (c_int, [c_void_p, c_uint64, c_uint32, POINTER(c_uint64), POINTER(c_double)]),
            "mref_dedup_concurrent": (c_int, [c_void_p, c_uint64, c_uint32, c_uint32, c_uint64, POINTER(c_uint64), POINTER(c_double)]),
        }
        for name, (res, args) in sig.items():
            f = getattr(L, name)
            f.restype = res
            f.argtypes = args
        _lib = L
    return _lib


def _err() -> str:
    return lib().mref_last_error().decode()


def _p(a: np.ndarray | None):
    return None if a is None else a.ctypes.data


class RefTask:
    """A reference Task (Task::from_text_file) plus its one-instance TaskTable."""

    MODES = {"auto": 0, "reachable": 1, "dense": 2, "lazy": 3}

    def __init__(self, path: str, atoms: str = "auto"):
        h = lib().mref_task_load(str(path).encode(), self.MODES[atoms])
        if not h:
            raise RuntimeError(_err())
        self._h = c_void_p(h)
        self.refresh()

    def refresh(self):
        """Reads the task's sizes again (lazy slots grow as searches meet atoms)."""
        info = np.zeros(9, dtype=np.uint64)
        assert lib().mref_task_info(self._h, info.ctypes.data) == 0
        (self.words, self.fluent_slots, mode, self.num_schemas, self.label_width, self.num_objects, self.max_arity,
         self.table_words, self.dense_fluent) = (int(x) for x in info)
        self.atom_mode = {0: "reachable", 1: "dense", 2: "lazy"}[mode]

    def slot_records(self):
        stride = 1 + max(1, self.max_arity)
        rec = np.zeros((self.fluent_slots, stride), dtype=np.uint32)
        cid = np.zeros(self.fluent_slots, dtype=np.uint64)
        if lib().mref_task_slots(self._h, rec.ctypes.data, cid.ctypes.data) != 0:
            raise RuntimeError(_err())
        return rec, cid

    def initial_state(self, words: int | None = None) -> np.ndarray:
        w = self.table_words if words is None else words
        row = np.zeros(w, dtype=np.uint64)
        if lib().mref_task_initial(self._h, row.ctypes.data, w) != 0:
            raise RuntimeError(_err())
        return row

    def is_goal(self, row: np.ndarray) -> bool:
        row = np.ascontiguousarray(row, dtype=np.uint64)
        return lib().mref_task_goal(self._h, row.ctypes.data, row.size) == 1

    def canonical_hash(self, row: np.ndarray) -> int:
        row = np.ascontiguousarray(row, dtype=np.uint64)
        return int(lib().mref_canonical_hash(self._h, row.ctypes.data, row.size))

    def successors(self, row: np.ndarray, witness: bool = False, canonical: bool = True, cap: int = 1 << 16):
        """(schema [k], binding [k, L], rows [k, W]) in the reference generator's order."""
        row = np.ascontiguousarray(row, dtype=np.uint64)
        L = max(1, self.label_width)
        W = self.table_words
        schema = np.zeros(cap, dtype=np.int32)
        binding = np.zeros((cap, L), dtype=np.int32)
        rows = np.zeros((cap, W), dtype=np.uint64)
        k = lib().mref_successors(self._h, row.ctypes.data, row.size, int(witness), int(canonical), schema.ctypes.data,
                                  binding.ctypes.data, L, rows.ctypes.data, W, cap)
        if k < 0:
            raise RuntimeError(_err())
        if k > cap:
            return self.successors(row, witness, canonical, cap=int(k))
        return schema[:k], binding[:k], rows[:k]

    def __del__(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().mref_task_free(self._h)
            self._h = c_void_p()


class RefEnv:
    """rl::HostEnv over a one-instance table (reference env step semantics)."""

    def __init__(self, task: RefTask, seed=0, max_steps=0, step_reward=0.0, goal_reward=1.0, dead_end_reward=0.0,
                 dead_end="no_successors", dead_end_terminal=True, autoreset=True, canonical_order=True,
                 witness_pruning=False, threads=1):
        self.task = task
        self.cfg = EnvConfig(seed, max_steps, step_reward, goal_reward, dead_end_reward, 1 if dead_end == "none" else 0,
                             int(dead_end_terminal), int(autoreset), int(canonical_order), int(witness_pruning))
        h = lib().mref_env_create(task._h, ctypes.byref(self.cfg), threads)
        if not h:
            raise RuntimeError(_err())
        self._h = c_void_p(h)

    def reset(self, states, steps, draws, at_goal, count, first_env=0):
        rows, words = states.shape
        if lib().mref_env_reset(self._h, states.ctypes.data, rows, words, _p(steps), _p(draws), _p(at_goal), _p(count), first_env) != 0:
            raise RuntimeError(_err())

    def step(self, states, steps, draws, at_goal, first_env=0, actions=None, reward=None, terminated=None, truncated=None,
             count=None, schema=None, binding=None, goal=None, invalid=None, final_states=None):
        rows, words = states.shape
        lw = 0 if binding is None else binding.shape[1]
        rc = lib().mref_env_step(self._h, states.ctypes.data, rows, words, _p(steps), _p(draws), _p(at_goal), first_env, _p(actions),
                                 _p(reward), _p(terminated), _p(truncated), _p(count), _p(schema), _p(binding), lw, _p(goal),
                                 _p(invalid), _p(final_states))
        if rc != 0:
            raise RuntimeError(_err())

    def __del__(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().mref_env_free(self._h)
            self._h = c_void_p()


class TableBatch(Structure):
    _fields_ = [
        ("states", c_void_p), ("rows", c_uint64), ("words", c_uint32), ("reserved", c_uint32), ("steps", c_void_p),
        ("draws", c_void_p), ("at_goal", c_void_p), ("first_env", c_uint64), ("task_ids", c_void_p), ("goal_pos", c_void_p),
        ("goal_neg", c_void_p), ("reset_counts", c_void_p), ("seeds", c_void_p), ("env_ids", c_void_p),
        ("sampling_seeds", c_void_p), ("visited", c_void_p), ("visited_count", c_void_p), ("visited_status", c_void_p),
        ("visited_capacity", c_uint32), ("reserved2", c_uint32),
    ]


class RefTableEnv:
    """rl::HostEnv over TaskTable::create(tasks) (suite=True: TaskSuite::group(tasks), several domains): per-row task ids,
    with an instance sampler when `sampler` = (instances, thresholds, indices) is given (empty arrays: uniform)."""

    def __init__(self, tasks: list, seed=0, max_steps=0, step_reward=0.0, goal_reward=1.0, dead_end_reward=0.0,
                 dead_end="no_successors", dead_end_terminal=True, autoreset=True, sampler=None, suite=False, labels=False):
        self.tasks = tasks
        self.cfg = EnvConfig(seed, max_steps, step_reward, goal_reward, dead_end_reward, 1 if dead_end == "none" else 0,
                             int(dead_end_terminal), int(autoreset), 1, 0, int(labels))
        arr = (c_void_p * len(tasks))(*[t._h.value for t in tasks])
        inst, thr, idx = sampler if sampler is not None else (0, [], [])
        self._thr = np.asarray(thr, np.uint32)
        self._idx = np.asarray(idx, np.int32)
        h = lib().mref_table_env_create(arr, len(tasks), ctypes.byref(self.cfg), inst, self._thr.ctypes.data, self._idx.ctypes.data,
                                        len(self._idx), int(suite))
        if not h:
            raise RuntimeError(_err())
        self._h = c_void_p(h)

    @staticmethod
    def batch(b: dict, first_env: int = 0) -> TableBatch:
        """The harness batch over a dict of numpy arrays (states, steps, draws, at_goal, task_ids, and optionally
        goal_pos, goal_neg, reset_counts, seeds, env_ids, sampling_seeds)."""
        rows, words = b["states"].shape
        g = lambda k: _p(b.get(k))
        H = b["visited"].shape[1] if b.get("visited") is not None else 0
        return TableBatch(b["states"].ctypes.data, rows, words, 0, g("steps"), g("draws"), g("at_goal"), first_env, g("task_ids"),
                          g("goal_pos"), g("goal_neg"), g("reset_counts"), g("seeds"), g("env_ids"), g("sampling_seeds"), g("visited"),
                          g("visited_count"), g("visited_status"), H, 0)

    def clear_visited(self, b: dict, mask=None):
        tb = self.batch(b)
        if lib().mref_table_env_clear_visited(self._h, ctypes.byref(tb), _p(mask)) != 0:
            raise RuntimeError(_err())

    def reset(self, b: dict, count, mask=None, keep_goals=False, sample=False, first_env=0):
        tb = self.batch(b, first_env)
        if lib().mref_table_env_reset(self._h, ctypes.byref(tb), _p(count), _p(mask), int(keep_goals), int(sample)) != 0:
            raise RuntimeError(_err())

    def step(self, b: dict, first_env=0, actions=None, next_task_ids=None, reward=None, terminated=None, truncated=None, count=None,
             schema=None, binding=None, goal=None, invalid=None, final_states=None, revisited=None, labels=None):
        tb = self.batch(b, first_env)
        lw = 0 if binding is None else binding.shape[1]
        fw = 0 if final_states is None else final_states.shape[1]
        if labels is not None:
            ls, lb = np.ascontiguousarray(labels[0], np.int32), np.ascontiguousarray(labels[1], np.int32)
            rc = lib().mref_table_env_step_labels(self._h, ctypes.byref(tb), ls.ctypes.data, lb.ctypes.data, lb.shape[1], _p(next_task_ids),
                                                  _p(reward), _p(terminated), _p(truncated), _p(count), _p(schema), _p(binding), lw,
                                                  _p(goal), _p(invalid), _p(final_states), fw, _p(revisited))
            if rc != 0:
                raise RuntimeError(_err())
            return
        rc = lib().mref_table_env_step(self._h, ctypes.byref(tb), _p(actions), _p(next_task_ids), _p(reward), _p(terminated),
                                       _p(truncated), _p(count), _p(schema), _p(binding), lw, _p(goal), _p(invalid), _p(final_states), fw,
                                       _p(revisited))
        if rc != 0:
            raise RuntimeError(_err())

    def __del__(self):
        if getattr(self, "_h", None) is not None and self._h.value:
            lib().mref_env_free(self._h)
            self._h = c_void_p()


def table_expand(tasks: list, states: np.ndarray, task_ids: np.ndarray, drop_noops: bool = False) -> dict:
    """rl::expand over TaskTable::create(tasks): every output of the flat expansion (capacity = every successor)."""
    arr = (c_void_p * len(tasks))(*[t._h.value for t in tasks])
    rows, words = states.shape
    L = max(1, max(t.label_width for t in tasks))
    total = c_uint64()
    states = np.ascontiguousarray(states, np.uint64)
    ids = np.ascontiguousarray(task_ids, np.int32)
    off = np.zeros(rows + 1, np.int32)
    gen = lib().mref_table_expand(arr, len(tasks), states.ctypes.data, ids.ctypes.data, rows, words, int(drop_noops), 0, None, None, None,
                                  None, L, None, None, None, None, off.ctypes.data, ctypes.byref(total))
    if gen < 0:
        raise RuntimeError(_err())
    cap = int(gen)
    out = {"succ": np.zeros((cap, words), np.uint64), "parent": np.zeros(cap, np.int32), "schema": np.zeros(cap, np.int32),
           "binding": np.zeros((cap, L), np.int32), "goal": np.zeros(cap, np.uint8), "succ_hash": np.zeros(cap, np.uint64),
           "noop": np.zeros(cap, np.uint8), "index": np.zeros(cap, np.int32), "offsets": off}
    g = lib().mref_table_expand(arr, len(tasks), states.ctypes.data, ids.ctypes.data, rows, words, int(drop_noops), cap,
                                out["succ"].ctypes.data, out["parent"].ctypes.data, out["schema"].ctypes.data, out["binding"].ctypes.data,
                                L, out["goal"].ctypes.data, out["succ_hash"].ctypes.data, out["noop"].ctypes.data, out["index"].ctypes.data,
                                off.ctypes.data, ctypes.byref(total))
    if g < 0:
        raise RuntimeError(_err())
    kept = int(total.value)
    for k in ("succ", "parent", "schema", "binding", "goal", "succ_hash", "noop", "index"):
        out[k] = out[k][:kept]
    out["generated"], out["total"] = int(g), kept
    return out


def table_pad(tasks: list, states: np.ndarray, task_ids: np.ndarray, k: int, drop_noops: bool = False) -> dict:
    """rl::pad of the full flat expansion of a batch over TaskSuite::group(tasks) into [rows, k] arrays."""
    arr = (c_void_p * len(tasks))(*[t._h.value for t in tasks])
    rows, words = states.shape
    L = max(1, max(t.label_width for t in tasks))
    out = {"index": np.zeros((rows, k), np.int32), "mask": np.zeros((rows, k), np.uint8), "count": np.zeros(rows, np.int32),
           "succ": np.zeros((rows, k, words), np.uint64), "schema": np.zeros((rows, k), np.int32),
           "binding": np.zeros((rows, k, L), np.int32), "goal": np.zeros((rows, k), np.uint8), "succ_hash": np.zeros((rows, k), np.uint64),
           "noop": np.zeros((rows, k), np.uint8), "canonical": np.zeros((rows, k), np.int32)}
    states = np.ascontiguousarray(states, np.uint64)
    ids = np.ascontiguousarray(task_ids, np.int32)
    r = lib().mref_table_pad(arr, len(tasks), states.ctypes.data, ids.ctypes.data, rows, words, int(drop_noops), k, L,
                             *[out[n].ctypes.data for n in ("index", "mask", "count", "succ", "schema", "binding", "goal", "succ_hash",
                                                           "noop", "canonical")])
    if r < 0:
        raise RuntimeError(_err())
    out["overflow"] = bool(r)
    return out


def visited_insert(table: np.ndarray, count: int, hashes) -> tuple[np.ndarray, int]:
    """rl::visited_insert of each hash into one table (uint64 [H], written in place): (present flags, new count)."""
    h = np.ascontiguousarray(hashes, np.uint64)
    c = np.array([count], np.int32)
    present = np.zeros(len(h), np.uint8)
    lib().mref_visited_insert(table.ctypes.data, len(table), c.ctypes.data, h.ctypes.data, len(h), present.ctypes.data)
    return present, int(c[0])


def visited_mask(table: np.ndarray, count: np.ndarray, succ_hash, parent, rows=None) -> np.ndarray:
    """rl::visited_mask: table uint64 [n, H], count int32 [n]."""
    table = np.ascontiguousarray(table, np.uint64)
    count = np.ascontiguousarray(count, np.int32)
    h = np.ascontiguousarray(succ_hash, np.uint64)
    p = np.ascontiguousarray(parent, np.int32)
    r = None if rows is None else np.ascontiguousarray(rows, np.int32)
    out = np.zeros(len(h), np.uint8)
    lib().mref_visited_mask(table.ctypes.data, count.ctypes.data, table.shape[1], h.ctypes.data, p.ctypes.data,
                            None if r is None else r.ctypes.data, len(h), out.ctypes.data)
    return out


def instance_draw(seed, env, reset_count, instances, thresholds=(), indices=()) -> int:
    thr = np.asarray(thresholds, np.uint32)
    idx = np.asarray(indices, np.int32)
    return int(lib().mref_instance_draw(seed, env, reset_count, instances, thr.ctypes.data, idx.ctypes.data, len(idx)))


def pool_run(task: RefTask, num_envs: int, threads: int, steps: int, **cfg) -> tuple[float, int]:
    """CpuEnvPool (threads workers): reset, then `steps` random-policy steps of every env. (seconds, checksum)."""
    e = RefEnv.__new__(RefEnv)
    c = EnvConfig(cfg.get("seed", 0), cfg.get("max_steps", 0), cfg.get("step_reward", 0.0), cfg.get("goal_reward", 1.0),
                  cfg.get("dead_end_reward", 0.0), 1 if cfg.get("dead_end") == "none" else 0,
                  int(cfg.get("dead_end_terminal", True)), int(cfg.get("autoreset", True)), 1, 0)
    secs = c_double()
    chk = c_uint64()
    if lib().mref_pool_run(task._h, ctypes.byref(c), num_envs, threads, steps, ctypes.byref(secs), ctypes.byref(chk)) != 0:
        raise RuntimeError(_err())
    del e
    return secs.value, chk.value


def brfs(task: RefTask, threads=1, max_depth=0xFFFFFFFF, max_states=(1 << 64) - 1, witness_pruning=True, canonical_order=True,
         stop_at_goal=False, fingerprint=True, max_expanded=(1 << 64) - 1, start=None, blocked_states=None, max_seconds=float("inf"),
         goal=None, layer_order="queue", seed=0, max_next_layer_states=None, prefer_more_satisfied_goals=True, beam_width=None,
         randomize_ties=False, record_events=False, goal_hash=None, goal_atoms=None):
    """brfs(Task, BrfsOptions) of the reference: counts, status, fingerprint, and for a solved search the plan
    (schema, binding) pairs, the goal state's words and the cost; the result's words, fluent_slots, threads_used, store
    and message. start [words] and blocked_states [k, words] are rows of the task's table words; goal (None: the task's)
    is BrfsOptions::goal = search::any_of over ground conditions, each a list of (predicate, positive, objects);
    goal_hash = (m, r) makes it a custom goal test instead (GoalSpec::Custom): hash_state(state) % m == r;
    goal_atoms = k the custom test that the state has k true atoms."""
    if goal_atoms is not None:
        goal_hash = (0, int(goal_atoms))
    custom = 3 if goal_atoms is not None else 2
    if goal_hash is not None:
        goal = []
    W = task.table_words
    st = None if start is None else np.ascontiguousarray(np.asarray(start, np.uint64).reshape(-1)[:W])
    bl = None if blocked_states is None else np.ascontiguousarray(np.asarray(blocked_states, np.uint64).reshape(-1, W))
    go, gl = goal_records(goal) if goal is not None and goal_hash is None else (None, None)
    if callable(layer_order):
        score = layer_order

        def call(_u, rows, n, words, out):
            v = np.asarray(score(np.ctypeslib.as_array(rows, shape=(n, words)).copy()), np.float64).reshape(-1)
            for i in range(n):
                out[i] = float(v[i])

        kind, cb = 5, SCORER(call)
    else:
        kind, cb = LAYER_KINDS[layer_order], SCORER()
    o = BrfsOptions(threads, max_depth, max_states, int(witness_pruning), int(canonical_order), int(stop_at_goal), int(fingerprint),
                    max_expanded, _p(st), _p(bl), 0 if bl is None else bl.shape[0], W, 0, max_seconds,
                    0 if goal is None else (custom if goal_hash is not None else 1), 0 if goal is None or goal_hash is not None else len(goal),
                    _p(go), _p(gl), kind, int(not prefer_more_satisfied_goals),
                    seed, max_next_layer_states or 0, beam_width or 0, int(randomize_ties), int(record_events), cb, None,
                    goal_hash[0] if goal_hash else 0, goal_hash[1] if goal_hash else 0)
    r = BrfsResult()
    lc = np.zeros((4096, 3), dtype=np.uint64)
    L = max(1, task.label_width)
    cap = 4096
    ps = np.zeros(cap, np.int32)
    pb = np.zeros((cap, L), np.int32)
    gs = np.zeros(max(1, task.words, (task.dense_fluent + 63) // 64) + 64, np.uint64)
    n = lib().mref_brfs(task._h, ctypes.byref(o), ctypes.byref(r), lc.ctypes.data, 4096, ps.ctypes.data, pb.ctypes.data, L, cap,
                        gs.ctypes.data, gs.size)
    if n < 0:
        raise RuntimeError(_err())
    out = {
        "states": r.states, "expanded": r.expanded, "generated": r.generated, "goal_states": r.goal_states,
        "fingerprint": r.fingerprint, "layers": r.layers, "status": r.status, "solved": bool(r.solved),
        "exhausted": bool(r.exhausted), "seconds": r.seconds, "layer_counts": lc[:n].tolist(), "pruned": r.pruned,
        "words": r.words, "fluent_slots": r.fluent_slots, "threads_used": r.threads_used, "store": r.store.decode(),
        "message": r.message.decode(),
    }
    del st, bl, go, gl
    if record_events:
        ne = lib().mref_brfs_events(None, 0)
        ev = np.zeros((ne, 7), np.uint64)
        lib().mref_brfs_events(ev.ctypes.data, ne)
        out["events"] = ev
    task.refresh()
    if r.solved:
        k = min(r.plan_len, cap)
        out["plan"] = [[int(ps[i])] + [int(x) for x in pb[i] if x >= 0] for i in range(k)]
        out["cost"] = r.cost
        out["goal_state"] = [f"{int(x):016x}" for x in gs[:min(r.goal_words, gs.size)]]
    return out


class RefPool:
    """The reference CpuEnvPool (rl/pool.hpp:114-172) over one task: reset, send, recv, recv_ticket, pending. Batches come
    back as dicts of numpy arrays in the reference's PoolBatch field names."""

    STEP_FIELDS = ("reward", "truncated", "invalid", "final_states", "schema", "binding")

    def __init__(self, task: RefTask, num_envs: int, threads: int = 4, first_env: int = 0, **cfg):
        c = EnvConfig(cfg.get("seed", 0), cfg.get("max_steps", 0) or 0, cfg.get("step_reward", 0.0), cfg.get("goal_reward", 1.0),
                      cfg.get("dead_end_reward", 0.0), 1 if cfg.get("dead_end") == "none" else 0, int(cfg.get("dead_end_terminal", True)),
                      int(cfg.get("autoreset", True)), 1, 0, 0)
        h = lib().mref_pool_create(task._h, ctypes.byref(c), num_envs, threads, first_env)
        if not h:
            raise RuntimeError(_err())
        self._h = c_void_p(h)
        self.N, self.W, self.L = num_envs, task.table_words, max(1, task.label_width)

    def _out(self):
        N, W, L = self.N, self.W, self.L
        a = {"env_ids": np.zeros(N, np.uint32), "states": np.zeros((N, W), np.uint64), "task_ids": np.zeros(N, np.int32),
             "count": np.zeros(N, np.int32), "steps": np.zeros(N, np.int32), "at_goal": np.zeros(N, np.uint8),
             "terminated": np.zeros(N, np.uint8), "goal": np.zeros(N, np.uint8), "reward": np.zeros(N, np.float32),
             "truncated": np.zeros(N, np.uint8), "invalid": np.zeros(N, np.uint8), "final_states": np.zeros((N, W), np.uint64),
             "schema": np.zeros(N, np.int32), "binding": np.zeros((N, L), np.int32)}
        o = PoolOut(N, W, L, *[a[n].ctypes.data for n in ("env_ids", "states", "task_ids", "count", "steps", "at_goal", "terminated", "goal",
                                                           "reward", "truncated", "invalid", "final_states", "schema", "binding")])
        return a, o

    @staticmethod
    def _ids(env_ids):
        return None if env_ids is None else np.ascontiguousarray(env_ids, np.uint32)

    def _batch(self, a, rows, step):
        keys = [k for k in a if step or k not in self.STEP_FIELDS]
        return {k: a[k][:rows].copy() for k in keys}

    def reset(self, env_ids=None) -> dict:
        ids = self._ids(env_ids)
        a, o = self._out()
        n = lib().mref_pool_reset(self._h, _p(ids), 0 if ids is None else ids.size, ctypes.byref(o))
        if n < 0:
            raise RuntimeError(_err())
        return self._batch(a, n, False)

    def send(self, env_ids=None, actions=None) -> int:
        ids = self._ids(env_ids)
        act = None if actions is None else np.ascontiguousarray(actions, np.int64)
        t = lib().mref_pool_send(self._h, _p(ids), 0 if ids is None else ids.size, _p(act))
        if t < 0:
            raise RuntimeError(_err())
        return t

    def recv(self, min_rows: int = 0) -> dict:
        a, o = self._out()
        n = lib().mref_pool_recv(self._h, min_rows, ctypes.byref(o))
        if n < 0:
            raise RuntimeError(_err())
        return self._batch(a, n, True)

    def recv_ticket(self, ticket: int) -> dict:
        a, o = self._out()
        n = lib().mref_pool_recv_ticket(self._h, ticket, ctypes.byref(o))
        if n < 0:
            raise RuntimeError(_err())
        return self._batch(a, n, True)

    @property
    def pending(self) -> int:
        return int(lib().mref_pool_pending(self._h))

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib().mref_pool_free(h)
            self._h = c_void_p()


def dedup_flat(rows: np.ndarray) -> tuple[int, float]:
    """Unique count and insert seconds of the reference FlatStateStore over rows [n, words] (one thread)."""
    rows = np.ascontiguousarray(rows, dtype=np.uint64)
    u, s = c_uint64(), c_double()
    if lib().mref_dedup_flat(rows.ctypes.data, rows.shape[0], rows.shape[1], ctypes.byref(u), ctypes.byref(s)) != 0:
        raise RuntimeError(_err())
    return u.value, s.value


def dedup_concurrent(rows: np.ndarray, threads: int, batch: int = 1 << 20) -> tuple[int, float]:
    """Unique count and insert seconds of the reference ConcurrentStateStore over rows [n, words] on `threads`
    threads, in batches of `batch` rows."""
    rows = np.ascontiguousarray(rows, dtype=np.uint64)
    u, s = c_uint64(), c_double()
    if lib().mref_dedup_concurrent(rows.ctypes.data, rows.shape[0], rows.shape[1], threads, batch, ctypes.byref(u), ctypes.byref(s)) != 0:
        raise RuntimeError(_err())
    return u.value, s.value


def hash_words(w: np.ndarray, seed: int = 0x2D358DCCAA6C78A5) -> int:
    w = np.ascontiguousarray(w, dtype=np.uint64)
    return int(lib().mref_hash_words(w.ctypes.data, w.size, seed))


def hash_state(w: np.ndarray) -> int:
    w = np.ascontiguousarray(w, dtype=np.uint64)
    return int(lib().mref_hash_state(w.ctypes.data, w.size))


def hash_rows(rows: np.ndarray, words: int | None = None) -> np.ndarray:
    """hash::state of every row of a [n, W] array (its first `words` words; default all), uint64 [n]."""
    rows = np.ascontiguousarray(rows, dtype=np.uint64)
    n, W = rows.shape
    out = np.zeros(n, np.uint64)
    lib().mref_hash_rows(rows.ctypes.data, n, W if words is None else words, W, out.ctypes.data)
    return out


def philox(seed: int, env: int, draw: int, purpose: int = 0) -> list[int]:
    out = np.zeros(4, dtype=np.uint32)
    lib().mref_philox(seed, env, draw, purpose, out.ctypes.data)
    return [int(x) for x in out]


def successor_index(seed: int, env: int, draw: int, count: int) -> int:
    return int(lib().mref_successor_index(seed, env, draw, count))
