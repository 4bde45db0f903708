"""Fixture helpers shared by tests/golden/make_golden.py and the tests: file locations and the per-step digest of env
trajectories."""

from __future__ import annotations

import hashlib
import json
import os

import numpy as np

GOLDEN = os.path.dirname(os.path.abspath(__file__))
TASKS = os.path.join(GOLDEN, "tasks")

# suite tasks of the reference (tests/data/tasks) that the device path supports, with the reference's published
# exhaustive BrFS counts {states, generated (witness pruning on), goal_states} (tests/cpp/support/suite.hpp:33-56)
SUITE_COUNTS = {
    "gripper__prob05": (376832, 2031616, 2),
    "blocks__probBLOCKS-8-0": (695417, 2094752, 1),
    "logistics00__probLOGISTICS-6-1": (941192, 10487568, 8),
    "miconic__s7-4": (229376, 3153920, 1792),
    "visitall__visitall_x-6_y-3_r-100": (193456, 597411, 18),
    "sokoban-opt08-strips__p14": (348955, 866027, 27),
    "depot__p02": (40320, 376560, 9),
    "driverlog__p03": (348750, 2826000, 40),
    "zenotravel__p05": (1016064, 17224704, 784),
    "transport-opt08-strips__p23": (1185759, 6993720, 81),
    "snake-opt18-strips__p05": (1320037, 2200339, 88669),
    "parcprinter-opt11-strips__p03": (173942, 488868, 1),
    "pegsol-08-strips__p22": (99457, 189967, 2),
    "pathways__p02": (669078, 11237052, 12288),
    "freecell__p02": (159924, 1371273, 1),
    "folding-opt23-adl__p01": (148260, 170776, 1),
    "organic-synthesis-opt18-strips__p20": (41311, 52548, 24),
    "miconic-simpleadl__s10-2": (316680, 6333600, 20),
    "caldera-split-opt18-adl__p04": (468041, 630395, 4472),
}
# suite tasks with conditional effects: searched by the ground driver only (the lifted entry points refuse them)
CE_TASKS = ["miconic-simpleadl__s10-2", "caldera-split-opt18-adl__p04"]
# suite tasks outside the published counts whose slot tables are pinned too (rovers__p02's schemas have two witness
# parameters; its BrFS is pinned in brfs_witness.json)
LAYOUT_ONLY = ["rovers__p02"]

# layer scorers of the scored-layer fixtures (brfs_layers.json), by name; the tests pass the same functions to the
# device search. They depend on the number of set atoms only, so they score a state alike under every slot numbering.
LAYER_SCORERS = {
    "popcount": lambda rows: [sum(bin(int(w)).count("1") for w in r) for r in rows],
    "neg_popcount_mod3": lambda rows: [-(sum(bin(int(w)).count("1") for w in r) % 3) for r in rows],
}

# the reference's own determinism digests of search.brfs(max_states=20000, fingerprint=True, stop_at_goal=False):
# sha256(json.dumps([states, expanded, generated, layers, fingerprint], sort_keys=True))[:16]
# (tests/data/determinism.json, tests/python/test_determinism.py:63-104)
DETERMINISM_BRFS = {
    "blocks__probBLOCKS-8-0": "4a2c176284577ee8",
    "depot__p02": "a8bc749fad052dbe",
    "gripper__prob05": "393197c282f5c1d2",
    "logistics00__probLOGISTICS-6-1": "ab1c7b50f936cad0",
}


def determinism_digest(states, expanded, generated, layers, fingerprint) -> str:
    return hashlib.sha256(json.dumps([states, expanded, generated, layers, fingerprint], sort_keys=True).encode()).hexdigest()[:16]


def step_digest(n: int, states, reward, terminated, truncated, count, schema, binding, goal) -> str:
    """sha256 of the first n rows of one step's arrays, in a fixed order and dtype."""
    h = hashlib.sha256()
    for a, dt in ((states, np.uint64), (reward, np.float32), (terminated, np.uint8), (truncated, np.uint8), (count, np.int32),
                  (schema, np.int32), (binding, np.int32), (goal, np.uint8)):
        h.update(np.ascontiguousarray(np.asarray(a)[:n]).astype(dt, copy=False).tobytes())
    return h.hexdigest()[:16]


def rows_digest(row_hashes, reward, terminated, truncated, count, schema, binding, goal) -> str:
    """sha256 of one step over a whole batch: each row's state as its 64-bit state hash, then the other arrays, in a
    fixed order and dtype."""
    h = hashlib.sha256()
    for a, dt in ((row_hashes, np.uint64), (reward, np.float32), (terminated, np.uint8), (truncated, np.uint8),
                  (count, np.int32), (schema, np.int32), (binding, np.int32), (goal, np.uint8)):
        h.update(np.ascontiguousarray(np.asarray(a)).astype(dt, copy=False).tobytes())
    return h.hexdigest()[:16]


def load(name: str):
    with open(os.path.join(GOLDEN, name)) as f:
        return json.load(f)


def task_path(name: str) -> str:
    return os.path.join(TASKS, f"{name}.txt")


def arrays_digest(*arrays) -> str:
    """sha256 of the arrays' bytes in order (each as given: the caller fixes the dtypes)."""
    h = hashlib.sha256()
    for a in arrays:
        h.update(np.ascontiguousarray(np.asarray(a)).tobytes())
    return h.hexdigest()[:16]


# Task-table env trajectories (rl::HostEnv over TaskTable::create, src/mymyr/rl/env.cpp:179-255, 351-528): per-row
# instances, autoresets into the instances of next_task_ids or of an instance sampler (rl/sampling.hpp), masked resets
# that move rows to other instances or draw them, keep_goals resets with per-env goal masks, and per-row RNG keys and
# env ids. Every input of a case is drawn here from numpy's PCG64 with the case's seed, so the golden script, the
# oracle test and the device test replay the same trajectory.
TABLE_CASES = {
    "gridworld_ids": dict(table="gridworld_table", rows=48, steps=40, seed=21, policy="random",
                          env={"seed": 3, "max_steps": 14, "step_reward": -1.0, "goal_reward": 5.0}),
    "gridworld_goals": dict(table="gridworld_table", rows=48, steps=40, seed=22, policy="given", goals=True,
                            env={"seed": 4, "max_steps": 10, "step_reward": -0.5, "goal_reward": 2.0, "dead_end_reward": -3.0}),
    "transport_ids": dict(table="transport_table", rows=24, steps=16, seed=23, policy="random", goals=True,
                          env={"seed": 5, "max_steps": 6}),
    "gridworld_sampled": dict(table="gridworld_table", rows=40, steps=40, seed=26, policy="random", sampler="uniform", keys=True,
                              env={"seed": 8, "max_steps": 9, "step_reward": -1.0}),
    "transport_weighted": dict(table="transport_table", rows=24, steps=20, seed=27, policy="given", goals=True,
                               sampler=[2.0, 0.0, 1.0], keys=True, env={"seed": 9, "max_steps": 5}),
    "gridworld_large": dict(table="gridworld_table", rows=4096, steps=96, seed=24, policy="random",
                            env={"seed": 6, "max_steps": 30, "step_reward": -1.0, "goal_reward": 0.0}),
    "transport_large": dict(table="transport_table", rows=2048, steps=48, seed=25, policy="given", goals=True,
                            env={"seed": 7, "max_steps": 16}),
    "gridworld_many": dict(table="gridworld_many", rows=96, steps=40, seed=29, policy="random", sampler="uniform",
                           env={"seed": 11, "max_steps": 12, "step_reward": -1.0, "goal_reward": 3.0}),
    "gridworld_many_large": dict(table="gridworld_many", rows=8192, steps=48, seed=30, policy="given", goals=True,
                                 env={"seed": 12, "max_steps": 25}),
    "suite_mixed": dict(table="mixed_suite", suite=True, rows=40, steps=30, seed=31, policy="random", sampler="uniform", goals=True,
                        env={"seed": 13, "max_steps": 8, "step_reward": -1.0, "goal_reward": 2.0}),
    "suite_mixed_large": dict(table="mixed_suite", suite=True, rows=4096, steps=40, seed=32, policy="given", sampler=[1.0, 2.0, 1.0, 3.0, 1.0],
                              env={"seed": 14, "max_steps": 12}),
    "gridworld_visited": dict(table="gridworld_table", rows=40, steps=40, seed=33, policy="random", visited=8,
                              env={"seed": 15, "max_steps": 30, "step_reward": -1.0}),
    "transport_visited": dict(table="transport_table", rows=24, steps=24, seed=34, policy="given", visited=16, goals=True,
                              env={"seed": 16, "max_steps": 10, "autoreset": False}),
    "gridworld_visited_large": dict(table="gridworld_table", rows=4096, steps=48, seed=35, policy="random", visited=64, sampler="uniform",
                                    env={"seed": 17, "max_steps": 40}),
    "gridworld_sampled_large": dict(table="gridworld_table", rows=4096, steps=64, seed=28, policy="random", sampler=[1.0, 3.0, 2.0],
                                    keys=True, env={"seed": 10, "max_steps": 20}),
}
# cases small enough for the oracle's pure-Python restatement
TABLE_ORACLE_CASES = ["gridworld_ids", "gridworld_goals", "transport_ids", "gridworld_sampled", "transport_weighted", "gridworld_many",
                      "suite_mixed", "gridworld_visited", "transport_visited"]


def sampler_arrays(weights) -> tuple[np.ndarray, np.ndarray]:
    """An instance sampler's arrays from its weights (mymyr.rl.InstanceSampler, python/mymyr/rl/_sampling.py:29-39):
    indices = the instances of positive weight, thresholds = the cumulative distribution of their weights (scaled by the
    largest) over 2^32, without its last entry. Uniform (None): both empty."""
    if weights is None:
        return np.empty(0, np.uint32), np.empty(0, np.int32)
    w = np.asarray(weights, np.float64)
    idx = np.flatnonzero(w > 0).astype(np.int32)
    positive = w[idx] / w.max()
    cum = np.cumsum(positive / positive.sum())[:-1]
    return np.minimum(np.floor(cum * 2**32), 0xFFFFFFFF).astype(np.uint32), idx


def case_sampler(case: str, instances: int):
    """(instances, thresholds, indices) of the case's sampler, or None."""
    spec = TABLE_CASES[case].get("sampler")
    if spec is None:
        return None
    thr, idx = sampler_arrays(None if spec == "uniform" else spec)
    return instances, thr, idx


def table_inputs(case: str, instances: int) -> dict:
    """The inputs of a table case: initial task ids, per step the next_task_ids (even steps without a sampler; None
    otherwise) and the uniforms behind the given actions, the masked resets (step -> (mask, new task ids, keep_goals,
    sample)), and with `keys` the per-row RNG keys, env ids and sampling keys."""
    c = TABLE_CASES[case]
    rows, steps, goals, sampler = c["rows"], c["steps"], c.get("goals", False), c.get("sampler")
    rng = np.random.default_rng(c["seed"])
    out = {"task_ids": rng.integers(0, instances, rows, dtype=np.int32), "next": [], "u": []}
    for k in range(steps):
        nxt = rng.integers(0, instances, rows, dtype=np.int32)
        given = k % 2 == 0 if sampler is None else k % 4 == 1
        out["next"].append(nxt if given else None)
        out["u"].append(rng.random(rows))
    resets = {}
    m = rng.random(rows) < 0.25
    resets[steps // 2] = (m.astype(np.uint8), rng.integers(0, instances, rows, dtype=np.int32), False, False)
    if goals:
        m = rng.random(rows) < 0.25
        resets[steps // 4] = (m.astype(np.uint8), None, True, False)
    if sampler is not None:
        m = rng.random(rows) < 0.4
        resets[3 * steps // 4] = (m.astype(np.uint8), None, False, True)
    out["resets"] = resets
    out["clears"] = {}
    if c.get("visited"):
        out["clears"][steps // 3] = (rng.random(rows) < 0.3).astype(np.uint8)
    if c.get("keys"):
        out["seeds"] = rng.integers(0, 2**63, rows, dtype=np.int64).view(np.uint64)
        out["env_ids"] = rng.integers(0, 2**32, rows, dtype=np.uint64).astype(np.uint32)
        out["sampling_seeds"] = rng.integers(0, 2**63, rows, dtype=np.int64).view(np.uint64)
    return out


# table cases whose batch, after step TABLE_EXPAND_STEP, is also expanded by rl::expand over the table
# (include/mymyr/rl/expand.hpp:133-150), with and without drop_noops
TABLE_EXPAND_CASES = ["gridworld_ids", "transport_ids", "gridworld_many", "transport_large", "suite_mixed", "suite_mixed_large"]
TABLE_EXPAND_STEP = 5


def expansion_digest(x: dict) -> str:
    """sha256 of a flat expansion's arrays in a fixed order and dtype (succ, parent, schema, binding, goal, succ_hash,
    noop, index, offsets)."""
    return arrays_digest(np.asarray(x["succ"], np.uint64), np.asarray(x["parent"], np.int32), np.asarray(x["schema"], np.int32),
                         np.asarray(x["binding"], np.int32), np.asarray(x["goal"], np.uint8), np.asarray(x["succ_hash"], np.uint64),
                         np.asarray(x["noop"], np.uint8), np.asarray(x["index"], np.int32), np.asarray(x["offsets"], np.int32))


def pad_ks(offsets) -> tuple:
    """The k a table expansion is padded to: the automatic one (the next power of two at or above the largest count)
    and 3 (below most counts: overflow and cut rows)."""
    off = np.asarray(offsets, np.int64)
    m = int((off[1:] - off[:-1]).max()) if len(off) > 1 else 0
    return (1 << (max(m, 1) - 1).bit_length(), 3)


def padded_digest(p: dict) -> str:
    """sha256 of a padded expansion's arrays in a fixed order and dtype (index, mask, count, succ, schema, binding, goal,
    succ_hash, noop, canonical)."""
    return arrays_digest(np.asarray(p["index"], np.int32), np.asarray(p["mask"], np.uint8), np.asarray(p["count"], np.int32),
                         np.asarray(p["succ"], np.uint64), np.asarray(p["schema"], np.int32), np.asarray(p["binding"], np.int32),
                         np.asarray(p["goal"], np.uint8), np.asarray(p["succ_hash"], np.uint64), np.asarray(p["noop"], np.uint8),
                         np.asarray(p["canonical"], np.int32))


def table_state(b: dict) -> list:
    """The batch arrays a table case's digests cover, in order (those the batch has)."""
    keys = ("states", "task_ids", "steps", "draws", "at_goal", "goal_pos", "goal_neg", "reset_counts", "visited", "visited_count",
            "visited_status")
    return [b[k] for k in keys if b.get(k) is not None]


def given_actions(u, count) -> np.ndarray:
    """The given policy's actions: uniform over [-1, count] (so some are invalid: -1 and count)."""
    c = np.asarray(count, np.int64)
    return np.floor(np.asarray(u) * (c + 2)).astype(np.int64) - 1


# The dedup workload at its stated size: 2^26 rows of 16 words from the seeded stream (seed 0, 30% duplicates), inserted
# in 2^20-row batches. Its exact unique count is the number of the stream's fresh rows (a duplicate copies an earlier
# row, which resolves to a fresh one); tests/test_oracle.py recounts it from the generator's closed form.
DEDUP_WORKLOAD = {"rows": 1 << 26, "words": 16, "seed": 0, "dup": 0.3, "batch": 1 << 20, "unique": 46975112}


# The pool's asynchronous API (CpuEnvPool reset / send / recv / recv_ticket, include/mymyr/rl/pool.hpp:114-172) over a
# scripted sequence of calls: resets of all and of some envs, sends of subsets (shuffled env ids, given actions with
# invalid ones among them, the random policy), received whole (recv), several at once (recv with min_rows) and by ticket.
# The calls are drawn here from the case's seed, so the golden script and the device test make the same ones; every
# batch a call returns is recorded as a digest of its arrays in PoolBatch order.
POOL_CASES = {
    "gridworld": {"num_envs": 256, "first_env": 3, "rounds": 24, "seed": 41,
                  "env": {"seed": 7, "max_steps": 12, "step_reward": -1.0, "goal_reward": 2.0}},
    "transport": {"num_envs": 192, "first_env": 0, "rounds": 16, "seed": 43, "env": {"seed": 1}},
}

POOL_FIELDS = (("env_ids", np.uint32), ("states", np.uint64), ("task_ids", np.int32), ("count", np.int32), ("steps", np.int32),
               ("at_goal", np.uint8), ("terminated", np.uint8), ("goal", np.uint8))
POOL_STEP_FIELDS = (("reward", np.float32), ("truncated", np.uint8), ("invalid", np.uint8), ("final_states", np.uint64),
                    ("schema", np.int32), ("binding", np.int32))


def pool_batch_digest(b, step: bool, label_width: int) -> str:
    """Digest of a pool batch (a mapping of arrays: numpy, or tensors with .cpu()) in PoolBatch field order."""
    def arr(k, dt):
        a = b[k]
        a = a.cpu().numpy() if hasattr(a, "cpu") else np.asarray(a)
        if k == "binding":
            a = a[:, :label_width]
        return np.ascontiguousarray(a).view(dt) if a.dtype.itemsize == np.dtype(dt).itemsize else a.astype(dt)
    fields = POOL_FIELDS + (POOL_STEP_FIELDS if step else ())
    return arrays_digest(*[arr(k, dt) for k, dt in fields])


def pool_script(case: str) -> list:
    """The calls of a pool case: ("reset", ids | None), ("send", ids | None, actions | None), ("recv", min_rows) and
    ("recv_ticket", k) for the k-th send. Each round sends some idle envs and receives every pending send; only idle
    envs are sent or reset."""
    c = POOL_CASES[case]
    N = c["num_envs"]
    rng = np.random.default_rng(c["seed"])
    calls = [("reset", None)]
    busy = np.zeros(N, bool)
    pending = []  # (send index, ids or None: every env), in send order
    nsend = 0
    for r in range(c["rounds"]):
        kind = r % 4
        if kind == 3 and r % 8 == 3:
            calls.append(("send", None, None))
            pending.append((nsend, None))
            nsend += 1
            busy[:] = True
        else:
            for _ in range(1 + int(rng.integers(0, 3))):
                idle = np.flatnonzero(~busy)
                if idle.size == 0:
                    break
                take = max(1, int(rng.integers(1, idle.size + 1)) // 2)
                ids = rng.permutation(idle)[:take]
                busy[ids] = True
                acts = rng.integers(-1, 5, ids.size) if kind == 1 else None
                calls.append(("send", ids.tolist(), None if acts is None else acts.tolist()))
                pending.append((nsend, ids))
                nsend += 1
        while pending:
            if kind == 2 and len(pending) > 1:
                calls.append(("recv_ticket", pending.pop(-1)[0]))  # a later send first
            elif kind == 0 and len(pending) > 1:
                rows = sum(N if ids is None else ids.size for _, ids in pending[:2])
                calls.append(("recv", rows))  # the two oldest sends together
                pending = pending[2:]
            else:
                pending.pop(0)
                calls.append(("recv", 0))
        busy[:] = False
        if r % 5 == 4:
            calls.append(("reset", rng.permutation(N)[: int(rng.integers(1, N // 3))].tolist()))
    return calls


def run_pool_script(pool, case: str, label_width: int) -> list:
    """Digests of the batches the calls of a pool case return, on a pool with the reference's reset / send / recv /
    recv_ticket methods (env ids and actions as numpy arrays)."""
    out = []
    tickets = []
    for call in pool_script(case):
        if call[0] == "reset":
            ids = None if call[1] is None else np.asarray(call[1], np.uint32)
            out.append(pool_batch_digest(pool.reset(ids), False, label_width))
        elif call[0] == "send":
            ids = None if call[1] is None else np.asarray(call[1], np.uint32)
            acts = None if call[2] is None else np.asarray(call[2], np.int64)
            tickets.append(pool.send(ids, acts))
        elif call[0] == "recv":
            out.append(pool_batch_digest(pool.recv(call[1]), True, label_width))
        else:
            out.append(pool_batch_digest(pool.recv_ticket(tickets[call[1]]), True, label_width))
    return out

