"""Batched environments on the device: the drop-in for the reference's ``rl.CpuEnvPool`` (python/src/rl_bindings.cpp:
2465-2600, include/mymyr/rl/pool.hpp:114-172) and its device env (include/mymyr/cuda/env.hpp), with the same keyword
arguments and defaults (seed 0, step_reward 0, goal_reward 1, dead_end "no_successors", autoreset True,
canonical_order True, witness_pruning False, first_env 0).

Every array lives on the device as a torch tensor (uint64 state words are carried as int64 tensors with the same
bits); step() runs on torch's current stream and returns views of the pool's own buffers (a PoolBatch-like dict), which
the next call overwrites, as the reference's recycled batches.
"""

from __future__ import annotations

import ctypes
from typing import Optional

import numpy as np
import torch

from . import _lib
from ._lib import check, lib
from .task import Task


def _stream() -> int:
    return _lib.current_stream()


def _p(t: torch.Tensor | None):
    return None if t is None else t.data_ptr()


def visited_capacity(track_visited: bool | int, max_steps: int | None) -> int:
    """The capacity of an env's visited tables (python/src/py_pool.hpp:17-35): False 0; True the next power of two at
    least 2 * (max_steps + 1) (max_steps in [1, 524287]); an int must be a power of two in [2, 2^20]."""
    if isinstance(track_visited, bool):
        if not track_visited:
            return 0
        if not max_steps or max_steps > (1 << 19) - 1:
            raise ValueError("mymyr: track_visited=True needs max_steps in [1, 524287]; pass an explicit capacity otherwise")
        H = 2
        while H < 2 * (max_steps + 1):
            H *= 2
        return H
    H = int(track_visited)
    if H < 2 or H > (1 << 20) or (H & (H - 1)):
        raise ValueError("mymyr: track_visited must be a power of two in [2, 2^20]")
    return H


def _checked_weights(weights, n: int) -> tuple:
    """The weights as floats, one per instance, finite and nonnegative with a positive sum (the reference's messages)."""
    w = np.asarray(weights, np.float64)
    if w.shape != (n,):
        raise ValueError("mymyr: sampling weights need one value per instance")
    ok = bool(np.isfinite(w).all()) and not bool((w < 0).any()) and bool((w > 0).any())
    if not ok:
        raise ValueError("mymyr: sampling weights must be finite, nonnegative and have a positive sum")
    return tuple(float(x) for x in w)


def _draw_tables(weights) -> tuple[np.ndarray, np.ndarray]:
    """The instances of positive weight and the cumulative thresholds over 2^32 between them that rl::rng::instance_draw
    compares a draw against (include/mymyr/rl/rng.hpp:94-115); the float64 steps (weights over their maximum, each
    over the sum, the running sum, scaled by 2^32 and floored) must match the reference's bit for bit. None (uniform):
    empty tables."""
    if weights is None:
        return np.empty(0, np.int32), np.empty(0, np.uint32)
    w = np.asarray(weights, np.float64)
    kept = np.flatnonzero(w > 0).astype(np.int32)
    scaled = w[kept] / w.max()
    running = np.cumsum(scaled / scaled.sum())[:-1]
    return kept, np.minimum(np.floor(running * 2**32), 0xFFFFFFFF).astype(np.uint32)


class InstanceSampler:
    """Draws the instance an env resets into (mymyr.rl.InstanceSampler, python/mymyr/rl/_sampling.py:16-104; the draw
    is rl::rng::instance_draw, include/mymyr/rl/rng.hpp:94-115): uniform over num_instances, or weighted by `weights`
    (finite, nonnegative, positive sum), as cumulative thresholds over 2^32 of the instances of positive weight."""

    def __init__(self, num_instances: int, weights=None):
        if not 1 <= num_instances <= 0x7FFFFFFF:
            raise ValueError("mymyr: instance sampling needs between 1 and 2**31 - 1 instances")
        self.num_instances = num_instances
        self.weights = None if weights is None else _checked_weights(weights, num_instances)
        self.indices, self.thresholds = _draw_tables(self.weights)

    def sample(self, seed: int, env_id: int, reset_count: int) -> int:
        """The instance of env `env_id`'s draw number `reset_count` under `seed` (host)."""
        thr = np.ascontiguousarray(self.thresholds)
        idx = np.ascontiguousarray(self.indices)
        return int(lib.mya_instance_draw(seed & 0xFFFFFFFFFFFFFFFF, env_id, reset_count & 0xFFFFFFFF, self.num_instances,
                                         thr.ctypes.data, idx.ctypes.data, len(idx)))


class PoolBatch(dict):
    """The results of one or more sends, or of a reset (PoolBatch, include/mymyr/rl/pool.hpp:92-112): device tensors of
    B rows in the order of their env ids, under the reference's field names (env_ids, states, task_ids, count, steps,
    at_goal, goal, terminated and, for a send's batch, reward, truncated, invalid, final_states, schema, binding,
    revisited; goal_pos / goal_neg with per-env goals); the fields are also attributes. `step` tells a send's batch
    from a reset's; `rows`, `words` and `label_width` give its shape."""

    def __init__(self, fields: dict, rows: int, words: int, label_width: int, step: bool, goals: bool):
        super().__init__(fields)
        self.rows, self.words, self.label_width, self.step, self.goals = rows, words, label_width, step, goals

    def __getattr__(self, name):
        try:
            return self[name]
        except KeyError:
            raise AttributeError(name) from None


_SAMPLER_ARG = "mymyr: sampler must be 'auto', 'uniform', an InstanceSampler or None"


def resolve_sampler(sampler, instances: int, *, auto_uniform: bool = True, mismatch: str | None = None) -> InstanceSampler | None:
    """The instance sampling a `sampler` argument asks for, with the reference's rules and messages
    (python/mymyr/rl/_sampling.py:153-163): "uniform" samples uniformly, "auto" too unless `auto_uniform` is off (a
    BatchedEnv given task ids), None not at all, and an InstanceSampler as it is if it covers the `instances`; a
    table of one instance never samples. `mismatch`: the message for a sampler over another number of instances."""
    if isinstance(sampler, InstanceSampler):
        if sampler.num_instances != instances:
            raise ValueError(mismatch or f"mymyr: env: a sampler over {sampler.num_instances} instances for {instances}")
        chosen = sampler
    elif sampler is None:
        chosen = None
    elif not isinstance(sampler, str):
        raise TypeError(_SAMPLER_ARG)
    elif sampler == "uniform" or (sampler == "auto" and auto_uniform):
        chosen = InstanceSampler(instances)
    elif sampler == "auto":
        chosen = None
    else:
        raise ValueError(_SAMPLER_ARG)
    return chosen if instances > 1 else None


class DeviceEnvPool:
    """num_envs environments over one task, or over a task table (a list of instances of one domain: TaskTable,
    include/mymyr/rl/task_table.hpp:1-28), stepped together on the device (random policy unless actions are given).
    Over a table every env has an instance ("task_ids", int32 [num_envs], initially `task_ids` or all 0) and its rows
    are the widest instance's words; reset(task_ids=...) moves envs to other instances and step(next_task_ids=...)
    names the instance an autoresetting env restarts in."""

    def __init__(self, task: Task | list[Task], num_envs: int, *, seed: int = 0, max_steps: int | None = None, step_reward: float = 0.0,
                 goal_reward: float = 1.0, dead_end: str = "no_successors", dead_end_reward: float = 0.0,
                 dead_end_terminal: bool = True, autoreset: bool = True, canonical_order: bool = True,
                 witness_pruning: bool = False, first_env: int = 0, words: int | None = None, device: str | int = "cuda",
                 count_cache: bool = True, goals: bool = False, task_ids=None, sampler: InstanceSampler | str | None = None,
                 env_ids=None, seeds=None, sampling_seeds=None, reset_counts: bool | None = None, track_visited: bool | int = False):
        if num_envs < 1 or num_envs > 0x7FFFFFFF:
            raise ValueError("mymyr: num_envs must be in [1, 2^31 - 1]")
        if dead_end not in ("no_successors", "none"):
            raise ValueError("mymyr: dead_end must be 'no_successors' or 'none'")
        suite = isinstance(task, TaskSuite)
        if isinstance(task, TaskTable):
            task = task.tasks
        self.tasks = list(task) if isinstance(task, (list, tuple)) else [task]
        if not self.tasks:
            raise ValueError("mymyr: TaskTable: no instances")
        self.task = self.tasks[0]
        self.num_schemas = max(t.num_schemas for t in self.tasks)
        self.num_envs = num_envs
        self.first_env = first_env
        widest = max(t.words for t in self.tasks)
        self.words = widest if words is None else words
        if self.words < widest:
            raise ValueError(f"mymyr: env: state rows of {self.words} words; the task needs {widest}")
        self.label_width = max(1, max(t.label_width for t in self.tasks))
        self.device = torch.device(device)
        self._dead_end_none = dead_end == "none"
        self._dead_end_terminal = bool(dead_end_terminal)
        self._busy = np.zeros(num_envs, bool)  # envs with a send not yet received
        self._sends = []  # (ticket, env ids, batch, event) in send order
        self._next_ticket = 0
        self._spare = {}  # rows -> recycled output arrays
        cfg = _lib.EnvConfig(seed, max_steps or 0, step_reward, goal_reward, dead_end_reward, 1 if dead_end == "none" else 0,
                             int(dead_end_terminal), int(autoreset), int(canonical_order), int(witness_pruning), 0)
        h = ctypes.c_void_p()
        handles = (ctypes.c_void_p * len(self.tasks))(*[t.handle.value for t in self.tasks])
        create = lib.mya_env_create_suite if suite else lib.mya_env_create_table
        check(create(handles, len(self.tasks), ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h
        N, W, L, dev = num_envs, self.words, self.label_width, self.device
        self.states = torch.zeros((N, W), dtype=torch.int64, device=dev)
        self.steps = torch.zeros(N, dtype=torch.int32, device=dev)
        self.draws = torch.zeros(N, dtype=torch.int64, device=dev)
        self.at_goal = torch.zeros(N, dtype=torch.uint8, device=dev)
        self.count = torch.zeros(N, dtype=torch.int32, device=dev)
        self.reward = torch.zeros(N, dtype=torch.float32, device=dev)
        self.terminated = torch.zeros(N, dtype=torch.uint8, device=dev)
        self.truncated = torch.zeros(N, dtype=torch.uint8, device=dev)
        self.goal = torch.zeros(N, dtype=torch.uint8, device=dev)
        self.invalid = torch.zeros(N, dtype=torch.uint8, device=dev)
        self.schema = torch.zeros(N, dtype=torch.int32, device=dev)
        self.binding = torch.zeros((N, L), dtype=torch.int32, device=dev)
        self.final_states: torch.Tensor | None = None
        # the count cache (the reference device env's EnvBatch::counts): per-schema successor counts of each row's
        # state plus its fingerprint, so a step counts only the reached states; zeros match no state
        self.counts_cache = (torch.zeros((N, self.num_schemas + 2), dtype=torch.int32, device=dev) if count_cache else None)
        # per-env goal masks (goals=True, CpuEnvPool's `goals`): goal_pos / goal_neg [N, W], the task's goal after a reset
        self.goal_pos = torch.zeros((N, W), dtype=torch.int64, device=dev) if goals else None
        self.goal_neg = torch.zeros((N, W), dtype=torch.int64, device=dev) if goals else None
        # each env's instance (a table of several instances only)
        self.task_ids = None
        if len(self.tasks) > 1:
            self.task_ids = torch.zeros(N, dtype=torch.int32, device=dev)
            if task_ids is not None:
                self.task_ids.copy_(torch.as_tensor(task_ids, dtype=torch.int32))
        # per-row RNG keys and env ids (EnvBatch::seeds / env_ids), the sampler's per-row keys and reset counters
        # (EnvBatch::sampling_seeds / reset_counts; on by default with a sampler)
        def as_dev(a, unsigned, signed):  # unsigned words carried in a signed tensor with the same bits
            if a is None:
                return None
            if isinstance(a, torch.Tensor):
                return a.to(device=dev, dtype=torch.int64 if signed is np.int64 else torch.int32).contiguous()
            return torch.from_numpy(np.ascontiguousarray(np.asarray(a).astype(unsigned)).view(signed)).to(dev)

        self.seeds = as_dev(seeds, np.uint64, np.int64)
        self.env_ids = as_dev(env_ids, np.uint32, np.int32)
        self.sampling_seeds = as_dev(sampling_seeds, np.uint64, np.int64)
        for name, t in (("seeds", self.seeds), ("env_ids", self.env_ids), ("sampling_seeds", self.sampling_seeds)):
            if t is not None and t.shape != (N,):
                raise ValueError(f"mymyr: env: {name} must have shape ({N},)")
        sampler = resolve_sampler(sampler, len(self.tasks))
        self.reset_counts = None
        if reset_counts or (reset_counts is None and sampler is not None):
            self.reset_counts = torch.zeros(N, dtype=torch.int32, device=dev)
        self.sampler = sampler
        if sampler is not None:
            thr = np.ascontiguousarray(sampler.thresholds)
            idx = np.ascontiguousarray(sampler.indices)
            check(lib.mya_env_set_sampling(self._h, sampler.num_instances, thr.ctypes.data, idx.ctypes.data, len(idx)))
        # visited tables (track_visited: rl/visited.hpp): keys [N, H] (uint64 bits in int64), counts [N], sticky status [1]
        H = visited_capacity(track_visited, max_steps)
        self.visited = torch.zeros((N, H), dtype=torch.int64, device=dev) if H else None
        self.visited_count = torch.zeros(N, dtype=torch.int32, device=dev) if H else None
        self.visited_status = torch.zeros(1, dtype=torch.int32, device=dev) if H else None
        self.revisited = torch.zeros(N, dtype=torch.uint8, device=dev) if H else None
        self._batch = _lib.EnvBatch(self.states.data_ptr(), N, W, 0, self.steps.data_ptr(), self.draws.data_ptr(),
                                    self.at_goal.data_ptr(), first_env, _p(self.counts_cache), _p(self.goal_pos),
                                    _p(self.goal_neg), _p(self.task_ids), _p(self.seeds), _p(self.env_ids), _p(self.reset_counts),
                                    _p(self.sampling_seeds), _p(self.visited), _p(self.visited_count), _p(self.visited_status), H, 0)

    def initial_count(self, instance: int = 0) -> tuple[int, bool]:
        c = ctypes.c_uint32()
        g = ctypes.c_uint8()
        check(lib.mya_env_initial_count(self._h, instance, ctypes.byref(c), ctypes.byref(g)))
        return c.value, bool(g.value)

    def reset(self, mask: torch.Tensor | None = None, keep_goals: bool = False, task_ids=None, sample: bool = False, *,
              env_ids=None, goal_pos=None, goal_neg=None) -> PoolBatch:
        """Resets every env, those with mask != 0, or the envs env_ids to the initial state of its instance
        (HostEnv::reset, include/mymyr/rl/env.hpp:208-219); draws are kept, reset counters advance. task_ids (over a
        table) first sets the instances of the envs being reset (per env of env_ids, or over the whole batch with a
        mask); sample=True draws them from the sampler instead. With per-env goals the instance's goal is written into
        goal_pos / goal_neg unless keep_goals or goal masks are given (per env of env_ids; at_goal is their test on the
        initial state). Returns the observations as a PoolBatch: the reset envs' rows in env_ids order, or views of the
        whole batch."""
        if self._busy.any():
            raise ValueError("mymyr: DeviceEnvPool.reset: envs have a step in flight (recv first)")
        ids = None
        if env_ids is not None:
            if mask is not None:
                raise ValueError("mymyr: DeviceEnvPool.reset: give a mask or env ids, not both")
            ids = self._env_ids_arg(env_ids, "reset")
            mask = torch.zeros(self.num_envs, dtype=torch.uint8, device=self.device)
            mask[ids] = 1
        if mask is not None:
            mask = mask.to(device=self.device, dtype=torch.uint8).contiguous()
        if (goal_pos is None) != (goal_neg is None):
            raise ValueError("mymyr: CpuEnvPool.reset: goals need both goal_pos and goal_neg")
        if goal_pos is not None:
            if self.goal_pos is None:
                raise ValueError("mymyr: CpuEnvPool.reset: goal masks given, but the pool has no per-env goals")
            rows = ids if ids is not None else torch.arange(self.num_envs, device=self.device)
            for dst, src in ((self.goal_pos, goal_pos), (self.goal_neg, goal_neg)):
                g = torch.as_tensor(np.ascontiguousarray(src).view(np.int64) if isinstance(src, np.ndarray) else src).to(self.device)
                g = g.view(torch.int64) if g.dtype == torch.uint64 else g
                if g.dim() != 2 or g.shape[0] != rows.numel() or g.shape[1] > self.words:
                    raise ValueError("mymyr: CpuEnvPool.reset: goal masks must be [n, W] with W at most the pool's words")
                full = torch.zeros((rows.numel(), self.words), dtype=torch.int64, device=self.device)
                full[:, : g.shape[1]] = g
                dst.index_copy_(0, rows, full)
            keep_goals = True
        if task_ids is not None:
            if self.task_ids is None:
                raise ValueError("mymyr: env: task ids need a table of several instances")
            tid = torch.as_tensor(task_ids, dtype=torch.int32).to(self.device)
            if ids is not None:
                if tid.shape != (ids.numel(),):
                    raise ValueError(f"mymyr: CpuEnvPool.reset: task_ids must have shape ({ids.numel()},)")
                self.task_ids.index_copy_(0, ids, tid)
            elif mask is None:
                self.task_ids.copy_(tid)
            else:
                self.task_ids.copy_(torch.where(mask != 0, tid, self.task_ids))
        check(lib.mya_env_reset(self._h, ctypes.byref(self._batch), _p(mask), self.count.data_ptr(), int(keep_goals), int(sample),
                                _stream()))
        goal = self.at_goal
        dead_end_terminal = not self._dead_end_none and self._dead_end_terminal
        term = (goal != 0) | ((self.count == 0) & dead_end_terminal)
        r = {"env_ids": torch.arange(self.num_envs, dtype=torch.int32, device=self.device), "states": self.states,
             "task_ids": self.task_ids if self.task_ids is not None else self._zero_ids(), "count": self.count, "steps": self.steps,
             "at_goal": self.at_goal, "goal": goal, "terminated": term.to(torch.uint8)}
        if self.reset_counts is not None:
            r["reset_counts"] = self.reset_counts
        if self.goal_pos is not None:
            r["goal_pos"] = self.goal_pos
            r["goal_neg"] = self.goal_neg
        if ids is not None:
            r = {k: (v.index_select(0, ids) if k != "env_ids" else ids.to(torch.int32)) for k, v in r.items()}
        n = self.num_envs if ids is None else ids.numel()
        return PoolBatch(r, n, self.words, self.label_width, False, self.goal_pos is not None)

    def step(self, env_ids=None, actions=None, *, next_task_ids=None, final_states: bool = False, labels: bool = True,
             encode: int = 0) -> PoolBatch:
        """One step of every env (env_ids None: in place, the returned arrays are views that the next step overwrites) or
        of envs env_ids (send + recv_ticket: the reference pool's step). actions [n] int64 indices into the canonical
        successor order (None: the random policy). next_task_ids [n] (over a table): the instance each autoresetting env
        restarts in. encode > 0 (whole-batch steps) also emits the observed states' true-atom slots ("atoms", int32
        [num_envs, encode], -1 padded) and applicable-schema masks ("masks", uint8 [num_envs, num_schemas]), both in
        library-owned device buffers taken over DLPack."""
        if env_ids is not None:
            if encode:
                raise ValueError("mymyr_amd: DeviceEnvPool.step: the encoding outputs come with whole-batch steps")
            return self.recv_ticket(self.send(env_ids, actions, next_task_ids=next_task_ids))
        if self._busy.any():
            raise ValueError("mymyr: CpuEnvPool.send: envs have a step in flight (recv first)")
        if actions is not None:
            actions = torch.as_tensor(actions).to(device=self.device, dtype=torch.int64).contiguous()
            if actions.shape != (self.num_envs,):
                raise ValueError(f"mymyr: env: actions must have shape ({self.num_envs},)")
        if final_states and self.final_states is None:
            self.final_states = torch.zeros((self.num_envs, self.words), dtype=torch.int64, device=self.device)
        fs = self.final_states if final_states else None
        atoms = masks = None
        if encode:
            if getattr(self, "_atoms", None) is None or self._atoms.shape[1] != encode:
                self._atoms, self._masks = self._encoding_outputs(encode)
            atoms, masks = self._atoms, self._masks
        out = _lib.StepOutputs(self.reward.data_ptr(), self.terminated.data_ptr(), self.truncated.data_ptr(), self.count.data_ptr(),
                               _p(fs), self.schema.data_ptr() if labels else None, self.binding.data_ptr() if labels else None,
                               self.label_width, self.words, self.invalid.data_ptr(), self.goal.data_ptr(), _p(atoms), _p(masks),
                               encode, 0)
        nxt = self._next_ids_arg(next_task_ids, self.num_envs)
        out.revisited = _p(self.revisited)
        check(lib.mya_env_step(self._h, ctypes.byref(self._batch), ctypes.byref(out), _p(actions), _p(nxt), _stream()))
        r = {"env_ids": self._all_ids(), "states": self.states, "reward": self.reward, "terminated": self.terminated,
             "truncated": self.truncated, "count": self.count, "steps": self.steps, "at_goal": self.at_goal, "goal": self.goal,
             "invalid": self.invalid, "task_ids": self.task_ids if self.task_ids is not None else self._zero_ids()}
        if self.revisited is not None:
            r["revisited"] = self.revisited
        if labels:
            r["schema"] = self.schema
            r["binding"] = self.binding
        if fs is not None:
            r["final_states"] = fs
        if encode:
            r["atoms"] = atoms
            r["masks"] = masks
        if self.goal_pos is not None:
            r["goal_pos"] = self.goal_pos
            r["goal_neg"] = self.goal_neg
        return PoolBatch(r, self.num_envs, self.words, self.label_width, True, self.goal_pos is not None)

    # ---- the reference pool's asynchronous API (CpuEnvPool send / recv / recv_ticket / recycle / pending,
    # include/mymyr/rl/pool.hpp:114-172). A send steps its envs on the device at once, in stream order: their rows are
    # gathered into a batch of their own (each keeping its env id's RNG and instance streams, so the results are those
    # of stepping them with the whole batch), stepped by the HIP env step, and the envs' state is written back; the
    # batch's arrays are the send's results. recv hands them out in send order.

    def _all_ids(self) -> torch.Tensor:
        if getattr(self, "_arange", None) is None:
            self._arange = torch.arange(self.num_envs, dtype=torch.int32, device=self.device)
        return self._arange

    def _zero_ids(self) -> torch.Tensor:
        if getattr(self, "_zeros", None) is None:
            self._zeros = torch.zeros(self.num_envs, dtype=torch.int32, device=self.device)
        return self._zeros

    def _env_ids_arg(self, env_ids, what: str) -> torch.Tensor:
        """env_ids as a device int64 tensor, checked: each an env of the pool, at most once, none in flight."""
        a = env_ids.detach().cpu().numpy() if isinstance(env_ids, torch.Tensor) else np.asarray(env_ids)
        a = a.astype(np.int64).reshape(-1)
        if a.size and (a.min() < 0 or a.max() >= self.num_envs):
            raise ValueError(f"mymyr: CpuEnvPool.{what}: env id out of range [0, {self.num_envs})")
        if np.unique(a).size != a.size:
            raise ValueError(f"mymyr: CpuEnvPool.{what}: an env id is repeated")
        if self._busy[a].any():
            raise ValueError(f"mymyr: CpuEnvPool.{what}: env {int(a[self._busy[a]][0])} has a step in flight")
        return torch.from_numpy(a).to(self.device)

    def _next_ids_arg(self, next_task_ids, rows: int):
        if next_task_ids is None:
            return None
        if self.task_ids is None:
            raise ValueError("mymyr: env: next_task_ids needs a table of several instances")
        nxt = torch.as_tensor(next_task_ids, dtype=torch.int32).to(self.device).contiguous()
        if nxt.shape != (rows,):
            raise ValueError(f"mymyr: env: next_task_ids must have shape ({rows},)")
        return nxt

    def _batch_arrays(self, B: int) -> dict:
        """The output arrays of a send of B rows: recycled ones of that size, or new."""
        spare = self._spare.get(B)
        if spare:
            return spare.pop()
        dev, W, L = self.device, self.words, self.label_width
        a = {"reward": torch.empty(B, dtype=torch.float32, device=dev), "terminated": torch.empty(B, dtype=torch.uint8, device=dev),
             "truncated": torch.empty(B, dtype=torch.uint8, device=dev), "count": torch.empty(B, dtype=torch.int32, device=dev),
             "final_states": torch.empty((B, W), dtype=torch.int64, device=dev), "schema": torch.empty(B, dtype=torch.int32, device=dev),
             "binding": torch.empty((B, L), dtype=torch.int32, device=dev), "invalid": torch.empty(B, dtype=torch.uint8, device=dev),
             "goal": torch.empty(B, dtype=torch.uint8, device=dev)}
        if self.revisited is not None:
            a["revisited"] = torch.empty(B, dtype=torch.uint8, device=dev)
        return a

    def send(self, env_ids=None, actions=None, *, next_task_ids=None) -> int:
        """Enqueues one step of envs env_ids [n] (None: every env) and returns its ticket at once: actions [n] (indices into
        the canonical successor order; None: the random policy), next_task_ids [n] (over a table: the instances
        autoresetting envs restart in). Raises for an unknown or repeated env id or one with a step in flight."""
        if env_ids is None:
            if self._busy.any():
                raise ValueError("mymyr: CpuEnvPool.send: envs have a step in flight (recv first)")
            ids = torch.arange(self.num_envs, dtype=torch.int64, device=self.device)
        else:
            ids = self._env_ids_arg(env_ids, "send")
        B = ids.numel()
        act = None
        if actions is not None:
            act = torch.as_tensor(np.asarray(actions) if not isinstance(actions, torch.Tensor) else actions)
            act = act.to(device=self.device, dtype=torch.int64).contiguous()
            if act.shape != (B,):
                raise ValueError(f"mymyr: CpuEnvPool.send: actions must have shape ({B},)")
        nxt = self._next_ids_arg(next_task_ids, B)
        out = self._batch_arrays(B)
        # the envs' rows as a batch of their own: their env ids carry their RNG streams
        sub = {"states": self.states.index_select(0, ids), "steps": self.steps.index_select(0, ids),
               "draws": self.draws.index_select(0, ids), "at_goal": self.at_goal.index_select(0, ids)}
        rng_ids = self.env_ids.index_select(0, ids) if self.env_ids is not None else (ids + self.first_env).to(torch.int32)
        opt = {}
        for name in ("counts_cache", "goal_pos", "goal_neg", "task_ids", "seeds", "reset_counts", "sampling_seeds", "visited",
                     "visited_count"):
            t = getattr(self, name)
            opt[name] = t.index_select(0, ids) if t is not None else None
        H = 0 if self.visited is None else self.visited.shape[1]
        batch = _lib.EnvBatch(sub["states"].data_ptr(), B, self.words, 0, sub["steps"].data_ptr(), sub["draws"].data_ptr(),
                              sub["at_goal"].data_ptr(), self.first_env, _p(opt["counts_cache"]), _p(opt["goal_pos"]),
                              _p(opt["goal_neg"]), _p(opt["task_ids"]), _p(opt["seeds"]), rng_ids.data_ptr(), _p(opt["reset_counts"]),
                              _p(opt["sampling_seeds"]), _p(opt["visited"]), _p(opt["visited_count"]), _p(self.visited_status), H, 0)
        so = _lib.StepOutputs(out["reward"].data_ptr(), out["terminated"].data_ptr(), out["truncated"].data_ptr(),
                              out["count"].data_ptr(), out["final_states"].data_ptr(), out["schema"].data_ptr(), out["binding"].data_ptr(),
                              self.label_width, self.words, out["invalid"].data_ptr(), out["goal"].data_ptr(), None, None, 0, 0)
        so.revisited = _p(out.get("revisited"))
        if B:
            check(lib.mya_env_step(self._h, ctypes.byref(batch), ctypes.byref(so), _p(act), _p(nxt), _stream()))
        # the envs' state back into the pool
        for name, t in sub.items():
            getattr(self, name).index_copy_(0, ids, t)
        for name, t in opt.items():
            if t is not None and name not in ("seeds", "sampling_seeds"):
                getattr(self, name).index_copy_(0, ids, t)
        res = dict(out)
        res.update({"env_ids": ids.to(torch.int32), "states": sub["states"], "steps": sub["steps"], "at_goal": sub["at_goal"],
                    "task_ids": opt["task_ids"] if opt["task_ids"] is not None else torch.zeros(B, dtype=torch.int32, device=self.device)})
        if opt["goal_pos"] is not None:
            res["goal_pos"], res["goal_neg"] = opt["goal_pos"], opt["goal_neg"]
        ev = torch.cuda.Event()
        ev.record()
        ticket = self._next_ticket
        self._next_ticket += 1
        idx = ids.cpu().numpy()
        self._busy[idx] = True
        self._sends.append((ticket, idx, PoolBatch(res, B, self.words, self.label_width, True, opt["goal_pos"] is not None), ev))
        return ticket

    def _collect(self, taken: list) -> PoolBatch:
        for _, idx, _, ev in taken:
            ev.synchronize()
            self._busy[idx] = False
        if len(taken) == 1:
            return taken[0][2]
        parts = [t[2] for t in taken]
        cat = {k: torch.cat([p[k] for p in parts]) for k in parts[0]}
        return PoolBatch(cat, sum(p.rows for p in parts), self.words, self.label_width, True, parts[0].goals)

    def recv(self, min_rows: int = 0) -> PoolBatch:
        """The results of the oldest pending sends, in send order: whole sends with at least min_rows rows together
        (0: exactly one send). Blocks until they are done; raises if fewer rows are pending."""
        taken, rows = [], 0
        for s in self._sends:
            taken.append(s)
            rows += s[2].rows
            if rows >= min_rows:
                break
        if not taken or rows < min_rows:
            raise ValueError(f"mymyr: CpuEnvPool.recv: {rows} rows pending, {max(min_rows, 1)} asked for (send first)")
        del self._sends[: len(taken)]
        return self._collect(taken)

    def recv_ticket(self, ticket: int) -> PoolBatch:
        """The results of the send with this ticket (blocks until it is done)."""
        for k, s in enumerate(self._sends):
            if s[0] == ticket:
                del self._sends[k]
                return self._collect([s])
        raise ValueError(f"mymyr: CpuEnvPool.recv: no pending send has ticket {ticket}")

    def recycle(self, batch: PoolBatch) -> None:
        """Hands a send's batch back: a later send of as many rows fills its arrays instead of allocating new ones."""
        if not isinstance(batch, PoolBatch) or not batch.step:
            return
        keys = ("reward", "terminated", "truncated", "count", "final_states", "schema", "binding", "invalid", "goal", "revisited")
        arrays = {k: batch[k] for k in keys if k in batch}
        self._spare.setdefault(batch.rows, []).append(arrays)

    @property
    def pending(self) -> int:
        """Sends not yet received."""
        return len(self._sends)

    def _encoding_outputs(self, encode: int) -> tuple[torch.Tensor, torch.Tensor]:
        """The atom-index and mask outputs live in library-owned device buffers that torch takes over DLPack without a
        copy (the reference's pool arrays are DLPack-exported blocks, python/src/arrays.cpp:100-235)."""
        from .dlpack import DeviceBuffer
        S = max(1, self.num_schemas)
        with torch.cuda.device(self.device):
            ab = DeviceBuffer(self.num_envs * encode * 4)
            mb = DeviceBuffer(self.num_envs * S)
            atoms = torch.from_dlpack(ab.array("int32", (self.num_envs, encode)))
            masks = torch.from_dlpack(mb.array("uint8", (self.num_envs, S)))
        ab.release()
        mb.release()
        return atoms, masks

    def encode_atoms(self, states: torch.Tensor, max_atoms: int) -> torch.Tensor:
        """True-atom slots of each row, ascending, -1 padded (int32 [rows, max_atoms])."""
        s = states.view(torch.int64) if states.dtype == torch.uint64 else states.contiguous()
        out = torch.empty((s.shape[0], max_atoms), dtype=torch.int32, device=s.device)
        check(lib.mya_encode_atoms(self._h, s.data_ptr(), s.shape[0], s.shape[1], out.data_ptr(), max_atoms, _stream()))
        return out

    def schema_masks(self, states: torch.Tensor) -> torch.Tensor:
        """Per row and schema, whether some binding is applicable (uint8 [rows, num_schemas])."""
        s = states.view(torch.int64) if states.dtype == torch.uint64 else states.contiguous()
        out = torch.empty((s.shape[0], max(1, self.task.num_schemas)), dtype=torch.uint8, device=s.device)
        check(lib.mya_schema_masks(self._h, s.data_ptr(), s.shape[0], s.shape[1], out.data_ptr(), _stream()))
        return out

    def refresh(self) -> torch.Tensor:
        """Recomputes at_goal and the count cache from the current states after they were written directly
        (DeviceEnv::refresh); returns the successor counts."""
        check(lib.mya_env_refresh(self._h, ctypes.byref(self._batch), self.count.data_ptr(), _stream()))
        return self.count

    def clear_visited(self, mask: torch.Tensor | None = None) -> None:
        """The visited tables of every env (or those with mask != 0) hold their current states' keys only
        (HostEnv::clear_visited); the overflow status is kept."""
        if self.visited is None:
            return
        if mask is not None:
            mask = mask.to(device=self.device, dtype=torch.uint8).contiguous()
        check(lib.mya_env_clear_visited(self._h, ctypes.byref(self._batch), _p(mask), _stream()))

    def check(self) -> None:
        """Raises if a step set the device's sticky error status."""
        check(lib.mya_env_check(self._h))

    def __del__(self):
        h = getattr(self, "_h", None)
        try:
            if h is not None and h.value:
                lib.mya_env_free(h)
                self._h = ctypes.c_void_p()
        except Exception:
            pass


class EnvPool(DeviceEnvPool):
    """The reference's rl.CpuEnvPool on the device (python/src/rl_bindings.cpp:2465-2600, include/mymyr/rl/pool.hpp:
    114-172): num_envs envs over a task, a TaskTable or a TaskSuite, with its keyword arguments and defaults. reset(
    env_ids, task_ids), send(env_ids, actions) / recv(min_rows) / recv_ticket(ticket), step(env_ids, actions) =
    send + recv_ticket, recycle(batch) and pending behave as the reference pool's, with batches of device tensors
    (PoolBatch). sampler ("auto" and "uniform": uniform over the instances, an InstanceSampler, or None) places every
    env in a sampled instance and restarts it in its next one on each reset without task_ids and each autoreset
    without next_task_ids, with the draws of the reference pool (seed, env id first_env + e, reset counter).
    `threads` is accepted for the reference's signature (the device steps every env of a send at once); batch rows are
    the widest instance's words (the reference's PoolOptions::words)."""

    def __init__(self, table, num_envs: int, *, threads: int = 1, goals: bool = False, seed: int = 0, max_steps: int | None = None,
                 step_reward: float = 0.0, goal_reward: float = 1.0, dead_end: str = "no_successors", dead_end_reward: float = 0.0,
                 dead_end_terminal: bool = True, autoreset: bool = True, canonical_order: bool = True, witness_pruning: bool = False,
                 framework=None, words: int | None = None, sampler="auto", track_visited: bool | int = False, first_env: int = 0,
                 device: str | int = "cuda"):
        if framework not in (None, "torch"):
            raise ValueError("mymyr_amd: EnvPool: batches are device tensors (framework None or 'torch')")
        n = len(table.tasks) if isinstance(table, TaskTable) else len(table) if isinstance(table, (list, tuple)) else 1
        super().__init__(table, num_envs, seed=seed, max_steps=max_steps, step_reward=step_reward, goal_reward=goal_reward,
                         dead_end=dead_end, dead_end_reward=dead_end_reward, dead_end_terminal=dead_end_terminal, autoreset=autoreset,
                         canonical_order=canonical_order, witness_pruning=witness_pruning, first_env=first_env, words=words,
                         device=device, goals=goals, sampler=resolve_sampler(sampler, n), track_visited=track_visited)
        self.threads = threads
        self.seed = seed
        self.max_steps = max_steps
        self.dead_end = dead_end
        self.goals = goals
        self.table = table
        self.framework = framework  # the reference's framework argument (batches are device tensors either way)
        self.numeric_words = 0      # classical tasks: no numeric words after the atom words
        if self.sampler is not None:
            # every env starts in a sampled instance (the draw of its reset counter 0, which then stands at 1)
            check(lib.mya_env_reset(self._h, ctypes.byref(self._batch), None, self.count.data_ptr(), 0, 1, _stream()))

    def reset(self, env_ids=None, task_ids=None, *, goal_pos=None, goal_neg=None) -> PoolBatch:
        """Resets envs env_ids [n] (None: every env) into instances task_ids [n] (None: sampled ones, or their current
        ones without a sampler) with goal masks goal_pos / goal_neg [n, W] (per-env goals only; None: their instances'
        goals); returns their observations. Draw counters are kept. Raises if one of them has a step in flight."""
        sample = task_ids is None and self.sampler is not None
        if env_ids is None and goal_pos is None:
            return super().reset(task_ids=task_ids, sample=sample)
        ids = np.arange(self.num_envs) if env_ids is None else env_ids
        return super().reset(env_ids=ids, task_ids=task_ids, sample=sample, goal_pos=goal_pos, goal_neg=goal_neg)

    def step(self, env_ids=None, actions=None, *, next_task_ids=None) -> PoolBatch:
        """send + recv_ticket: one step of envs env_ids (None: every env), its results."""
        return self.recv_ticket(self.send(env_ids, actions, next_task_ids=next_task_ids))


def successors(task: Task, states: torch.Tensor, cap: int = 4096) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor]:
    """Canonical successor listing of each row (witness pruning off): (count [n], schema [n, cap], binding [n, cap, L],
    rows [n, cap, words]); entries past count are unspecified."""
    s = states.view(torch.int64) if states.dtype == torch.uint64 else states
    if not s.is_cuda or s.dim() != 2:
        raise ValueError("mymyr_amd: successors: states must be a 2-d device tensor")
    s = s.contiguous()
    n, w = s.shape
    L = max(1, task.label_width)
    count = torch.zeros(n, dtype=torch.int32, device=s.device)
    schema = torch.full((n, cap), -1, dtype=torch.int32, device=s.device)
    binding = torch.full((n, cap, L), -1, dtype=torch.int32, device=s.device)
    rows = torch.zeros((n, cap, w), dtype=torch.int64, device=s.device)
    check(lib.mya_successors(task.handle, s.data_ptr(), n, w, cap, count.data_ptr(), schema.data_ptr(), binding.data_ptr(),
                             rows.data_ptr(), _stream()))
    return count, schema, binding, rows


class TaskTable:
    """Instances of one domain batched together (rl.TaskTable, include/mymyr/rl/task_table.hpp:1-28): created only if
    every task has instance 0's action schemas and predicates in the same order; rows are the widest instance's words
    and labels the largest schema arity wide. The table lives in a device env handle (the reference's default env
    configuration), which table expansions run on."""

    def __init__(self, tasks: list[Task]):
        self.tasks = list(tasks)
        if not self.tasks:
            raise ValueError("mymyr: TaskTable: no instances")
        cfg = _lib.EnvConfig(0, 0, 0.0, 1.0, 0.0, 0, 1, 1, 1, 0, 0)
        handles = (ctypes.c_void_p * len(self.tasks))(*[t.handle.value for t in self.tasks])
        h = ctypes.c_void_p()
        check(lib.mya_env_create_table(handles, len(self.tasks), ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h
        self.num_instances = len(self.tasks)
        self.words = max(t.words for t in self.tasks)
        self.label_width = max(t.label_width for t in self.tasks)
        self.num_schemas = self.tasks[0].num_schemas

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def __del__(self):
        h = getattr(self, "_h", None)
        try:
            if h is not None and h.value:
                lib.mya_env_free(h)
                self._h = ctypes.c_void_p()
        except Exception:
            pass


class TaskSuite(TaskTable):
    """Instances of several domains batched together (rl.TaskSuite.group, include/mymyr/rl/task_suite.hpp:1-30):
    global ids in the tasks' order, each instance's labels in its own domain's schemas and objects; rows the widest
    instance's words, labels the largest arity wide, count caches and masks the most schemas of any instance."""

    def __init__(self, tasks: list[Task]):
        self.tasks = list(tasks)
        if not self.tasks:
            raise ValueError("mymyr: TaskSuite: no instances")
        cfg = _lib.EnvConfig(0, 0, 0.0, 1.0, 0.0, 0, 1, 1, 1, 0, 0)
        handles = (ctypes.c_void_p * len(self.tasks))(*[t.handle.value for t in self.tasks])
        h = ctypes.c_void_p()
        check(lib.mya_env_create_suite(handles, len(self.tasks), ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h
        self.num_instances = len(self.tasks)
        self.words = max(t.words for t in self.tasks)
        self.label_width = max(t.label_width for t in self.tasks)
        self.num_schemas = max(t.num_schemas for t in self.tasks)


def expand(task: Task | TaskTable, states: torch.Tensor, *, task_ids: torch.Tensor | None = None, capacity: int | None = None,
           goal: bool = False, hashes: bool = False, noops: bool = False, drop_noops: bool = False, index: bool = False,
           validate: bool = True, words: int | None = None, witness_pruning: bool = False) -> dict:
    """The flat expansion of states [N, W] on the device (rl.expand, include/mymyr/rl/expand.hpp:1-130): successor rows
    "succ" [M, words], "parent", "schema" [M] int32, "binding" [M, label_width] int32 (-1 padded), "offsets" [N + 1]
    int32, with goal=True "goal" [M] uint8, hashes=True "succ_hash" [M] (uint64 bits in int64), noops=True "noop" [M]
    uint8, and "index" [M] int32 (the position in the parent's full successor order) with drop_noops or index=True;
    plus "generated", "total", "words_needed" and "overflow". capacity None sizes the buffers to every successor (a
    first call counts them). Canonical order; witness_pruning keeps one successor per effect-relevant binding of a schema
    with witness parameters (the binding the reference's matcher finds first; one task only, as the reference's default
    is off); drop_noops removes a state's no-op successors unless all of them are no-ops. Over a TaskTable, row i is a
    state of instance task_ids[i] ([N] int32 on the device).
    A task with lazy slots interns the atoms its successors add without a slot (ascending canonical id); with words
    None the rows then take the task's new width (the expansion runs once more when its successors outgrew them)."""
    s = states.view(torch.int64) if states.dtype == torch.uint64 else states
    if not s.is_cuda or s.dim() != 2 or s.dtype != torch.int64:
        raise ValueError("mymyr_amd: expand: states must be a 2-d int64/uint64 device tensor")
    s = s.contiguous()
    rows, w = s.shape
    table = isinstance(task, TaskTable)
    ids = None
    if table:
        if task_ids is not None:
            ids = torch.as_tensor(task_ids).to(device=s.device, dtype=torch.int32).contiguous()
            if ids.shape != (rows,):
                raise ValueError(f"mymyr: expand: task_ids must have shape ({rows},)")
    elif task_ids is not None:
        raise ValueError("mymyr: expand: task ids need a TaskTable")
    ow = task.words if words is None else words
    L = max(1, task.label_width)
    opts = _lib.ExpandOptions(1, int(witness_pruning), int(validate), int(drop_noops))

    def run(x):
        if table:
            check(lib.mya_env_expand(task.handle, s.data_ptr(), _p(ids), rows, w, ctypes.byref(opts), ctypes.byref(x), _stream()))
        else:
            check(lib.mya_expand(task.handle, s.data_ptr(), rows, w, ctypes.byref(opts), ctypes.byref(x), _stream()))

    if capacity is None:
        probe = _lib.Expansion()
        run(probe)
        capacity = probe.generated
    dev = s.device
    cap = int(capacity)
    succ = torch.zeros((cap, ow), dtype=torch.int64, device=dev)
    parent = torch.empty(cap, dtype=torch.int32, device=dev)
    schema = torch.empty(cap, dtype=torch.int32, device=dev)
    binding = torch.empty((cap, L), dtype=torch.int32, device=dev)
    offsets = torch.empty(rows + 1, dtype=torch.int32, device=dev)
    gl = torch.empty(cap, dtype=torch.uint8, device=dev) if goal else None
    sh = torch.empty(cap, dtype=torch.int64, device=dev) if hashes else None
    np_ = torch.empty(cap, dtype=torch.uint8, device=dev) if noops else None
    ix = torch.empty(cap, dtype=torch.int32, device=dev) if (drop_noops or index) else None
    x = _lib.Expansion(cap, ow, L, succ.data_ptr(), parent.data_ptr(), schema.data_ptr(), binding.data_ptr(), _p(gl),
                       offsets.data_ptr(), _p(sh), _p(np_), _p(ix), 0, 0, 0, 0)
    run(x)
    if words is None and not table and not task.frozen and x.words_needed > ow:
        # lazy slots grew the rows: their atoms have slots now, so the successors fit rows of the task's new width
        return expand(task, states, capacity=cap, goal=goal, hashes=hashes, noops=noops, drop_noops=drop_noops, index=index,
                      validate=validate, words=max(task.words, int(x.words_needed)), witness_pruning=witness_pruning)
    kept = min(x.total, cap)
    out = {"succ": succ[:kept], "parent": parent[:kept], "schema": schema[:kept], "binding": binding[:kept],
           "offsets": offsets, "generated": x.generated, "total": x.total, "words_needed": x.words_needed,
           "overflow": x.generated > cap or x.total > cap or x.words_needed > ow, "capacity": cap}
    for name, t in (("goal", gl), ("succ_hash", sh), ("noop", np_), ("index", ix)):
        if t is not None:
            out[name] = t[:kept]
    return out


def auto_k(offsets: torch.Tensor) -> int:
    """The k of pad(k=None): the next power of two at or above the largest successor count (at least 1)."""
    m = int((offsets[1:] - offsets[:-1]).max()) if offsets.numel() > 1 else 0
    return 1 << (max(m, 1) - 1).bit_length()


def pad(flat: dict, k: int | None = None, *, words: int | None = None, label_width: int | None = None) -> dict:
    """The padded [N, k] view of a flat expansion of expand() (rl::pad, src/mymyr/rl/expand.cpp:799-873), scattered on
    the device: "index" [N, k] int32 (flat row, -1 padding), "mask" [N, k] uint8, "count" [N] int32 (true counts, which
    may exceed k), "succ" [N, k, words] (zero padding), "schema" [N, k] (-1), "binding" [N, k, label_width] (-1), and
    "goal", "succ_hash", "noop" (0 padding) and "canonical" (the flat "index", -1 padding) when the flat expansion has
    them; "overflow" is set by a count above k, a successor past the flat capacity or the flat expansion's own
    overflow. k None sizes k to the next power of two at or above the largest count."""
    offsets = flat["offsets"]
    rows = offsets.numel() - 1
    if k is None:
        k = auto_k(offsets)
    if k < 0:
        raise ValueError("mymyr: pad: k must be non-negative")
    fw, fl = flat["succ"].shape[1], flat["binding"].shape[1]
    ow = fw if words is None else words
    L = fl if label_width is None else label_width
    dev = offsets.device
    out = {"index": torch.empty((rows, k), dtype=torch.int32, device=dev), "mask": torch.empty((rows, k), dtype=torch.uint8, device=dev),
           "count": torch.empty(rows, dtype=torch.int32, device=dev), "succ": torch.empty((rows, k, ow), dtype=torch.int64, device=dev),
           "schema": torch.empty((rows, k), dtype=torch.int32, device=dev),
           "binding": torch.empty((rows, k, L), dtype=torch.int32, device=dev)}
    for name, dt in (("goal", torch.uint8), ("succ_hash", torch.int64), ("noop", torch.uint8)):
        if name in flat:
            out[name] = torch.empty((rows, k), dtype=dt, device=dev)
    if "index" in flat:
        out["canonical"] = torch.empty((rows, k), dtype=torch.int32, device=dev)
    x = _lib.Expansion(flat["capacity"], fw, fl, flat["succ"].data_ptr(), flat["parent"].data_ptr(), flat["schema"].data_ptr(),
                       flat["binding"].data_ptr(), _p(flat.get("goal")), offsets.data_ptr(), _p(flat.get("succ_hash")),
                       _p(flat.get("noop")), _p(flat.get("index")), flat["generated"], flat["total"], flat["words_needed"], 0)
    p = _lib.PaddedExpansion(k, ow, L, 0, out["index"].data_ptr(), out["mask"].data_ptr(), out["count"].data_ptr(), out["succ"].data_ptr(),
                             out["schema"].data_ptr(), out["binding"].data_ptr(), _p(out.get("goal")), _p(out.get("succ_hash")),
                             _p(out.get("noop")), _p(out.get("canonical")), 0, 0)
    check(lib.mya_pad(ctypes.byref(x), rows, ctypes.byref(p), _stream()))
    out["k"] = k
    out["overflow"] = bool(p.overflow)
    return out


def visited_mask(table: torch.Tensor, count: torch.Tensor, succ_hash: torch.Tensor, parent: torch.Tensor,
                 rows: torch.Tensor | None = None) -> torch.Tensor:
    """Membership of successor hashes in visited tables (rl::visited_mask of include/mymyr/rl/visited.hpp:63-74) on the
    device, on the current stream without a host synchronization: out[j] = succ_hash[j] is in the table (table [n, H]
    int64/uint64, count [n] int32) of row parent[j], or of rows[parent[j]]; -1 is padding, and parents or rows outside
    the tables read as not visited. The same as torch.ops.mymyr.visited_mask (registered below with a fake
    implementation, so torch.compile traces it; python/mymyr/rl/torch/_ops.py:464-486)."""
    return torch.ops.mymyr.visited_mask(table, count, succ_hash, parent, rows)


@torch.library.custom_op("mymyr::visited_mask", mutates_args=())
def _visited_mask_op(table: torch.Tensor, count: torch.Tensor, succ_hash: torch.Tensor, parent: torch.Tensor,
                     rows: Optional[torch.Tensor]) -> torch.Tensor:
    if table.dim() != 2 or not table.is_cuda:
        raise ValueError("mymyr: visited_mask: table must be a 2-d device tensor")
    n, H = table.shape
    tab = table.view(torch.int64) if table.dtype == torch.uint64 else table
    h = succ_hash.view(torch.int64) if succ_hash.dtype == torch.uint64 else succ_hash
    if tab.dtype != torch.int64 or h.dtype != torch.int64:
        raise TypeError("mymyr: visited_mask: table and succ_hash must be int64 or uint64")
    for name, t in (("count", count), ("parent", parent)) + ((("rows", rows),) if rows is not None else ()):
        if t.dtype != torch.int32 or t.device != table.device:
            raise TypeError(f"mymyr: visited_mask: {name} must be an int32 tensor on the table's device")
    if count.shape != (n,) or parent.shape != h.shape or h.dim() != 1:
        raise ValueError("mymyr: visited_mask: count [n], succ_hash [size] and parent [size] expected")
    tab, h, count, parent = tab.contiguous(), h.contiguous(), count.contiguous(), parent.contiguous()
    rows = None if rows is None else rows.contiguous()
    out = torch.empty(h.shape, dtype=torch.bool, device=table.device)
    check(lib.mya_visited_mask(tab.data_ptr(), count.data_ptr(), n, H, h.data_ptr(), parent.data_ptr(), _p(rows),
                               0 if rows is None else rows.numel(), h.numel(), out.data_ptr(), _stream()))
    return out


@_visited_mask_op.register_fake
def _visited_mask_fake(table, count, succ_hash, parent, rows):
    return torch.empty(succ_hash.shape, dtype=torch.bool, device=succ_hash.device)


def label_actions(flat: dict, schema: torch.Tensor, binding: torch.Tensor) -> torch.Tensor:
    """The index form of label actions (HostEnv::step with Labels, src/mymyr/rl/env.cpp:376-426) on the device: int64
    [N], the position of row i's label (schema [N] int32, binding [N, L'] int32 with L' at least the expansion's label
    width; columns past the schema's arity are ignored) among its successors of the flat expansion `flat` (expand()
    without drop_noops and without a capacity limit), or -1 when the label is not applicable."""
    offsets = flat["offsets"]
    rows = offsets.numel() - 1
    L = flat["binding"].shape[1]
    if schema.shape != (rows,) or schema.dtype != torch.int32 or binding.dtype != torch.int32 or binding.dim() != 2 or binding.shape[0] != rows:
        raise ValueError(f"mymyr: label actions require schema int32 [{rows}] and binding int32 [{rows}, L] tensors")
    if flat["overflow"] or "index" in flat:
        raise ValueError("mymyr: label actions need a complete expansion without dropped no-ops")
    schema, binding = schema.contiguous(), binding.contiguous()
    out = torch.empty(rows, dtype=torch.int64, device=offsets.device)
    check(lib.mya_label_actions(offsets.data_ptr(), flat["schema"].data_ptr(), flat["binding"].data_ptr(), L, rows, schema.data_ptr(),
                                binding.data_ptr(), binding.shape[1], out.data_ptr(), _stream()))
    return out
