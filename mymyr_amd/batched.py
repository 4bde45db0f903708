"""BatchedEnv: N planning environments whose state lives in torch tensors on the device, stepped by the HIP env (the
drop-in for the reference's ``mymyr.rl.torch.BatchedEnv``, python/mymyr/rl/torch/_batched.py:115-600, and its
``CapturedRollout``, python/mymyr/rl/torch/_graph.py).

The environments' tensors are ``states`` [N, row_words] int64 (the widest instance's words), ``task_ids`` [N] int32,
``steps`` [N] int32, ``draws`` [N] int64, ``reset_counts`` [N] int32 (the sampler's counters, uint32 bits), ``count``
[N] int32, ``at_goal`` [N] bool, ``counts`` (the count cache) and, with ``goals=True``, ``goal_pos`` / ``goal_neg``
[N, words] int64. reset, refresh and step run on torch's current stream and write them in place, so they keep their
addresses: loops of steps capture into HIP graphs (:meth:`BatchedEnv.capture`, or ``torch.cuda.graph`` around the
calls). Writing ``states``, ``task_ids`` or the goal masks directly needs :meth:`BatchedEnv.refresh`.

The reference's observation encoders are not part of this path; asking for them raises NotImplementedError. Label
actions (``actions="label"``, ``step((schema, binding))``) move each row by its label where the label is applicable in
the row's state (else the row is invalid), in the step kernel itself, so label steps are captured like index steps;
counts are 0/1 in label mode. Visited tables (``track_visited``) are kept on the device: ``visited`` [N, H] int64, ``visited_count``
[N] int32, ``visited_status`` [1] int32.
"""

from __future__ import annotations

import ctypes
from typing import Any, Callable, NamedTuple, Optional

import numpy as np
import torch
from torch import Tensor

from . import _lib, rl
from ._lib import check, lib
from .rl import InstanceSampler, TaskSuite, TaskTable, resolve_sampler, visited_capacity
from .task import Task

__all__ = ["BatchedEnv", "CapturedRollout", "Observation", "Rollout", "StepResult"]


class Observation(NamedTuple):
    """Policy inputs, owned copies by default (``BatchedEnv.observation(copy=False)`` borrows the live tensors)."""

    states: Tensor
    task_ids: Tensor
    count: Tensor
    goal_pos: Tensor
    goal_neg: Tensor
    at_goal: Tensor  # bool: the state is a goal; the next step absorbs it
    encoding: Any = None
    actions: Any = None
    action_visited: Any = None


class StepResult(NamedTuple):
    """The outputs of one :meth:`BatchedEnv.step` and the next observation. ``final_states`` are the reached states
    before the autoreset ([N, row_words] with final=True, else [0, row_words]); goal masks are [N, 0] without goals."""

    reward: Tensor  # float32
    terminated: Tensor  # bool
    truncated: Tensor  # bool
    goal: Tensor  # bool: the reached state is a goal
    invalid: Tensor  # bool: an out-of-range action in a nonterminal, non-stuck row
    schema: Tensor  # int32 (-1: no move)
    binding: Tensor  # [N, label_width] int32 (-1 padding)
    final_states: Tensor
    count: Tensor
    states: Tensor
    task_ids: Tensor
    goal_pos: Tensor
    goal_neg: Tensor
    at_goal: Tensor
    obs: Any = None
    final_obs: Any = None
    revisited: Optional[Tensor] = None  # bool [N]: the reached state's key was in the env's visited table (false without tables)
    actions: Any = None
    action_visited: Any = None


class Rollout(NamedTuple):
    """A captured rollout's K steps stacked ([K, N, ...]; the same tensors after every replay)."""

    action: Optional[Tensor]
    reward: Tensor
    terminated: Tensor
    truncated: Tensor
    goal: Tensor
    invalid: Tensor
    schema: Tensor
    binding: Tensor
    final_states: Tensor
    count: Tensor
    states: Tensor
    task_ids: Tensor
    goal_pos: Tensor
    goal_neg: Tensor
    at_goal: Tensor
    obs: Optional[tuple] = None
    final_obs: Optional[tuple] = None
    revisited: Optional[Tensor] = None
    action_schema: Optional[Tensor] = None
    action_binding: Optional[Tensor] = None
    obs_actions: Optional[tuple] = None
    action_visited: Optional[tuple] = None


def _instance_sampler(value: Any, num_instances: int, default_uniform: bool) -> Optional[InstanceSampler]:
    """The sampler a BatchedEnv draws with: "auto" is uniform unless task ids pin the assignment (rl.resolve_sampler)."""
    return resolve_sampler(value, num_instances, auto_uniform=default_uniform,
                           mismatch="mymyr: sampler instance count does not match the environment's table or suite")


def _stream() -> int:
    return _lib.current_stream()


def _p(t: Optional[Tensor]):
    return None if t is None else t.data_ptr()


def _where(mask: Optional[Tensor], new: Tensor, old: Tensor) -> Tensor:
    if mask is None:
        return new
    m = mask.reshape(mask.shape + (1,) * (new.dim() - 1))
    return torch.where(m, new, old)


class BatchedEnv:
    """N environments over a task, a task table (a list of instances of one domain, or an rl.TaskTable) or a suite of
    several domains (rl.TaskSuite), stepped in lockstep on the device. Keyword arguments and defaults are the reference's (seed 0, step_reward 0, goal_reward 1, dead_end
    "no_successors", autoreset True, sampler "auto", first_env 0)."""

    def __init__(self, table: Task | list[Task] | TaskTable, num_envs: int, *, task_ids: Optional[Any] = None, sampler: Any = "auto",
                 device: str | torch.device = "cuda", goals: bool = False, seed: int = 0, max_steps: Optional[int] = None,
                 step_reward: float = 0.0, goal_reward: float = 1.0, dead_end: str = "no_successors", dead_end_reward: float = 0.0,
                 dead_end_terminal: bool = True, autoreset: bool = True, canonical_order: bool = True, witness_pruning: bool = False,
                 first_env: int = 0, observation: Any = None, actions: str = "index", track_visited: bool | int = False,
                 path: str = "auto", threads: int = 1, **unsupported: Any) -> None:
        if observation is not None or unsupported:
            raise NotImplementedError("mymyr_amd: BatchedEnv: observation encoders are not part of the device expansion path")
        if actions not in ("index", "label"):
            raise ValueError("mymyr: actions must be 'index' or 'label'")
        self.actions = actions
        if path not in ("auto", "fast"):
            raise ValueError("mymyr_amd: BatchedEnv runs the device's fast path only")
        if num_envs < 1 or num_envs > 0x7FFFFFFF:
            raise ValueError("mymyr: num_envs must be in [1, 2^31 - 1]")
        if dead_end not in ("no_successors", "none"):
            raise ValueError("mymyr: dead_end must be 'no_successors' or 'none'")
        suite = isinstance(table, TaskSuite)
        self._suite = suite
        if isinstance(table, TaskTable):
            table = table.tasks
        self.tasks = list(table) if isinstance(table, (list, tuple)) else [table]
        self.num_envs, self.first_env = int(num_envs), int(first_env)
        self.device = torch.device(device)
        if self.device.type != "cuda":
            raise ValueError("mymyr_amd: BatchedEnv runs on a HIP device")
        if self.device.index is None:
            self.device = torch.device("cuda", torch.cuda.current_device())
        I = len(self.tasks)
        self.multi = I > 1
        self.sampler = _instance_sampler(sampler, I, default_uniform=task_ids is None)
        self.launch = "widest"
        self._seed = int(seed)
        cfg = _lib.EnvConfig(seed, max_steps or 0, step_reward, goal_reward, dead_end_reward, 1 if dead_end == "none" else 0,
                             int(dead_end_terminal), int(autoreset), int(canonical_order), int(witness_pruning), 0)
        handles = (ctypes.c_void_p * I)(*[t.handle.value for t in self.tasks])
        h = ctypes.c_void_p()
        create = lib.mya_env_create_suite if suite else lib.mya_env_create_table
        with torch.cuda.device(self.device):
            check(create(handles, I, ctypes.byref(cfg), ctypes.byref(h)))
        self._h = h
        if self.sampler is not None:
            thr = np.ascontiguousarray(self.sampler.thresholds)
            idx = np.ascontiguousarray(self.sampler.indices)
            check(lib.mya_env_set_sampling(self._h, I, thr.ctypes.data, idx.ctypes.data, len(idx)))
        self._words = max(t.words for t in self.tasks)
        self._label_width = max(1, max(t.label_width for t in self.tasks))
        n, d, W = self.num_envs, self.device, self._words
        self.states = torch.zeros((n, W), dtype=torch.int64, device=d)
        self.task_ids = torch.zeros(n, dtype=torch.int32, device=d)
        self.reset_counts = torch.zeros(n, dtype=torch.int32, device=d)
        self.steps = torch.zeros(n, dtype=torch.int32, device=d)
        self.draws = torch.zeros(n, dtype=torch.int64, device=d)
        self.counts = torch.zeros((n, max(t.num_schemas for t in self.tasks) + 2), dtype=torch.int32, device=d)
        self.count = torch.zeros(n, dtype=torch.int32, device=d)
        self.at_goal = torch.zeros(n, dtype=torch.bool, device=d)
        self.goal_pos: Optional[Tensor] = None
        self.goal_neg: Optional[Tensor] = None
        if goals:
            self.goal_pos = torch.zeros((n, W), dtype=torch.int64, device=d)
            self.goal_neg = torch.zeros((n, W), dtype=torch.int64, device=d)
        # visited tables (track_visited): keys [N, H] int64, counts [N] int32, sticky status [1] int32
        self.visited_capacity = visited_capacity(track_visited, max_steps)
        H = self.visited_capacity
        self.visited = torch.zeros((n, H), dtype=torch.int64, device=d) if H else None
        self.visited_count = torch.zeros(n, dtype=torch.int32, device=d) if H else None
        self.visited_status = torch.zeros(1, dtype=torch.int32, device=d) if H else None
        self._batch = _lib.EnvBatch(self.states.data_ptr(), n, W, 0, self.steps.data_ptr(), self.draws.data_ptr(),
                                    self.at_goal.data_ptr(), self.first_env, self.counts.data_ptr(), _p(self.goal_pos),
                                    _p(self.goal_neg), self.task_ids.data_ptr() if self.multi else None, None, None,
                                    self.reset_counts.data_ptr() if self.sampler is not None else None, None, _p(self.visited),
                                    _p(self.visited_count), _p(self.visited_status), H, 0)
        # the scratch of N rows now: later calls allocate nothing, so they capture into graphs
        check(lib.mya_env_reserve(self._h, n))
        self.capturable = True
        initial = None if task_ids is None else self._task_ids(task_ids, None, "task_ids")
        self.reset(task_ids=initial)

    # ---------------------------------------------------------------------------------------------- properties
    @property
    def table(self) -> Task | list[Task]:
        return self.tasks if self.multi else self.tasks[0]

    @property
    def num_instances(self) -> int:
        return len(self.tasks)

    @property
    def row_words(self) -> int:
        return self._words

    @property
    def words(self) -> int:
        return self._words

    @property
    def label_width(self) -> int:
        return self._label_width

    @property
    def goals(self) -> bool:
        return self.goal_pos is not None

    # ---------------------------------------------------------------------------------------------- helpers
    def _task_ids(self, ids: Any, mask: Optional[Tensor], name: str) -> Tensor:
        """``ids`` (one id for every row, or [N]) as [N] int32 on the device; host values are checked here (ValueError
        for an id outside the table in a row the call uses), device values on the device (check_errors)."""
        n, I = self.num_envs, self.num_instances
        t = torch.as_tensor(ids)
        if t.dim() == 0:
            t = t.expand(n)
        if t.device.type == "cpu":
            flat = t.reshape(n).to(torch.int64)
            bad = (flat < 0) | (flat >= I)
            if mask is not None:
                bad &= mask.reshape(n).to(device="cpu", dtype=torch.bool)
            if bool(bad.any()):
                r = int(bad.nonzero()[0])
                raise ValueError(f"mymyr: {name}: task id {int(flat[r])} of row {r} is outside the table's {I} instances")
        return t.reshape(n).to(device=self.device, dtype=torch.int32).contiguous()

    def _empty_goals(self) -> Tensor:
        return self.states.new_empty((self.num_envs, 0))

    def observation(self, *, copy: bool = True) -> Observation:
        """Policy inputs that survive later steps and resets (``copy=False`` borrows the live tensors)."""
        keep = (lambda t: t.clone()) if copy else (lambda t: t)
        gp = keep(self.goal_pos) if self.goals else self._empty_goals()
        gn = keep(self.goal_neg) if self.goals else self._empty_goals()
        return Observation(keep(self.states), keep(self.task_ids), keep(self.count), gp, gn, keep(self.at_goal))

    # ---------------------------------------------------------------------------------------------- env calls
    def is_goal(self) -> Tensor:
        """Whether each environment's current state is a goal ([N] bool), without stepping."""
        out = torch.empty(self.num_envs, dtype=torch.bool, device=self.device)
        check(lib.mya_env_goal(self._h, ctypes.byref(self._batch), out.data_ptr(), _stream()))
        return out

    def reset(self, mask: Optional[Tensor] = None, *, task_ids: Optional[Any] = None, goal_pos: Optional[Tensor] = None,
              goal_neg: Optional[Tensor] = None) -> Tensor:
        """Resets all environments, or those with mask[i], to sampled instances (their current ones without a sampler;
        ``task_ids`` overrides sampling for reset rows); ``goal_pos`` / ``goal_neg`` (goals=True) set the reset rows'
        goals (default: their instances' goals). Returns ``count``."""
        if mask is not None:
            mask = mask.reshape(self.num_envs).to(device=self.device, dtype=torch.bool).contiguous()
        sample = task_ids is None and self.sampler is not None
        if task_ids is not None:
            new = self._task_ids(task_ids, mask, "reset")
            if self.multi:
                self.task_ids.copy_(_where(mask, new, self.task_ids))
        keep = goal_pos is not None or goal_neg is not None
        if keep:
            if not self.goals or goal_pos is None or goal_neg is None:
                raise ValueError("mymyr: per-env goals need goals=True and both goal_pos and goal_neg")
            self.goal_pos.copy_(_where(mask, goal_pos.to(self.goal_pos).expand_as(self.goal_pos), self.goal_pos))
            self.goal_neg.copy_(_where(mask, goal_neg.to(self.goal_neg).expand_as(self.goal_neg), self.goal_neg))
        m8 = None if mask is None else mask.view(torch.uint8)
        check(lib.mya_env_reset(self._h, ctypes.byref(self._batch), _p(m8), self.count.data_ptr(), int(keep), int(sample), _stream()))
        if getattr(self, "actions", "index") == "label":
            self.count.clamp_(max=1)
        return self.count

    def refresh(self) -> Tensor:
        """Recomputes the count cache, ``count`` and ``at_goal`` after the caller wrote states, task ids or goal masks."""
        check(lib.mya_env_refresh(self._h, ctypes.byref(self._batch), self.count.data_ptr(), _stream()))
        if self.actions == "label":
            self.count.clamp_(max=1)
        return self.count

    def _outputs(self, final: bool) -> list[Tensor]:
        n, d = self.num_envs, self.device
        fs = torch.empty((n if final else 0, self._words), dtype=torch.int64, device=d)
        return [torch.empty(n, dtype=torch.float32, device=d), torch.empty(n, dtype=torch.bool, device=d),
                torch.empty(n, dtype=torch.bool, device=d), torch.empty(n, dtype=torch.bool, device=d),
                torch.empty(n, dtype=torch.bool, device=d), torch.empty(n, dtype=torch.int32, device=d),
                torch.empty((n, self._label_width), dtype=torch.int32, device=d), fs]

    def _label_action(self, action: Any) -> tuple:
        """Label mode: each row's (schema int32 [N], binding int32 [N, L]) as device tensors; the step applies a row's
        label where it is applicable (the reference's label step, its counts clamped to 0/1)."""
        if not isinstance(action, tuple) or len(action) != 2:
            raise ValueError("mymyr: label mode requires action=(schema, binding); the random policy is unavailable")
        schema, binding = action
        if not isinstance(schema, Tensor) or not isinstance(binding, Tensor):
            raise ValueError("mymyr: label actions require schema and binding tensors")
        n = self.num_envs
        schema = schema.reshape(n).to(device=self.device, dtype=torch.int32).contiguous()
        binding = binding.to(device=self.device, dtype=torch.int32)
        if binding.dim() != 2 or binding.shape[0] != n:
            raise ValueError(f"mymyr: label actions require a binding tensor of shape [{n}, L]")
        if binding.shape[1] < self._label_width:
            raise ValueError(f"mymyr: label bindings have {binding.shape[1]} columns; the largest schema arity is {self._label_width}")
        return schema, binding.contiguous()

    def _action(self, action: Any) -> Optional[Tensor]:
        if self.actions == "label":
            return self._label_action(action)
        if action is None:
            return None
        if isinstance(action, tuple):
            raise ValueError("mymyr: label actions require actions='label'")
        a = torch.as_tensor(action)
        if a.dtype.is_floating_point or a.dtype.is_complex or a.dtype == torch.bool:
            raise TypeError(f"mymyr: actions must be integer successor indices, not {a.dtype}")
        return a.reshape(self.num_envs).to(device=self.device, dtype=torch.int64).contiguous()

    def _next_ids(self, next_task_ids: Optional[Any]) -> Optional[Tensor]:
        if next_task_ids is None:
            return None
        ids = self._task_ids(next_task_ids, None, "next_task_ids")
        return ids if self.multi else None  # a table of one: every instance is 0

    def _step_raw(self, outs: list[Tensor], action: Any, next_ids: Optional[Tensor], final: bool,
                  revisited: Optional[Tensor] = None) -> None:
        """One step into `outs`: action None (the random policy), int64 [N] indices, or a (schema, binding) label pair."""
        reward, term, trunc, goal, invalid, schema, binding, fs = outs
        o = _lib.StepOutputs(reward.data_ptr(), term.data_ptr(), trunc.data_ptr(), self.count.data_ptr(), fs.data_ptr() if final else None,
                             schema.data_ptr(), binding.data_ptr(), self._label_width, self._words, invalid.data_ptr(),
                             goal.data_ptr(), None, None, 0, 0, _p(revisited))
        if isinstance(action, tuple):
            ls, lb = action
            check(lib.mya_env_step_labels(self._h, ctypes.byref(self._batch), ctypes.byref(o), ls.data_ptr(), lb.data_ptr(), lb.shape[1],
                                          _p(next_ids), _stream()))
        else:
            check(lib.mya_env_step(self._h, ctypes.byref(self._batch), ctypes.byref(o), _p(action), _p(next_ids), _stream()))

    def step(self, action: Any = None, *, next_task_ids: Optional[Any] = None, final: bool = True, copy: bool = True) -> StepResult:
        """One step of every environment: ``action`` [N] int64 indexes the canonical successor order (None: the
        random policy); ``next_task_ids`` [N] overrides sampling for autoresetting environments; ``final=True`` keeps
        the reached states before the autoreset; ``copy=False`` borrows the live observation tensors."""
        outs = self._outputs(final)
        revisited = torch.zeros(self.num_envs, dtype=torch.bool, device=self.device)
        self._step_raw(outs, self._action(action), self._next_ids(next_task_ids), final, revisited if self.visited_capacity else None)
        if self.actions == "label":
            self.count.clamp_(max=1)  # ActionSpace::Label: whether an applicable action exists
        obs = self.observation(copy=copy)
        return StepResult(*outs, obs.count, obs.states, obs.task_ids, obs.goal_pos, obs.goal_neg, obs.at_goal, revisited=revisited)

    def clear_visited(self, mask: Optional[Tensor] = None) -> None:
        """Clear all visited tables, or rows selected by bool mask [N], and insert their current states."""
        if not self.visited_capacity:
            return
        m8 = None
        if mask is not None:
            m8 = mask.reshape(self.num_envs).to(device=self.device, dtype=torch.bool).contiguous().view(torch.uint8)
        check(lib.mya_env_clear_visited(self._h, ctypes.byref(self._batch), _p(m8), _stream()))

    def random_actions(self, max_actions: Optional[int] = None) -> Tensor:
        """The successors ``step(None)`` would take now, among the first ``max_actions`` (None: all); 0 where none."""
        if self.actions == "label":
            raise ValueError("mymyr: random_actions is unavailable in label mode")
        if max_actions is not None and int(max_actions) < 1:
            raise ValueError("mymyr: max_actions must be None or positive")
        out = torch.empty(self.num_envs, dtype=torch.int64, device=self.device)
        check(lib.mya_env_random_actions(self._h, ctypes.byref(self._batch), self.count.data_ptr(), int(max_actions or 0),
                                         out.data_ptr(), _stream()))
        return out

    def set_seed(self, seed: int) -> None:
        """New action and sampling RNG keys, in stream order on torch's current stream (steps and graph replays after
        it draw with the new key); the draw and reset counters restart at 0."""
        self._seed = int(seed)
        check(lib.mya_env_set_seed(self._h, self._seed & 0xFFFFFFFFFFFFFFFF, _stream()))
        self.draws.zero_()
        self.reset_counts.zero_()

    def capture(self, steps: int, policy: Optional[Callable[["BatchedEnv"], Tensor]] = None, *,
                next_task_ids: Optional[Tensor] = None, final: bool = False, pool: Any = None) -> "CapturedRollout":
        """``steps`` steps (actions from ``policy(self)``, or the random policy) captured into one HIP graph."""
        return CapturedRollout(self, steps, policy, next_task_ids=next_task_ids, final=final, pool=pool)

    def set_launch(self, launch: str) -> None:
        """'widest' or 'per_bucket' (BatchedEnv.set_launch, python/mymyr/rl/torch/_batched.py:573-575): how the
        reference's device env launches over a table's row-width buckets. The HIP env picks its launch shape itself
        (rows grouped by instance on the device, one launch per instance of a table of at most 16 instances, else one
        per kernel variant); the outputs do not depend on it, so either value is accepted and recorded."""
        if launch not in ("widest", "per_bucket"):
            raise ValueError("mymyr: launch must be 'widest' or 'per_bucket'")
        self.launch = launch

    def check_errors(self) -> None:
        """Waits for the device work and raises if a step met task ids outside the table, goal masks outside the
        instance's slots, or another device-side failure."""
        check(lib.mya_env_check(self._h))

    def close(self) -> None:
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib.mya_env_free(h)
            self._h = ctypes.c_void_p()

    def __del__(self) -> None:
        try:
            self.close()
        except Exception:
            pass

    def __repr__(self) -> str:
        return f"BatchedEnv(num_envs={self.num_envs}, device={self.device}, instances={self.num_instances}, words={self._words})"


class CapturedRollout:
    """``steps`` steps of a BatchedEnv (actions from ``policy(env)``, or the random policy) captured into one HIP graph;
    :meth:`replay` runs them again from the environments' current state and returns their stacked outputs (a
    :class:`Rollout`, the same tensors after every replay). A replay equals the same calls made eagerly, byte for byte.
    ``next_task_ids`` [N] int32 (a device tensor) is read at every replay."""

    def __init__(self, env: BatchedEnv, steps: int, policy: Optional[Callable[[BatchedEnv], Tensor]] = None, *,
                 next_task_ids: Optional[Tensor] = None, final: bool = False, pool: Any = None) -> None:
        if steps < 1:
            raise ValueError("mymyr: a captured rollout needs at least one step")
        self.labels = env.actions == "label"
        if self.labels and policy is None:
            raise ValueError("mymyr: label mode has no random policy; pass a policy returning (schema, binding)")
        if next_task_ids is not None and (not isinstance(next_task_ids, Tensor) or next_task_ids.device != env.device):
            raise ValueError("mymyr: a captured rollout's next_task_ids must be a tensor on the environments' device")
        self.env, self.steps, self.policy, self.final = env, int(steps), policy, final
        self.next_task_ids = None if next_task_ids is None else env._next_ids(next_task_ids)
        K, n, W, d = self.steps, env.num_envs, env.words, env.device
        z = lambda *shape, dtype: torch.zeros(shape, dtype=dtype, device=d)
        gw = W if env.goals else 0
        self.label_schema, self.label_binding = None, None
        self.out = Rollout(
            z(K, n, dtype=torch.int64) if policy is not None and not self.labels else None, z(K, n, dtype=torch.float32), z(K, n, dtype=torch.bool),
            z(K, n, dtype=torch.bool), z(K, n, dtype=torch.bool), z(K, n, dtype=torch.bool), z(K, n, dtype=torch.int32),
            z(K, n, env.label_width, dtype=torch.int32), z(K, n if final else 0, W, dtype=torch.int64), z(K, n, dtype=torch.int32),
            z(K, n, W, dtype=torch.int64), z(K, n, dtype=torch.int32), z(K, n, gw, dtype=torch.int64), z(K, n, gw, dtype=torch.int64),
            z(K, n, dtype=torch.bool), revisited=z(K, n, dtype=torch.bool))
        # warm the policy up on a side stream (lazy initializations), without stepping
        if policy is not None:
            side = torch.cuda.Stream(device=d)
            side.wait_stream(torch.cuda.current_stream(d))
            with torch.cuda.stream(side):
                for _ in range(2):
                    policy(env)
            torch.cuda.current_stream(d).wait_stream(side)
        torch.cuda.synchronize(d)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph, pool=pool):
            for k in range(K):
                self._step(k)
        if self.labels:
            self.out = self.out._replace(action_schema=self.label_schema, action_binding=self.label_binding)

    def _step(self, k: int) -> None:
        env, o = self.env, self.out
        action = None
        if self.labels:
            # the policy's labels into the rollout's label arrays (allocated at the first step, with its binding width)
            ls, lb = env._action(self.policy(env))
            if self.label_binding is None:
                K, n = self.steps, env.num_envs
                self.label_schema = torch.empty((K, n), dtype=torch.int32, device=env.device)
                self.label_binding = torch.empty((K, n, lb.shape[1]), dtype=torch.int32, device=env.device)
            self.label_schema[k].copy_(ls)
            self.label_binding[k].copy_(lb)
            action = (self.label_schema[k], self.label_binding[k])
        elif self.policy is not None:
            action = env._action(self.policy(env))
            o.action[k].copy_(action)
        outs = [o.reward[k], o.terminated[k], o.truncated[k], o.goal[k], o.invalid[k], o.schema[k], o.binding[k], o.final_states[k]]
        env._step_raw(outs, action, self.next_task_ids, self.final, o.revisited[k] if env.visited_capacity else None)
        if self.labels:
            env.count.clamp_(max=1)  # ActionSpace::Label: whether an applicable action exists
        o.count[k].copy_(env.count)
        o.states[k].copy_(env.states)
        o.task_ids[k].copy_(env.task_ids)
        o.at_goal[k].copy_(env.at_goal)
        if env.goals:
            o.goal_pos[k].copy_(env.goal_pos)
            o.goal_neg[k].copy_(env.goal_neg)

    def replay(self) -> Rollout:
        self.graph.replay()
        return self.out
