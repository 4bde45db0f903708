"""The torch BatchedEnv drop-in (mymyr_amd.batched, the reference's mymyr.rl.torch.BatchedEnv and CapturedRollout)
on the HIP env: the task-table trajectories of the compiled reference (tests/golden/env_table.json) replayed through
BatchedEnv's reset / step / sampler calls, digest-equal; captured rollouts equal to eager steps, byte for byte;
random_actions, set_seed and is_goal against their definitions."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def host(t):
    return t.cpu().numpy()


def u64(t):
    return host(t).view(np.uint64)


def load_tasks(golden, table):
    from mymyr_amd import workloads
    from mymyr_amd.task import Task

    return [Task.from_text_file(p) for p in workloads.table_files(table, golden.TASKS)]


@pytest.mark.parametrize("case", ["gridworld_ids", "gridworld_goals", "transport_ids", "gridworld_many", "gridworld_many_large",
                                  "suite_mixed", "suite_mixed_large", "gridworld_visited", "transport_visited",
                                  "gridworld_visited_large"])
def test_batched_env_matches_reference(golden, case):
    from mymyr_amd import rl
    from mymyr_amd.batched import BatchedEnv

    g = golden.load("env_table.json")[case]
    c = golden.TABLE_CASES[case]
    rows, goals = c["rows"], c.get("goals", False)
    assert not c.get("keys"), "BatchedEnv has no per-row keys"
    ts = load_tasks(golden, c["table"])
    inp = golden.table_inputs(case, len(ts))
    print(f"batched env case {case}: {rows} envs x {c['steps']} steps", flush=True)
    sampler = None
    if c.get("sampler") is not None:
        sampler = rl.InstanceSampler(len(ts), None if c["sampler"] == "uniform" else c["sampler"])
    table = rl.TaskSuite(ts) if c.get("suite") else ts
    env = BatchedEnv(table, rows, task_ids=inp["task_ids"], sampler=sampler, first_env=5, goals=goals,
                     track_visited=c.get("visited", False), **c["env"])
    init = [t.initial_state(env.words) for t in ts]

    def state():
        b = {"states": u64(env.states), "task_ids": host(env.task_ids), "steps": host(env.steps), "draws": u64(env.draws),
             "at_goal": host(env.at_goal).view(np.uint8)}
        if goals:
            b["goal_pos"], b["goal_neg"] = u64(env.goal_pos), u64(env.goal_neg)
        if sampler is not None:
            b["reset_counts"] = host(env.reset_counts).view(np.uint32)
        if env.visited is not None:
            b["visited"], b["visited_count"], b["visited_status"] = u64(env.visited), host(env.visited_count), host(env.visited_status)
        return golden.table_state(b)

    assert golden.arrays_digest(*state(), host(env.count)) == g["resets"]["initial"]
    assert torch.equal(env.is_goal(), env.at_goal)
    for k in range(c["steps"]):
        if k in inp["clears"]:
            env.clear_visited(torch.from_numpy(inp["clears"][k].astype(bool)))
            assert golden.arrays_digest(*state()) == g["resets"]["clear" + str(k)], f"{case}: clear_visited at step {k}"
        if k in inp["resets"]:
            mask, new, keep, sample = inp["resets"][k]
            m = torch.from_numpy(mask.astype(bool))
            if keep:
                ids = host(env.task_ids)
                gp = np.zeros((rows, env.words), np.uint64)
                for i in range(rows):
                    gp[i] = init[ids[i]]
                # the fixture's keep-goals reset keeps the rows' instances: with a sampler, name them (BatchedEnv samples
                # the reset rows' instances unless task ids are given)
                env.reset(m, task_ids=env.task_ids.clone() if sampler is not None else None,
                          goal_pos=torch.from_numpy(gp.view(np.int64)).cuda(), goal_neg=torch.zeros_like(env.goal_neg))
            else:
                assert sample == (new is None)
                env.reset(m, task_ids=None if new is None else torch.from_numpy(new))
            assert golden.arrays_digest(*state(), host(env.count)) == g["resets"][str(k)], f"{case}: reset at step {k}"
        acts = None
        if c["policy"] == "given":
            acts = torch.from_numpy(golden.given_actions(inp["u"][k], host(env.count)))
        nxt = inp["next"][k]
        r = env.step(acts, next_task_ids=None if nxt is None else torch.from_numpy(nxt), final=True)
        extra = [host(r.revisited).view(np.uint8)] if env.visited is not None else []
        d = golden.arrays_digest(*state(), host(r.reward), host(r.terminated).view(np.uint8), host(r.truncated).view(np.uint8),
                                 host(r.count), host(r.schema), host(r.binding), host(r.goal).view(np.uint8),
                                 host(r.invalid).view(np.uint8), u64(r.final_states), *extra)
        assert d == g["digests"][k], f"{case}: step {k} differs from the reference"
        assert torch.equal(r.states, env.states) and torch.equal(r.at_goal, env.at_goal)
    env.check_errors()


def _twins(golden, **kw):
    from mymyr_amd.batched import BatchedEnv

    ts = load_tasks(golden, "transport_table")
    n = 2000
    return BatchedEnv(ts, n, **kw), BatchedEnv(ts, n, **kw)


@pytest.mark.parametrize("policy", [None, "argmax"])
def test_captured_rollout_equals_eager_steps(golden, policy):
    """K steps captured into one HIP graph and replayed twice equal the same calls made eagerly on a twin env."""
    a, b = _twins(golden, seed=3, max_steps=7, sampler="uniform", track_visited=16)
    pol = None
    if policy == "argmax":
        pol = lambda env: torch.clamp(env.count.to(torch.int64) - 1, min=0)  # the last successor: capturable, device only
    K = 6
    roll = a.capture(K, pol, final=True)
    for rep in range(2):
        out = roll.replay()
        torch.cuda.synchronize()
        for k in range(K):
            act = None if pol is None else pol(b)
            r = b.step(act, final=True)
            for name in ("reward", "terminated", "truncated", "goal", "invalid", "schema", "binding", "final_states", "count",
                         "states", "task_ids", "at_goal", "revisited"):
                assert torch.equal(getattr(out, name)[k], getattr(r, name)), f"replay {rep} step {k}: {name}"
            if pol is not None:
                assert torch.equal(out.action[k], act), f"replay {rep} step {k}: action"
        for name in ("states", "task_ids", "steps", "draws", "reset_counts", "count", "at_goal", "counts", "visited", "visited_count",
                     "visited_status"):
            assert torch.equal(getattr(a, name), getattr(b, name)), f"replay {rep}: env {name}"
    a.check_errors()
    b.check_errors()


def test_random_actions_set_seed_and_goal(golden):
    from mymyr_amd.batched import BatchedEnv

    a, b = _twins(golden, seed=11, max_steps=9, sampler="uniform")
    for k in range(5):
        act = a.random_actions()
        ra = a.step(act)
        rb = b.step(None)
        for name in ("reward", "schema", "binding", "count", "states", "task_ids"):
            assert torch.equal(getattr(ra, name), getattr(rb, name)), f"step {k}: {name}"
    capped = a.random_actions(max_actions=2)
    assert bool(((capped >= 0) & (capped < 2)).all())
    assert bool((capped[a.count == 0] == 0).all())
    # set_seed: the draws restart with the new key, as a fresh env with that seed
    ts = a.tasks
    c = BatchedEnv(ts, a.num_envs, seed=99, max_steps=9, sampler="uniform")
    a.set_seed(99)
    assert int(a.draws.abs().sum()) == 0 and int(a.reset_counts.abs().sum()) == 0
    ids = c.task_ids.clone()
    a.reset(task_ids=ids)
    c.reset(task_ids=ids)
    a.reset_counts.copy_(c.reset_counts)
    for k in range(4):
        ra, rc = a.step(), c.step()
        for name in ("reward", "states", "task_ids", "count"):
            assert torch.equal(getattr(ra, name), getattr(rc, name)), f"after set_seed step {k}: {name}"
    assert torch.equal(a.is_goal(), a.at_goal)
    a.check_errors()
    c.check_errors()


def test_batched_env_argument_errors(golden):
    from mymyr_amd.batched import BatchedEnv

    ts = load_tasks(golden, "gridworld_table")
    with pytest.raises(ValueError):
        BatchedEnv(ts, 8, actions="name")
    with pytest.raises(ValueError, match="task id 3 of row 2 is outside the table's 3 instances"):
        BatchedEnv(ts, 8, task_ids=[0, 1, 3, 0, 1, 2, 0, 1])
    env = BatchedEnv(ts, 8, sampler=None, task_ids=0)
    assert env.sampler is None and int(env.task_ids.sum()) == 0
    with pytest.raises(TypeError):
        env.step(torch.zeros(8, dtype=torch.float32))
    env.set_launch("per_bucket")
    with pytest.raises(ValueError):
        env.set_launch("fastest")


def _labels(rng, x, n, nobj):
    """Labels for the rows of expansion x: a successor's label with random objects past its arity (70%), 20% of those
    with one object within the arity replaced by a random object (applicable or not), and 30% random garbage; and each
    label's position in its row's canonical successor order (-1: not applicable)."""
    off, sch, bnd = host(x["offsets"]).astype(np.int64), host(x["schema"]), host(x["binding"])
    L = bnd.shape[1]
    c = off[1:] - off[:-1]
    idx = (rng.random(n) * np.maximum(c, 1)).astype(np.int64)
    ls = np.full(n, -1, np.int32)
    lb = rng.integers(-1, 6, (n, L + 1)).astype(np.int32)
    for i in range(n):
        if c[i]:
            ls[i] = sch[off[i] + idx[i]]
            row = bnd[off[i] + idx[i]]
            lb[i, :L] = np.where(row >= 0, row, lb[i, :L])
            arity = int((row >= 0).sum())
            if arity and rng.random() < 0.2:
                lb[i, rng.integers(arity)] = rng.integers(nobj)
    garbage = rng.random(n) < 0.3
    ls[garbage] = rng.integers(-1, 8, int(garbage.sum()))
    act = np.full(n, -1, np.int64)
    for i in range(n):
        for j in range(off[i], off[i + 1]):
            if sch[j] == ls[i] and np.all((bnd[j] < 0) | (bnd[j] == lb[i, :L])):
                act[i] = j - off[i]
                break
    return ls, lb, act


LABEL_CASES = [("gridworld_table", {}), ("transport_table", {}), ("transport_table", {"goals": True, "track_visited": 16}),
               ("gridworld_table", {"track_visited": 8}), ("mixed_suite", {"suite": True, "goals": True})]


@pytest.mark.parametrize("table,extra", LABEL_CASES)
def test_label_steps_equal_index_steps(golden, table, extra):
    """actions="label": a label step equals the index step at the label's position in the row's canonical successor
    order (-1, invalid, when the label is not applicable), with counts clamped to 0/1, as the reference's label steps
    equal its index steps (tests/test_label_equivalence.py), also with per-env goals and visited tables. Positions come
    from a host scan of rl.expand's output; labels are successors' labels with random objects past their arity, some
    with a random object within it, and 30% random garbage."""
    from mymyr_amd import rl
    from mymyr_amd.batched import BatchedEnv

    ts = load_tasks(golden, table)
    n = 256
    extra = dict(extra)
    suite = extra.pop("suite", False)
    tt = rl.TaskSuite(ts) if suite else rl.TaskTable(ts)  # a suite's labels carry each domain's own schema ids
    kw = dict(seed=5, max_steps=9, sampler="uniform", **extra)
    a, b = BatchedEnv(tt if suite else ts, n, actions="label", **kw), BatchedEnv(tt if suite else ts, n, **kw)
    print(f"label steps: {table} {extra} suite={suite}, {n} envs", flush=True)
    assert torch.equal(a.count, b.count.clamp(max=1))
    rng = np.random.default_rng(2)
    nobj = max(t.num_objects for t in ts)
    moved = invalid = 0
    names = ["reward", "terminated", "truncated", "goal", "invalid", "schema", "binding", "final_states", "states", "task_ids", "at_goal"]
    if extra.get("track_visited"):
        names.append("revisited")
    for k in range(10):
        assert torch.equal(a.states, b.states) and torch.equal(a.task_ids, b.task_ids)
        x = rl.expand(tt, b.states, task_ids=b.task_ids)
        ls, lb, act = _labels(rng, x, n, nobj)
        ra = a.step((torch.from_numpy(ls).cuda(), torch.from_numpy(lb).cuda()))
        rb = b.step(torch.from_numpy(act).cuda())
        for name in names:
            assert torch.equal(getattr(ra, name), getattr(rb, name)), f"step {k}: {name}"
        assert torch.equal(ra.count, rb.count.clamp(max=1)), f"step {k}: count"
        moved += int((ra.schema >= 0).sum())
        invalid += int(ra.invalid.sum())
    assert moved > 0 and invalid > 0, (moved, invalid)
    if extra.get("track_visited"):
        assert torch.equal(a.visited, b.visited) and torch.equal(a.visited_count, b.visited_count)
    with pytest.raises(ValueError):
        a.random_actions()
    with pytest.raises(ValueError):
        a.step(None)
    with pytest.raises(ValueError, match="columns"):
        a.step((torch.zeros(n, dtype=torch.int32).cuda(), torch.zeros((n, 0), dtype=torch.int32).cuda()))
    a.check_errors()
    b.check_errors()


def test_captured_label_rollout_equals_eager_steps(golden):
    """Label mode captured into one HIP graph (a label policy computed on the device from the states): replays equal the
    same label steps made eagerly on a twin env, and the rollout keeps the policy's labels."""
    from mymyr_amd.batched import BatchedEnv

    ts = load_tasks(golden, "transport_table")
    n = 512
    kw = dict(seed=4, max_steps=7, sampler="uniform", actions="label", track_visited=8)
    a, b = BatchedEnv(ts, n, **kw), BatchedEnv(ts, n, **kw)
    S = max(t.num_schemas for t in ts)
    nobj = max(t.num_objects for t in ts)
    L = a.label_width

    def pol(env):
        h = env.states[:, : 2 * L].to(torch.int64)
        schema = (h.sum(1) % S).to(torch.int32)
        binding = ((h[:, :L] ^ h[:, L : 2 * L]).abs() % nobj).to(torch.int32)
        return schema, binding

    with pytest.raises(ValueError, match="policy"):
        a.capture(3, None)
    K = 5
    roll = a.capture(K, pol, final=True)
    moved = 0
    for rep in range(2):
        out = roll.replay()
        torch.cuda.synchronize()
        for k in range(K):
            ls, lb = pol(b)
            r = b.step((ls, lb), final=True)
            assert torch.equal(out.action_schema[k], ls) and torch.equal(out.action_binding[k], lb), f"replay {rep} step {k}: labels"
            for name in ("reward", "terminated", "truncated", "goal", "invalid", "schema", "binding", "final_states", "count",
                         "states", "task_ids", "at_goal", "revisited"):
                assert torch.equal(getattr(out, name)[k], getattr(r, name)), f"replay {rep} step {k}: {name}"
            moved += int((r.schema >= 0).sum())
        for name in ("states", "task_ids", "steps", "count", "at_goal", "counts", "visited", "visited_count"):
            assert torch.equal(getattr(a, name), getattr(b, name)), f"replay {rep}: env {name}"
    assert out.action is None
    a.check_errors()
    b.check_errors()
