"""The device env over task tables (several instances of one domain, rows grouped by instance on the device) against
the compiled reference's rl::HostEnv over TaskTable::create: every reset and step of the fixture's trajectories
(tests/golden/env_table.json, from 24 to 8192 envs; tables of 3 instances step with one launch per instance, the
20-instance table with one launch per kernel variant) digest-equal, through the C ABI (mymyr_amd.rl.DeviceEnvPool).
Also: a table whose rows all sit in one instance steps exactly as a one-instance env of that task, task ids outside
the table raise through the sticky status, and a grouped step replays from a HIP graph."""

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


def initial_rows(ts, W):
    return [t.initial_state(W) for t in ts]


def replay(golden, case: str):
    from mymyr_amd import rl

    g = golden.load("env_table.json")[case]
    c = golden.TABLE_CASES[case]
    rows, steps, goals = c["rows"], c["steps"], c.get("goals", False)
    ts = load_tasks(golden, c["table"])
    inp = golden.table_inputs(case, len(ts))
    print(f"table case {case}: {rows} envs x {steps} steps", flush=True)
    sampler = None
    if c.get("sampler") is not None:
        sampler = rl.InstanceSampler(len(ts), None if c["sampler"] == "uniform" else c["sampler"])
    table = rl.TaskSuite(ts) if c.get("suite") else ts
    pool = rl.DeviceEnvPool(table, rows, first_env=5, goals=goals, task_ids=inp["task_ids"], sampler=sampler, seeds=inp.get("seeds"),
                            env_ids=inp.get("env_ids"), sampling_seeds=inp.get("sampling_seeds"), track_visited=c.get("visited", False),
                            **c["env"])
    assert (pool.words, pool.label_width) == (g["words"], g["label_width"])
    W = pool.words
    init = initial_rows(ts, W)

    def state():
        b = {"states": u64(pool.states), "task_ids": host(pool.task_ids), "steps": host(pool.steps), "draws": u64(pool.draws),
             "at_goal": host(pool.at_goal)}
        if goals:
            b["goal_pos"], b["goal_neg"] = u64(pool.goal_pos), u64(pool.goal_neg)
        if pool.reset_counts is not None:
            b["reset_counts"] = host(pool.reset_counts).view(np.uint32)
        if pool.visited is not None:
            b["visited"], b["visited_count"], b["visited_status"] = u64(pool.visited), host(pool.visited_count), host(pool.visited_status)
        return golden.table_state(b)

    pool.reset()
    assert golden.arrays_digest(*state(), host(pool.count)) == g["resets"]["initial"], f"{case}: initial reset"
    for k in range(steps):
        if k in inp["clears"]:
            pool.clear_visited(torch.from_numpy(inp["clears"][k]))
            assert golden.arrays_digest(*state()) == g["resets"]["clear" + str(k)], f"{case}: clear_visited at step {k}"
        if k in inp["resets"]:
            mask, new, keep, sample = inp["resets"][k]
            if keep:
                gp = u64(pool.goal_pos).copy()
                ids = host(pool.task_ids)
                for i in np.nonzero(mask)[0]:
                    gp[i] = init[ids[i]]
                pool.goal_pos.copy_(torch.from_numpy(gp.view(np.int64)))
                pool.goal_neg[torch.from_numpy(mask.astype(bool)).to(pool.device)] = 0
            pool.reset(torch.from_numpy(mask), keep_goals=keep, task_ids=None if new is None else torch.from_numpy(new), sample=sample)
            assert golden.arrays_digest(*state(), host(pool.count)) == g["resets"][str(k)], f"{case}: reset at step {k}"
        acts = None
        if c["policy"] == "given":
            acts = torch.from_numpy(golden.given_actions(inp["u"][k], host(pool.count)))
        nxt = inp["next"][k]
        o = pool.step(actions=acts, final_states=True, next_task_ids=None if nxt is None else torch.from_numpy(nxt))
        extra = [host(o["revisited"])] if pool.visited is not None else []
        d = golden.arrays_digest(*state(), host(o["reward"]), host(o["terminated"]), host(o["truncated"]), host(o["count"]),
                                 host(o["schema"]), host(o["binding"]), host(o["goal"]), host(o["invalid"]), u64(o["final_states"]),
                                 *extra)
        assert d == g["digests"][k], f"{case}: step {k} differs from the reference"
        if k == golden.TABLE_EXPAND_STEP and case in golden.TABLE_EXPAND_CASES:
            # rl::expand over the table on the batch after this step (rows of several instances, grouped on the device)
            group = rl.TaskSuite(ts) if c.get("suite") else rl.TaskTable(ts)
            for key, drop in (("all", False), ("drop", True)):
                x = rl.expand(group, pool.states, task_ids=pool.task_ids, goal=True, hashes=True, noops=True, index=True, drop_noops=drop)
                want = g["expand"][key]
                assert (x["generated"], x["total"]) == (want["generated"], want["total"]), f"{case}: expansion {key}"
                got = {"succ": u64(x["succ"]), "parent": host(x["parent"]), "schema": host(x["schema"]), "binding": host(x["binding"]),
                       "goal": host(x["goal"]), "succ_hash": u64(x["succ_hash"]), "noop": host(x["noop"]), "index": host(x["index"]),
                       "offsets": host(x["offsets"])}
                assert golden.expansion_digest(got) == want["digest"], f"{case}: expansion {key}"
                # the padded view (rl::pad) on the device, at the automatic k and at k = 3
                for kp in golden.pad_ks(got["offsets"]):
                    p = rl.pad(x, kp)
                    hp = {n: (u64(t) if n in ("succ", "succ_hash") else host(t)) for n, t in p.items() if isinstance(t, torch.Tensor)}
                    assert golden.padded_digest(hp) == want["pad"][str(kp)]["digest"], f"{case}: pad {key} k={kp}"
                    assert p["overflow"] == want["pad"][str(kp)]["overflow"], f"{case}: pad {key} k={kp} overflow"
    pool.check()
    return pool


@pytest.mark.parametrize("case", ["gridworld_ids", "gridworld_goals", "transport_ids", "gridworld_sampled", "transport_weighted",
                                  "gridworld_many", "suite_mixed", "gridworld_large", "transport_large", "gridworld_sampled_large",
                                  "gridworld_many_large", "suite_mixed_large", "gridworld_visited", "transport_visited",
                                  "gridworld_visited_large"])
def test_table_env_matches_reference(golden, case):
    replay(golden, case)


@pytest.mark.parametrize("table", ["gridworld_table", "transport_table"])
def test_one_instance_rows_step_as_the_task(golden, table):
    """Rows that all sit in instance k (next_task_ids = k) step exactly as a one-instance env of task k with rows as
    wide as the table's: the grouped kernels and the batch-order kernels agree word for word."""
    from mymyr_amd import rl

    ts = load_tasks(golden, table)
    W = max(t.words for t in ts)
    n = 1000
    for k, t in enumerate(ts):
        a = rl.DeviceEnvPool(ts, n, seed=9, max_steps=25, task_ids=np.full(n, k, np.int32), first_env=3)
        b = rl.DeviceEnvPool(t, n, seed=9, max_steps=25, words=W, first_env=3)
        a.reset()
        b.reset()
        nxt = torch.full((n,), k, dtype=torch.int32)
        for step in range(30):
            oa = a.step(next_task_ids=nxt, final_states=True)
            ob = b.step(final_states=True)
            for key in ("states", "reward", "terminated", "truncated", "count", "schema", "binding", "goal", "at_goal", "final_states"):
                assert torch.equal(oa[key], ob[key]), f"{table} instance {k} step {step}: {key}"
        a.check()
        b.check()


def test_task_ids_outside_the_table(golden):
    from mymyr_amd import rl
    from mymyr_amd._lib import MyaError

    ts = load_tasks(golden, "gridworld_table")
    pool = rl.DeviceEnvPool(ts, 64, task_ids=np.arange(64) % 3)
    pool.reset()
    pool.check()
    # a reset into an id outside the table puts the row in instance 0 and raises at the check
    with pytest.raises(MyaError, match="task id is outside the table's 3 instances"):
        pool.reset(task_ids=np.where(np.arange(64) == 7, 5, np.arange(64) % 3))
        pool.check()
    assert int(pool.task_ids[7]) == 0
    init0 = initial_rows(ts, pool.words)[0]
    assert np.array_equal(u64(pool.states)[7], init0)
    pool.check()
    # next_task_ids outside the table: reported, the row keeps its instance
    with pytest.raises(MyaError, match="task id is outside"):
        pool.step(next_task_ids=np.full(64, -1, np.int32))
        pool.check()
    assert np.array_equal(host(pool.task_ids), np.where(np.arange(64) == 7, 0, np.arange(64) % 3))
    pool.check()


def test_grouped_step_graph_replay(golden):
    """A grouped step (grouping kernels + per-variant step launches) captured into a HIP graph replays as eager steps."""
    from mymyr_amd import rl

    ts = load_tasks(golden, "transport_table")
    n = 3000
    ids = (np.arange(n) * 7) % 3
    kw = dict(seed=4, max_steps=12, task_ids=ids)
    a, b = rl.DeviceEnvPool(ts, n, **kw), rl.DeviceEnvPool(ts, n, **kw)
    a.reset()
    b.reset()
    nxt = torch.from_numpy(((np.arange(n) * 5) % 3).astype(np.int32)).cuda()
    a.step(next_task_ids=nxt)  # eager first call: scratch and LDS limits set up outside the capture
    b.step(next_task_ids=nxt)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        a.step(next_task_ids=nxt)
    for r in range(6):
        graph.replay()
        torch.cuda.synchronize()
        ob = b.step(next_task_ids=nxt)
        extra = (a.states.sum() + 1).item()  # eager work on the pool's arrays between replays
        assert extra is not None
        for key in ("states", "reward", "terminated", "truncated", "count", "at_goal", "task_ids"):
            assert torch.equal(getattr(a, key), ob[key]), f"replay {r}: {key}"
    a.check()
    b.check()


@pytest.mark.parametrize("k", [0, 1, 3, None, 40])
def test_pad_edges(golden, k):
    """rl::pad on the device against the oracle's pad on the same flat expansion: a flat capacity below the total (slots
    past it invalid, overflow), k = 0 and k above every count, wider padded rows and labels, and an empty batch."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task
    from mymyr_amd import workloads

    ts = [Task.from_text_file(p) for p in workloads.table_files("transport_table", golden.TASKS)]
    pool = rl.DeviceEnvPool(ts[0], 37, seed=4, max_steps=50)
    for _ in range(3):
        pool.step()
    print(f"pad edges: 37 transport rows, k={k}", flush=True)
    full = rl.expand(ts[0], pool.states, hashes=True, noops=True, drop_noops=True)
    for cap in (None, full["generated"] // 2):
        x = full if cap is None else rl.expand(ts[0], pool.states, capacity=cap, hashes=True, noops=True, drop_noops=True)
        hx = {n: (u64(t) if n in ("succ", "succ_hash") else host(t)) if isinstance(t, torch.Tensor) else t for n, t in x.items()}
        kk = rl.auto_k(x["offsets"]) if k is None else k
        p = rl.pad(x, k, words=ts[0].words + 2, label_width=x["binding"].shape[1] + 1)
        want = port_pad(hx, 37, kk, ts[0].words + 2, x["binding"].shape[1] + 1, x["capacity"])
        for n in ("index", "mask", "count", "succ", "schema", "binding", "succ_hash", "noop", "canonical"):
            got = u64(p[n]) if n in ("succ", "succ_hash") else host(p[n])
            assert np.array_equal(got, want[n]), f"cap={cap} k={kk}: {n}"
        assert p["overflow"] == want["overflow"]
        if cap is not None:
            assert p["overflow"]
    empty = rl.expand(ts[0], pool.states[:0])
    e = rl.pad(empty, k)
    assert e["count"].numel() == 0 and e["succ"].shape[0] == 0 and not e["overflow"]
    pool.check()


def port_pad(*a):
    from oracle import port

    return port.pad(*a)


def test_visited_mask_matches_reference(golden):
    """rl.visited_mask on the device against the compiled reference's rl::visited_mask on the same tables and queries
    (tests/golden/visited_mask.json), with and without a row mapping."""
    from mymyr_amd import rl

    g = golden.load("visited_mask.json")
    u = lambda xs: torch.from_numpy(np.array([int(x) for x in xs], np.uint64).view(np.int64)).cuda()
    table = torch.stack([u(t) for t in g["table"]])
    count = torch.tensor(g["count"], dtype=torch.int32, device="cuda")
    hashes = u(g["hashes"])
    print(f"visited mask: {len(g['hashes'])} queries over {len(g['count'])} tables", flush=True)
    got = rl.visited_mask(table, count, hashes, torch.tensor(g["parent"], dtype=torch.int32, device="cuda"))
    assert host(got).astype(np.uint8).tolist() == g["mask"]
    got = rl.visited_mask(table, count, hashes, torch.tensor(g["parent_mapped"], dtype=torch.int32, device="cuda"),
                          torch.tensor(g["rows"], dtype=torch.int32, device="cuda"))
    assert host(got).astype(np.uint8).tolist() == g["mask_mapped"]


def test_visited_mask_of_an_expansion(golden):
    """The successors of an env batch checked against the rows' own visited tables after a few steps (the novelty test
    of an expansion), against the oracle's visited_mask; out-of-range parents and mapped rows read as not visited."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task
    from mymyr_amd import workloads
    from oracle import port

    ts = [Task.from_text_file(p) for p in workloads.table_files("gridworld_table", golden.TASKS)]
    n = 300
    pool = rl.DeviceEnvPool(ts[0], n, seed=9, max_steps=40, track_visited=64)
    for _ in range(12):
        pool.step()
    print(f"visited mask of an expansion: {n} gridworld rows", flush=True)
    x = rl.expand(ts[0], pool.states, hashes=True)
    tab, cnt = u64(pool.visited), host(pool.visited_count)
    sh, par = u64(x["succ_hash"]), host(x["parent"])
    got = host(rl.visited_mask(pool.visited, pool.visited_count, x["succ_hash"], x["parent"]))
    want = port.visited_mask(tab, cnt, sh, par)
    assert np.array_equal(got.astype(np.uint8), want) and 0 < want.sum() < len(want)
    # padding, parents past the tables, and a row mapping with -1 and out-of-range rows
    rng = np.random.default_rng(1)
    p2 = rng.integers(-1, n + 5, len(sh)).astype(np.int32)
    got = host(rl.visited_mask(pool.visited, pool.visited_count, x["succ_hash"], torch.from_numpy(p2).cuda()))
    assert np.array_equal(got.astype(np.uint8), port.visited_mask(tab, cnt, sh, p2))
    rows = rng.integers(-1, n + 3, 50).astype(np.int32)
    p3 = rng.integers(-1, 55, len(sh)).astype(np.int32)
    got = host(rl.visited_mask(pool.visited, pool.visited_count, x["succ_hash"], torch.from_numpy(p3).cuda(), torch.from_numpy(rows).cuda()))
    assert np.array_equal(got.astype(np.uint8), port.visited_mask(tab, cnt, sh, p3, rows))
    with pytest.raises(RuntimeError, match="power of two"):
        rl.visited_mask(pool.visited[:, :48], pool.visited_count, x["succ_hash"], x["parent"])
    pool.check()
