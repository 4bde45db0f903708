"""The device env step against the reference HostEnv's trajectories (per-step digests of states, rewards,
terminations, truncations, counts, labels and goals written by the compiled reference), the canonical successor
listing against the reference's, and the per-step encodings against the oracle's closed forms.

An env's trajectory depends only on its row, its actions and its RNG stream (env id), so a full-size batch is checked
on its first rows against the reference's trajectory of a smaller batch (include/mymyr/rl/env.hpp:46-48)."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def host(t):
    return t.cpu().numpy()


def run_env(golden, fixture: str, num_envs: int | None = None, encode: int = 0, on_step=None, **pool_kw):
    """Steps num_envs envs (default: the fixture's rows) for the fixture's steps and compares the per-step digests of
    the rows whose env ids the fixture holds (first_env, first_env + 1, ...; the first rows unless it says otherwise)
    with the reference's; on_step(k, outputs) sees each step's outputs (device tensors over every env)."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task

    g = golden.load(fixture)
    atoms = "dense" if g["workload"] == "strips" else "auto"
    t = Task.from_text_file(golden.task_path(g["workload"]), atoms)
    n = num_envs or g["rows"]
    print(f"{fixture}: {n} envs x {g['steps']} steps", flush=True)
    pool = rl.DeviceEnvPool(t, n, **g["env"], **pool_kw)
    pool.reset()
    rows = g["rows"]
    r0 = g.get("first_env", 0)
    assert r0 + rows <= n
    L = max(1, t.label_width)
    for k in range(g["steps"]):
        o = pool.step(encode=encode)
        h = {key: host(o[key][r0:r0 + rows]) for key in ("states", "reward", "terminated", "truncated", "count", "schema", "binding", "goal")}
        d = golden.step_digest(rows, h["states"].view(np.uint64), h["reward"], h["terminated"], h["truncated"], h["count"], h["schema"],
                               h["binding"][:, :L], h["goal"])
        assert d == g["digests"][k], f"{fixture}: step {k} differs from the reference"
        if on_step:
            on_step(k, o)
    pool.check()
    return pool, t


def test_gridworld_full_workload(golden):
    """The gridworld workload at its full size (1024 envs x 256 steps), bit-exact every step."""
    run_env(golden, "env_gridworld.json")


def test_gridworld_truncation_goals_resets(golden):
    g = golden.load("env_gridworld_truncated.json")
    assert g["totals"]["truncated"] > 0 and g["totals"]["terminated"] > 0  # the fixture exercises both
    run_env(golden, "env_gridworld_truncated.json")


def test_transport_full_batch_first_rows(golden):
    """65536 envs (the transport workload's batch) stepped on the device; the first 2048 rows match the reference."""
    run_env(golden, "env_transport.json", num_envs=65536)


def test_transport_xl_first_rows_with_encoding(golden):
    """transport_xl with the encoding outputs on; the first rows match the reference's trajectory."""
    pool, t = run_env(golden, "env_transport_xl.json", num_envs=4096, encode=600)


def test_transport_whole_horizon_full_batch(golden):
    """The transport workload as run: 65536 envs for all 512 steps; the first 256 rows match the reference every step."""
    run_env(golden, "env_transport_long.json", num_envs=65536)


def test_transport_whole_horizon_last_rows(golden):
    """The transport workload as run (65536 envs, 512 steps): its last 64 rows (env ids 65472 to 65535, whose Philox
    counters, row offsets and places in the resident grid differ most from the first rows') match the reference's
    trajectory of those env ids every step."""
    run_env(golden, "env_transport_long_tail.json", num_envs=65536)


def test_transport_xl_whole_horizon_last_rows(golden):
    """The transport_xl workload as run (262144 envs, 128 steps, encoding on at 544 atoms): its last 64 rows (env ids
    262080 to 262143, whose rows start 2.8 GB into the batch, past 2^31 bytes) match the reference's trajectory every
    step."""
    run_env(golden, "env_transport_xl_long_tail.json", num_envs=262144, encode=544)


def run_batch(golden, fixture: str, encode: int = 0):
    """Steps a workload's whole batch over its whole horizon and compares, every step, the digest of every row (states
    as their state hashes, computed on the device; rewards, terminations, truncations, counts, labels and goals) with
    the reference's."""
    from mymyr_amd import hip, rl
    from mymyr_amd.task import Task

    g = golden.load(fixture)
    t = Task.from_text_file(golden.task_path(g["workload"]))
    n, L = g["rows"], max(1, t.label_width)
    print(f"{fixture}: {n} envs x {g['steps']} steps, every row", flush=True)
    pool = rl.DeviceEnvPool(t, n, **g["env"])
    pool.reset()
    for k in range(g["steps"]):
        o = pool.step(encode=encode)
        hashes = host(hip.hash_rows(o["states"][:, : t.words].contiguous())).view(np.uint64)
        d = golden.rows_digest(hashes, host(o["reward"]), host(o["terminated"]), host(o["truncated"]), host(o["count"]),
                               host(o["schema"]), host(o["binding"])[:, :L], host(o["goal"]))
        assert d == g["digests"][k], f"{fixture}: step {k} differs from the reference"
    pool.check()


def test_transport_every_row_whole_horizon(golden):
    """The transport workload as run (65536 envs, 512 steps): every row equals the reference's every step."""
    run_batch(golden, "env_transport_batch.json")


def test_transport_xl_every_row_whole_horizon(golden):
    """The transport_xl workload as run (262144 envs, 128 steps, the encoding on at its 544 atoms): every row equals the
    reference's every step."""
    run_batch(golden, "env_transport_xl_batch.json", encode=544)


def reference_masks(rt, row):
    """Per schema, whether the compiled reference generates a successor with it (rl::schema_masks semantics)."""
    m = np.zeros(rt.num_schemas, np.uint8)
    sc, _, _ = rt.successors(row)
    m[np.asarray(sc, dtype=np.int64)] = 1
    return m


def test_transport_xl_full_workload_with_encoding(golden):
    """The transport_xl workload as run: 262144 envs for all 128 steps with the encoding at the task's atom count (every
    state holds 544 true atoms: 32 trucks and 512 packages, one position each). The first 64 rows match the
    reference's trajectory every step; on sampled rows of the whole batch (the last rows included) at several steps,
    the atom indices are the state's set slots in ascending order, padded with -1 (the closed form of State::slots),
    and the schema masks equal the schemas of the compiled reference's successor listing of that state."""
    from oracle import port, ref

    rt = ref.RefTask(golden.task_path("transport_xl"))
    max_atoms = 544
    N = 262144
    sample = np.array([0, 1, 63, 64, 1000, 65535, 131072, 200001, N - 2, N - 1])
    idx = torch.as_tensor(sample, device="cuda")
    checked = []

    def on_step(k, o):
        if k % 37 not in (0, 36) and k != 127:
            return
        states = host(o["states"].index_select(0, idx)).view(np.uint64)
        atoms = host(o["atoms"].index_select(0, idx))
        masks = host(o["masks"].index_select(0, idx))
        for i in range(len(sample)):
            row = states[i, : rt.words]
            assert int(np.unpackbits(row.view(np.uint8)).sum()) == max_atoms
            assert np.array_equal(atoms[i], port.encode_atoms(row, max_atoms)), (k, int(sample[i]))
            assert np.array_equal(masks[i], reference_masks(rt, row)), (k, int(sample[i]))
        checked.append(k)

    pool, t = run_env(golden, "env_transport_xl_long.json", num_envs=N, encode=max_atoms, on_step=on_step)
    assert len(checked) >= 6


def test_encoding_closed_form(golden):
    from mymyr_amd import rl
    from mymyr_amd.task import Task
    from oracle import port

    text = open(golden.task_path("transport")).read()
    t = Task.from_text(text)
    pt = port.Task(text)
    pool = rl.DeviceEnvPool(t, 64, seed=11)
    pool.reset()
    for _ in range(5):
        o = pool.step(encode=160)
    states = host(o["states"]).view(np.uint64)
    atoms, masks = host(o["atoms"]), host(o["masks"])
    for i in range(0, 64, 7):
        assert np.array_equal(atoms[i], port.encode_atoms(states[i, : pt.words], 160))
        assert np.array_equal(masks[i], port.schema_masks(pt, states[i, : pt.words]))
    # the standalone ops agree with the fused outputs
    assert np.array_equal(host(pool.encode_atoms(o["states"], 160)), atoms)
    assert np.array_equal(host(pool.schema_masks(o["states"])), masks)


@pytest.mark.parametrize("name", ["gripper__prob05", "blocks__probBLOCKS-8-0", "depot__p02", "gridworld", "transport", "strips",
                                  "transport_xl"])
def test_successor_listing_golden(golden, name):
    from mymyr_amd import rl
    from mymyr_amd.task import Task
    from oracle import port

    g = golden.load("successors.json")[name]
    t = Task.from_text_file(golden.task_path(name), "dense" if name == "strips" else "auto")
    rows = np.array([[int(x, 16) for x in s["row"]][: t.words] for s in g], dtype=np.uint64)
    cap = max(s["count"] for s in g) + 1
    cnt, sch, bnd, succ = rl.successors(t, torch.from_numpy(rows.view(np.int64)).cuda(), cap=cap)
    cnt, sch, bnd, succ = host(cnt), host(sch), host(bnd), host(succ).view(np.uint64)
    for i, s in enumerate(g):
        k = s["count"]
        assert cnt[i] == k
        assert list(sch[i, :k]) == s["schema"]
        if k:
            assert bnd[i, :k, : len(s["binding"][0])].tolist() == s["binding"]
        assert [f"{port.hash_state(r):016x}" for r in succ[i, :k]] == s["succ_hash"]


def test_given_actions_and_invalid(golden):
    """Index actions: in-range ones move to that successor; out-of-range ones do not move and set invalid."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path("gridworld"))
    pool = rl.DeviceEnvPool(t, 8, seed=0)
    pool.reset()
    s0 = host(pool.states).copy()
    cnt, _, _, succ = rl.successors(t, pool.states, cap=8)
    acts = torch.tensor([0, 1, -1, 100, 0, 0, 0, 0], dtype=torch.int64)
    o = pool.step(actions=acts)
    inv = host(o["invalid"])
    assert list(inv[:4]) == [0, int(host(cnt)[1] <= 1), 1, 1]
    assert np.array_equal(host(o["states"])[0], host(succ)[0, 0])
    assert np.array_equal(host(o["states"])[2], s0[2])
    assert host(o["reward"])[2] == 0.0  # step_reward 0: an invalid action earns it, not the goal reward


def test_env_argument_errors(golden):
    from mymyr_amd import rl
    from mymyr_amd._lib import MyaError
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path("transport"))
    with pytest.raises(MyaError, match="witness_pruning"):
        rl.DeviceEnvPool(t, 4, witness_pruning=True)
    with pytest.raises(ValueError, match="words"):
        rl.DeviceEnvPool(t, 4, words=2)
    pool = rl.DeviceEnvPool(t, 4)
    with pytest.raises(ValueError, match="shape"):
        pool.step(actions=torch.zeros(3, dtype=torch.int64))


def test_without_count_cache(golden):
    """The step without the count cache (every step counts its state's successors) gives the same trajectories."""
    run_env(golden, "env_gridworld_truncated.json", count_cache=False)
    run_env(golden, "env_transport.json", count_cache=False)


def test_count_cache_with_states_written_directly(golden):
    """Rows whose states are written directly, without refresh, are counted again (their cache fingerprints no longer
    match), and refresh() rebuilds at_goal and the cache: the cached pool follows the uncached one step for step."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task

    g = golden.load("env_gridworld_truncated.json")
    t = Task.from_text_file(golden.task_path(g["workload"]), "auto")
    a = rl.DeviceEnvPool(t, 512, **g["env"])
    b = rl.DeviceEnvPool(t, 512, **g["env"], count_cache=False)
    a.reset()
    b.reset()
    keys = ("states", "reward", "terminated", "truncated", "count", "schema", "binding", "goal", "steps", "at_goal")

    def step_both(k):
        oa, ob = a.step(), b.step()
        for key in keys:
            assert torch.equal(oa[key], ob[key]), f"step {k}: {key} differs"

    for k in range(6):
        step_both(k)
    # rows take other rows' states (with their goal flags), written directly: the cache rows no longer match them
    for p in (a, b):
        p.states.copy_(p.states.roll(7, dims=0))
        p.at_goal.copy_(p.at_goal.roll(7, dims=0))
    for k in range(6, 12):
        step_both(k)
    # a write followed by refresh(): at_goal and the cache are recomputed from the states
    init = torch.from_numpy(t.initial_state().view(np.int64)).cuda()
    for p in (a, b):
        p.states[::3] = init
        p.refresh()
    assert torch.equal(a.at_goal, b.at_goal) and torch.equal(a.count, b.count)
    for k in range(12, 20):
        step_both(k)
    a.check()
    b.check()


def test_step_replayed_from_a_hip_graph(golden):
    """A step recorded into a HIP graph (torch.cuda.graph) and replayed follows the eager steps of a twin pool: the
    step launches kernels only (no synchronization, allocation or memset), as the reference's device env contract
    for graph capture (include/mymyr/cuda/env.hpp:64-74) requires. Eager work and synchronizations run between the
    replays, and every replay is checked."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task

    g = golden.load("env_gridworld_truncated.json")
    t = Task.from_text_file(golden.task_path(g["workload"]), "auto")
    a = rl.DeviceEnvPool(t, 1024, **g["env"])
    b = rl.DeviceEnvPool(t, 1024, **g["env"])
    a.reset()
    b.reset()
    keys = ("states", "reward", "terminated", "truncated", "count", "schema", "binding", "goal", "steps", "at_goal")
    oa = a.step()  # eager first call: LDS limits set, outputs allocated
    ob = b.step()
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        a.step()
    for k in range(12):
        graph.replay()
        torch.cuda.synchronize()
        ob = b.step()
        extra = (a.states.sum() + 1).item()  # eager work on the pool's arrays between replays
        assert extra is not None
        for key in keys:
            assert torch.equal(oa[key], ob[key]), f"replay {k}: {key} differs"
    a.check()
    b.check()


def test_per_env_goals_default_to_the_task_goal(golden):
    """With per-env goal masks holding the task's goal (what reset writes), trajectories equal the reference's."""
    pool, t = run_env(golden, "env_gridworld_truncated.json", goals=True)
    from oracle import port

    pt = port.Task(open(golden.task_path("gridworld")).read())
    gp, gn = port.Env(pt).goal_masks(t.words)
    assert np.array_equal(host(pool.goal_pos).view(np.uint64), np.tile(gp, (pool.num_envs, 1)))
    assert not host(pool.goal_neg).any()


def _single(pt, slot):
    row = np.zeros(pt.words, np.uint64)
    row[slot >> 6] = np.uint64(1) << np.uint64(slot & 63)
    return row


def test_per_env_goals_against_the_oracle(golden):
    """Each env gets its own goal cell (mask_goal over per-env masks, kept by reset(keep_goals=True)); the steps,
    rewards, terminations, goal flags, autoresets (which write the task's goal back) and masks follow the oracle."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task
    from oracle import port

    text = open(golden.task_path("gridworld")).read()
    t, pt = Task.from_text(text), port.Task(text)
    n, steps = 96, 24
    cfg = dict(seed=11, step_reward=-0.5, goal_reward=2.0, max_steps=40)
    pool = rl.DeviceEnvPool(t, n, goals=True, **cfg)
    env = port.Env(pt, **cfg)
    b = env.reset(n, goals=True)
    pool.reset()
    rng = np.random.default_rng(3)
    # goals: at(c) for cells near the start (reachable in a few steps), one per env
    def bits(row):
        return {w * 64 + k for w in range(len(row)) for k in range(64) if (int(row[w]) >> k) & 1}

    near = set(bits(pt.initial))
    for _ in range(2):
        near |= {s for sl in list(near) for r in port.successors(pt, _single(pt, sl)) for s in bits(r[2])}
    cand = sorted(near)
    gp = np.zeros((n, t.words), np.uint64)
    for i in range(n):
        sl = cand[rng.integers(len(cand))]
        gp[i, sl >> 6] = np.uint64(1) << np.uint64(sl & 63)
    b["goal_pos"][:] = gp
    b["goal_neg"][:] = 0
    env.keep_goals_reset(b)
    pool.goal_pos.copy_(torch.from_numpy(gp.view(np.int64)))
    pool.goal_neg.zero_()
    pool.reset(keep_goals=True)
    assert np.array_equal(host(pool.at_goal), b["at_goal"])
    hits = int(b["at_goal"].sum())
    for k in range(steps):
        o = pool.step()
        e = env.step(b)
        hits += int(e["goal"].sum())
        for key in ("reward", "terminated", "truncated", "count", "goal"):
            assert np.array_equal(host(o[key]), e[key]), f"step {k}: {key}"
        assert np.array_equal(host(o["states"]).view(np.uint64), b["states"]), f"step {k}: states"
        assert np.array_equal(host(pool.at_goal), b["at_goal"]), f"step {k}: at_goal"
        assert np.array_equal(host(pool.goal_pos).view(np.uint64), b["goal_pos"]), f"step {k}: goal masks"
    assert hits > 0  # the per-env goals are reached (55 times in this setup)
    pool.check()


def test_goal_masks_past_the_slots_and_refresh(golden):
    from mymyr_amd import rl
    from mymyr_amd._lib import MyaError
    from mymyr_amd.task import Task
    from oracle import port

    text = open(golden.task_path("gridworld")).read()
    t, pt = Task.from_text(text), port.Task(text)
    pool = rl.DeviceEnvPool(t, 8, goals=True)
    pool.reset()
    if pt.slots % 64:
        pool.goal_pos[3, t.words - 1] = -1  # bits past the last fluent slot
        pool.reset(keep_goals=True)
        with pytest.raises(MyaError, match="goal masks set fluent slots"):
            pool.check()
    # refresh tests the current states against the masks written since
    pool.reset()
    pool.goal_pos.copy_(pool.states)  # every env's goal: its own current state
    pool.refresh()
    assert host(pool.at_goal).all()
    pool.check()
