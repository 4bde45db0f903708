"""The oracle's task-table env (oracle/port.py TableEnv: several instances of one domain, per-row instances,
autoresets into next_task_ids, masked resets into other instances, keep_goals resets with per-env masks) against the
compiled reference's rl::HostEnv over TaskTable::create: every reset and every step of the fixture's trajectories
(tests/golden/env_table.json) digest-equal, and the table's domain check with the reference's message."""

import numpy as np
import pytest

from mymyr_amd import workloads
from oracle import port


def load_table(golden, table: str):
    return [port.Task(open(p).read()) for p in workloads.table_files(table, golden.TASKS)]


def table_batch(golden, case: str, inp: dict, W: int) -> dict:
    c = golden.TABLE_CASES[case]
    rows = c["rows"]
    b = {"states": np.zeros((rows, W), np.uint64), "steps": np.zeros(rows, np.int32), "draws": np.zeros(rows, np.uint64),
         "at_goal": np.zeros(rows, np.uint8), "task_ids": inp["task_ids"].copy()}
    if c.get("goals"):
        b["goal_pos"] = np.zeros((rows, W), np.uint64)
        b["goal_neg"] = np.zeros((rows, W), np.uint64)
    if c.get("sampler") is not None:
        b["reset_counts"] = np.zeros(rows, np.uint32)
    for k in ("seeds", "env_ids", "sampling_seeds"):
        if k in inp:
            b[k] = inp[k]
    if c.get("visited"):
        b["visited"] = np.zeros((rows, c["visited"]), np.uint64)
        b["visited_count"] = np.zeros(rows, np.int32)
        b["visited_status"] = np.zeros(1, np.int32)
    return b


def replay_oracle(golden, case: str) -> None:
    g = golden.load("env_table.json")[case]
    c = golden.TABLE_CASES[case]
    ts = load_table(golden, c["table"])
    e = port.TableEnv(ts, sampler=golden.case_sampler(case, len(ts)), suite=c.get("suite", False), **c["env"])
    assert (e.words, e.label_width) == (g["words"], g["label_width"])
    inp = golden.table_inputs(case, len(ts))
    b = table_batch(golden, case, inp, e.words)
    b["count"] = np.zeros(c["rows"], np.int32)
    state = lambda: golden.table_state(b)
    e.reset(b, first_env=5)
    assert golden.arrays_digest(*state(), b["count"]) == g["resets"]["initial"]
    for k in range(c["steps"]):
        if k in inp["clears"]:
            e.clear_visited(b, inp["clears"][k])
            assert golden.arrays_digest(*state()) == g["resets"]["clear" + str(k)], f"{case}: clear_visited at step {k}"
        if k in inp["resets"]:
            mask, new, keep, sample = inp["resets"][k]
            if new is not None:
                b["task_ids"][mask == 1] = new[mask == 1]
            if keep:
                for i in np.nonzero(mask)[0]:
                    t = ts[b["task_ids"][i]]
                    b["goal_pos"][i] = 0
                    b["goal_pos"][i, : t.words] = t.initial
                    b["goal_neg"][i] = 0
            e.reset(b, mask=mask, keep_goals=keep, sample=sample, first_env=5)
            assert golden.arrays_digest(*state(), b["count"]) == g["resets"][str(k)], f"{case}: reset at step {k}"
        acts = golden.given_actions(inp["u"][k], b["count"]) if c["policy"] == "given" else None
        o = e.step(b, first_env=5, actions=acts, next_task_ids=inp["next"][k])
        extra = [o["revisited"]] if c.get("visited") else []
        d = golden.arrays_digest(*state(), o["reward"], o["terminated"], o["truncated"], o["count"], o["schema"], o["binding"],
                                 o["goal"], o["invalid"], o["final_states"], *extra)
        assert d == g["digests"][k], f"{case}: step {k} differs from the reference"
        b["count"] = o["count"]
        if k == golden.TABLE_EXPAND_STEP and case in golden.TABLE_EXPAND_CASES:
            # rl::expand over the table on the batch after this step, with and without drop_noops
            for key, drop in (("all", False), ("drop", True)):
                x = port.table_expand(ts, b["states"], b["task_ids"], drop_noops=drop)
                want = g["expand"][key]
                assert (x["generated"], x["total"]) == (want["generated"], want["total"]), f"{case}: expansion {key}"
                assert golden.expansion_digest(x) == want["digest"], f"{case}: expansion {key}"
                # rl::pad of that expansion (src/mymyr/rl/expand.cpp:799-873) at the automatic k and at k = 3
                for kp in golden.pad_ks(x["offsets"]):
                    p = port.pad(x, len(b["states"]), kp)
                    assert golden.padded_digest(p) == want["pad"][str(kp)]["digest"], f"{case}: pad {key} k={kp}"
                    assert p["overflow"] == want["pad"][str(kp)]["overflow"]


@pytest.mark.parametrize("case", ["gridworld_ids", "gridworld_goals", "transport_ids", "gridworld_sampled", "transport_weighted",
                                  "gridworld_many", "suite_mixed", "gridworld_visited", "transport_visited"])
def test_table_env_matches_reference(golden, case):
    assert case in golden.TABLE_ORACLE_CASES
    replay_oracle(golden, case)


def test_instance_draws(golden):
    """rl::rng::instance_draw (include/mymyr/rl/rng.hpp:94-115) against the reference's draws, uniform and weighted."""
    for d in golden.load("env_table.json")["instance_draws"]:
        thr, idx = golden.sampler_arrays(d["weights"])
        assert port.instance_draw(d["seed"], d["env"], d["reset_count"], d["instances"], thr, idx) == d["draw"]
    # thresholds on, just below and just above the draw's bits (the rule counts those at most the bits)
    for d in golden.load("instance_draw_edges.json"):
        assert port.instance_draw(d["seed"], d["env"], d["reset_count"], d["instances"], d["thresholds"], d["indices"]) == d["draw"]


def test_library_instance_draws_and_sampler(golden):
    """The library's host instance draw (mya_instance_draw) and InstanceSampler arrays against the reference's draws and
    the fixture's restatement of mymyr.rl.InstanceSampler (no device needed)."""
    from mymyr_amd import rl

    for d in golden.load("env_table.json")["instance_draws"]:
        s = rl.InstanceSampler(d["instances"], d["weights"])
        thr, idx = golden.sampler_arrays(d["weights"])
        assert np.array_equal(s.thresholds, thr) and np.array_equal(s.indices, idx)
        assert s.sample(d["seed"], d["env"], d["reset_count"]) == d["draw"]
    with pytest.raises(ValueError, match="positive sum"):
        rl.InstanceSampler(2, [0.0, 0.0])
    from mymyr_amd._lib import lib

    for d in golden.load("instance_draw_edges.json"):
        thr, idx = np.array(d["thresholds"], np.uint32), np.array(d["indices"], np.int32)
        assert lib.mya_instance_draw(d["seed"], d["env"], d["reset_count"], d["instances"], thr.ctypes.data, idx.ctypes.data,
                                     len(idx)) == d["draw"]


def test_sampler_arrays_closed_form(golden):
    """InstanceSampler's arrays (python/mymyr/rl/_sampling.py:29-39) on weights with known cumulative sums."""
    thr, idx = golden.sampler_arrays([1.0, 1.0])
    assert idx.tolist() == [0, 1] and thr.tolist() == [1 << 31]
    thr, idx = golden.sampler_arrays([1.0, 0.0, 3.0])
    assert idx.tolist() == [0, 2] and thr.tolist() == [1 << 30]
    thr, idx = golden.sampler_arrays([0.0, 5.0])
    assert idx.tolist() == [1] and thr.size == 0


def test_visited_overflow_is_reported(golden):
    """The small visited case overflows its 8-slot tables (a key past floor(3H/4) entries is skipped, the count
    saturates and the sticky status is set), as the reference's fixture records."""
    seen = {}
    orig = port.TableEnv.step

    def step(self, b, *a, **k):
        seen["b"] = b
        return orig(self, b, *a, **k)

    port.TableEnv.step = step
    try:
        replay_oracle(golden, "gridworld_visited")
    finally:
        port.TableEnv.step = orig
    b = seen["b"]
    assert b["visited_status"][0] == 1 and (b["visited_count"] == 8).any()
    assert golden.load("env_table.json")["gridworld_visited"]["totals"]["revisited"] > 0


def test_table_fixture_exercises_the_rules(golden):
    """The fixture's trajectories move rows between instances, truncate, terminate, and take invalid actions."""
    g = golden.load("env_table.json")
    for case in golden.TABLE_CASES:
        t = g[case]["totals"]
        assert all(n > 0 for n in t["instance_rows"]), case
        assert t["truncated"] > 0, case
        assert len(g[case]["resets"]) > 2 or golden.TABLE_CASES[case].get("sampler") is None, case
    assert g["gridworld_goals"]["totals"]["invalid"] > 0 and g["gridworld_large"]["totals"]["terminated"] > 0
    # instances of different widths: padding words exist in every table
    for table in workloads.TABLES:
        ts = load_table(golden, table)
        assert len({t.words for t in ts}) > 1


def test_domain_mismatch_message(golden):
    g = golden.load("env_table.json")
    grid = load_table(golden, "gridworld_table")[0]
    trans = load_table(golden, "transport_table")[0]
    with pytest.raises(ValueError) as ex:
        port.TableEnv([grid, trans])
    assert str(ex.value) == g["mismatch"]
    # a planted change in one schema name or predicate kind is caught
    assert port.domain_mismatch(grid, grid) == ""
    other = load_table(golden, "gridworld_table")[1]
    other.schemas[0] = ("walk",) + other.schemas[0][1:]
    assert port.domain_mismatch(grid, other) == "action schema 0 is walk/2, instance 0 has move/2"
    other = load_table(golden, "gridworld_table")[1]
    other.preds[0] = ("F",) + other.preds[0][1:]
    assert port.domain_mismatch(grid, other) == "domain predicate 0 is adj/2 (fluent), instance 0 has adj/2 (static)"


def test_task_id_checks(golden):
    e = port.TableEnv(load_table(golden, "gridworld_table"))
    b = {"states": np.zeros((2, e.words), np.uint64), "steps": np.zeros(2, np.int32), "draws": np.zeros(2, np.uint64),
         "at_goal": np.zeros(2, np.uint8), "count": np.zeros(2, np.int32), "task_ids": np.array([0, 3], np.int32)}
    with pytest.raises(ValueError, match="task id 3 of row 1 is outside the table's 3 instances"):
        e.reset(b)


def test_pad_round_trip_and_cuts():
    """pad against what it must be, independent of the digests: with k at least every count, the valid slots read back
    in row order are the flat expansion; a smaller k keeps each row's first k successors and flags the overflow; a flat
    capacity below the total invalidates exactly the slots at or past it."""
    rng = np.random.default_rng(5)
    counts = np.array([0, 3, 1, 5, 0, 2], np.int64)
    off = np.concatenate([[0], np.cumsum(counts)])
    M, W, L = int(off[-1]), 3, 2
    flat = {"offsets": off, "succ": rng.integers(0, 2**63, (M, W), dtype=np.uint64), "binding": rng.integers(0, 9, (M, L), dtype=np.int32),
            "schema": rng.integers(0, 4, M, dtype=np.int32), "goal": rng.integers(0, 2, M, dtype=np.uint8),
            "succ_hash": rng.integers(0, 2**63, M, dtype=np.uint64), "noop": rng.integers(0, 2, M, dtype=np.uint8),
            "index": rng.integers(0, 50, M, dtype=np.int32), "generated": M, "total": M}
    p = port.pad(flat, len(counts), 8, words=W + 1, label_width=L + 1)
    assert not p["overflow"] and p["count"].tolist() == counts.tolist()
    m = p["mask"].astype(bool)
    assert (p["index"][m] == np.arange(M)).all() and (p["index"][~m] == -1).all()
    assert (p["succ"][m][:, :W] == flat["succ"]).all() and (p["succ"][..., W] == 0).all() and (p["succ"][~m] == 0).all()
    assert (p["binding"][m][:, :L] == flat["binding"]).all() and (p["binding"][..., L] == -1).all()
    for name, fill in (("schema", -1), ("goal", 0), ("succ_hash", 0), ("noop", 0)):
        assert (p[name][m] == flat[name]).all() and (p[name][~m] == fill).all()
    assert (p["canonical"][m] == flat["index"]).all() and (p["canonical"][~m] == -1).all()
    # k = 2: rows with 3 and 5 successors are cut to their first two
    q = port.pad(flat, len(counts), 2)
    assert q["overflow"] and q["mask"].sum(1).tolist() == [0, 2, 1, 2, 0, 2]
    assert q["index"][3].tolist() == [4, 5]
    # capacity 5: flat rows 5.. are missing; row 3 (rows 4..8) keeps only row 4
    c = port.pad({**flat, "succ": flat["succ"][:5], "binding": flat["binding"][:5]}, len(counts), 8, capacity=5)
    assert c["overflow"] and c["index"][3].tolist() == [4] + [-1] * 7 and c["mask"][5].sum() == 0
