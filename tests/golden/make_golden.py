"""Writes the golden fixtures under tests/golden/ from the compiled reference (oracle/_ref, built by oracle/Makefile from
the reference's sources). Run in a container that has the reference checkout:

    make -C oracle && python tests/golden/make_golden.py [--quick]

Outputs (JSON): hash.json, philox.json, slots.json, successors.json, env_<workload>.json, brfs.json, plus the
workload task files under tests/golden/tasks/. --quick skips the slow BrFS fixtures.
"""

from __future__ import annotations

import argparse
import hashlib
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.dirname(os.path.abspath(__file__))))
sys.path.insert(0, ROOT)

from mymyr_amd import gen, workloads  # noqa: E402
from oracle import ref  # noqa: E402
from tests.golden import fixtures as fx  # noqa: E402

M64 = (1 << 64) - 1


def dump(name, obj):
    with open(os.path.join(fx.GOLDEN, name), "w") as f:
        json.dump(obj, f, indent=1, sort_keys=True)
    print("wrote", name, flush=True)


def hex_row(r):
    return [f"{int(x):016x}" for x in r]


def make_hash():
    rng = np.random.default_rng(12345)
    cases = []
    for n in [0, 1, 2, 3, 7, 8, 13, 16, 33, 176]:
        for k in range(3):
            w = rng.integers(0, 2**63, size=n, dtype=np.int64).view(np.uint64) ^ rng.integers(0, 2, size=n, dtype=np.uint64) << np.uint64(63)
            if k == 1 and n > 2:
                w[n // 2:] = 0  # trailing zero words: the state hash ignores them
            seed = int(rng.integers(0, 2**63)) if k == 2 else 0x2D358DCCAA6C78A5
            cases.append({"words": hex_row(w), "seed": f"{seed:016x}", "hash_words": f"{ref.hash_words(w, seed):016x}",
                          "hash_state": f"{ref.hash_state(w):016x}"})
    mix = [{"x": f"{x:016x}", "mix64": f"{int(ref.lib().mref_hash_mix64(x)):016x}"} for x in
           [0, 1, 0x9E3779B97F4A7C15, M64, 0x123456789ABCDEF0]]
    dump("hash.json", {"cases": cases, "mix64": mix})


def make_philox():
    # Random123 kat_vectors, philox4x32 10 (the reference's tests/cpp/rl/test_env.cpp:167-194)
    kats = [
        {"ctr": [0, 0, 0, 0], "key": [0, 0], "out": [0x6627E8D5, 0xE169C58D, 0xBC57AC4C, 0x9B00DBD8]},
        {"ctr": [0xFFFFFFFF] * 4, "key": [0xFFFFFFFF] * 2, "out": [0x408F276D, 0x41C83B0E, 0xA20BC7C6, 0x6D5451FD]},
        {"ctr": [0x243F6A88, 0x85A308D3, 0x13198A2E, 0x03707344], "key": [0xA4093822, 0x299F31D0],
         "out": [0xD16CFE09, 0x94FDCCEB, 0x5001E420, 0x24126EA1]},
    ]
    rng = np.random.default_rng(7)
    draws = []
    for _ in range(64):
        seed = int(rng.integers(0, 2**63))
        env = int(rng.integers(0, 2**32))
        draw = int(rng.integers(0, 2**40))
        count = int(rng.integers(1, 5000))
        draws.append({"seed": seed, "env": env, "draw": draw, "block": ref.philox(seed, env, draw, 0), "count": count,
                      "index": ref.successor_index(seed, env, draw, count)})
    dump("philox.json", {"kats": kats, "draws": draws})


def workload_tasks():
    for name in workloads.TASKS:
        workloads.task_file(name, fx.TASKS)


def make_slots():
    out = {}
    names = sorted(list(fx.SUITE_COUNTS) + fx.LAYOUT_ONLY)
    for name in names + list(workloads.TASKS):
        for atoms in ["auto", "dense", "reachable"]:
            t = ref.RefTask(fx.task_path(name), atoms)
            rec, cid = t.slot_records()
            out[f"{name}:{atoms}"] = {
                "words": t.words, "mode": t.atom_mode, "slots": t.fluent_slots, "dense_fluent": t.dense_fluent,
                "cid_sha": hashlib.sha256(cid.astype(np.uint64).tobytes()).hexdigest(),
                "rec_sha": hashlib.sha256(rec.astype(np.uint32).tobytes()).hexdigest(),
                "cid_head": [int(x) for x in cid[:32]], "initial": hex_row(t.initial_state(t.words)),
            }
    dump("slots.json", out)


def make_successors():
    out = {}
    for name, steps in [("gripper__prob05", 12), ("blocks__probBLOCKS-8-0", 12), ("depot__p02", 8), ("gridworld", 12),
                        ("transport", 8), ("strips", 4), ("transport_xl", 3)]:
        t = ref.RefTask(fx.task_path(name), "dense" if name == "strips" else "auto")
        rng = np.random.default_rng(3)
        row = t.initial_state()
        states = []
        for _ in range(steps):
            sc, bd, rs = t.successors(row)
            states.append({"row": hex_row(row), "count": int(len(sc)), "schema": [int(x) for x in sc],
                           "binding": bd.tolist(), "succ_hash": [f"{ref.hash_state(r):016x}" for r in rs],
                           "goal": t.is_goal(row)})
            if len(sc) == 0:
                break
            row = rs[int(rng.integers(len(sc)))]
        out[name] = states
    dump("successors.json", out)


def env_trajectory(w: workloads.EnvWorkload, rows: int, steps: int, threads: int = 8, first_env: int = 0):
    """The reference HostEnv's per-step digests of `rows` envs with ids first_env, first_env + 1, ... (a batch's rows
    [first_env, first_env + rows): an env's trajectory depends only on its row and its env id)."""
    t = ref.RefTask(fx.task_path(w.name), w.atoms)
    e = ref.RefEnv(t, threads=threads, **w.env)
    N, W, L = rows, t.table_words, max(1, t.label_width)
    S = np.zeros((N, W), np.uint64)
    st = np.zeros(N, np.int32)
    dr = np.zeros(N, np.uint64)
    ag = np.zeros(N, np.uint8)
    cnt = np.zeros(N, np.int32)
    e.reset(S, st, dr, ag, cnt, first_env=first_env)
    digests = []
    totals = {"terminated": 0, "truncated": 0, "reward": 0.0}
    t0 = time.time()
    for k in range(steps):
        R = np.zeros(N, np.float32)
        term = np.zeros(N, np.uint8)
        trunc = np.zeros(N, np.uint8)
        c = np.zeros(N, np.int32)
        sch = np.zeros(N, np.int32)
        bnd = np.zeros((N, L), np.int32)
        g = np.zeros(N, np.uint8)
        e.step(S, st, dr, ag, first_env=first_env, reward=R, terminated=term, truncated=trunc, count=c, schema=sch, binding=bnd, goal=g)
        digests.append(fx.step_digest(N, S, R, term, trunc, c, sch, bnd, g))
        totals["terminated"] += int(term.sum())
        totals["truncated"] += int(trunc.sum())
        totals["reward"] += float(R.astype(np.float64).sum())
    return {"workload": w.name, "rows": N, "steps": steps, "env": w.env, "digests": digests, "totals": totals,
            "first_env": first_env, "ref_seconds": time.time() - t0}


def make_env():
    g = workloads.GRIDWORLD
    dump("env_gridworld.json", env_trajectory(g, g.num_envs, g.steps))
    dump("env_transport.json", env_trajectory(workloads.TRANSPORT, 2048, 64))
    dump("env_transport_xl.json", env_trajectory(workloads.TRANSPORT_XL, 128, 32))
    make_env_long()
    # small instances with goals, truncation and dead ends reached often
    small = workloads.EnvWorkload("gridworld", 256, 200, {"seed": 3, "max_steps": 40, "step_reward": -1.0, "goal_reward": 5.0})
    dump("env_gridworld_truncated.json", env_trajectory(small, 256, 200))
    make_env_small()


def make_env_long():
    # the transport workloads over their whole horizons (512 and 128 steps) on their first rows
    dump("env_transport_long.json", env_trajectory(workloads.TRANSPORT, 256, workloads.TRANSPORT.steps))
    dump("env_transport_xl_long.json", env_trajectory(workloads.TRANSPORT_XL, 64, workloads.TRANSPORT_XL.steps))
    make_env_tail()


def make_env_tail():
    # the transport workloads over their whole horizons on their last 64 rows (env ids N - 64 .. N - 1 of the full
    # batches)
    tr, xl = workloads.TRANSPORT, workloads.TRANSPORT_XL
    dump("env_transport_long_tail.json", env_trajectory(tr, 64, tr.steps, first_env=tr.num_envs - 64))
    dump("env_transport_xl_long_tail.json", env_trajectory(xl, 64, xl.steps, first_env=xl.num_envs - 64))


def env_batch_digests(w: workloads.EnvWorkload, threads: int = 8):
    """The reference HostEnv over a workload's whole batch and horizon: per step, the digest of every row (states as
    their state hashes, fixtures.rows_digest)."""
    t = ref.RefTask(fx.task_path(w.name), w.atoms)
    e = ref.RefEnv(t, threads=threads, **w.env)
    N, W, L = w.num_envs, t.table_words, max(1, t.label_width)
    S = np.zeros((N, W), np.uint64)
    st = np.zeros(N, np.int32)
    dr = np.zeros(N, np.uint64)
    ag = np.zeros(N, np.uint8)
    e.reset(S, st, dr, ag, np.zeros(N, np.int32))
    R, term, trunc = np.zeros(N, np.float32), np.zeros(N, np.uint8), np.zeros(N, np.uint8)
    c, sch, bnd, g = np.zeros(N, np.int32), np.zeros(N, np.int32), np.zeros((N, L), np.int32), np.zeros(N, np.uint8)
    digests = []
    t0 = time.time()
    for k in range(w.steps):
        e.step(S, st, dr, ag, reward=R, terminated=term, truncated=trunc, count=c, schema=sch, binding=bnd, goal=g)
        digests.append(fx.rows_digest(ref.hash_rows(S, t.words), R, term, trunc, c, sch, bnd, g))
        if k % 32 == 0:
            print(w.name, "step", k, round(time.time() - t0, 1), flush=True)
    return {"workload": w.name, "rows": N, "steps": w.steps, "env": w.env, "digests": digests, "ref_seconds": time.time() - t0}


def make_env_batch():
    """Whole-batch digests of the transport workloads over their whole horizons (every env id, every step)."""
    dump("env_transport_batch.json", env_batch_digests(workloads.TRANSPORT))
    dump("env_transport_xl_batch.json", env_batch_digests(workloads.TRANSPORT_XL))


def make_env_small():
    # a trajectory short enough for the oracle's pure-Python restatement
    tiny = workloads.EnvWorkload("gridworld", 16, 60, {"seed": 3, "max_steps": 20, "step_reward": -1.0, "goal_reward": 5.0})
    dump("env_gridworld_small.json", env_trajectory(tiny, 16, 60))


def table_batch_arrays(case: str, inp: dict, W: int) -> dict:
    """The batch arrays of a table case, zeroed, with the case's task ids, per-row keys and reset counters."""
    c = fx.TABLE_CASES[case]
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


def table_trajectory(case: str) -> dict:
    """A task-table env trajectory of the compiled reference (rl::HostEnv over TaskTable::create): the digest of the
    batch after the first reset, after each masked reset and after every step."""
    c = fx.TABLE_CASES[case]
    table, rows, steps, policy = c["table"], c["rows"], c["steps"], c["policy"]
    ts = [ref.RefTask(p) for p in workloads.table_files(table, fx.TASKS)]
    I, W = len(ts), max(t.words for t in ts)
    L = max(1, max(t.label_width for t in ts))
    inp = fx.table_inputs(case, I)
    e = ref.RefTableEnv(ts, sampler=fx.case_sampler(case, I), suite=c.get("suite", False), **c["env"])
    b = table_batch_arrays(case, inp, W)
    cnt = np.zeros(rows, np.int32)
    init = [t.initial_state(W) for t in ts]
    e.reset(b, cnt, first_env=5)
    state = lambda: fx.table_state(b)
    resets = {"initial": fx.arrays_digest(*state(), cnt)}
    digests = []
    totals = {"terminated": 0, "truncated": 0, "invalid": 0, "goal": 0, "instance_rows": [0] * I}
    for k in range(steps):
        if k in inp["clears"]:
            e.clear_visited(b, inp["clears"][k])
            resets["clear" + str(k)] = fx.arrays_digest(*state())
        if k in inp["resets"]:
            mask, new_ids, keep, sample = inp["resets"][k]
            if new_ids is not None:
                b["task_ids"][mask == 1] = new_ids[mask == 1]
            if keep:
                for i in np.nonzero(mask)[0]:
                    b["goal_pos"][i] = init[b["task_ids"][i]]
                    b["goal_neg"][i] = 0
            e.reset(b, cnt, mask=mask, keep_goals=keep, sample=sample, first_env=5)
            resets[str(k)] = fx.arrays_digest(*state(), cnt)
        actions = fx.given_actions(inp["u"][k], cnt) if policy == "given" else None
        R, term, trunc = np.zeros(rows, np.float32), np.zeros(rows, np.uint8), np.zeros(rows, np.uint8)
        cc, sch, bnd = np.zeros(rows, np.int32), np.zeros(rows, np.int32), np.zeros((rows, L), np.int32)
        g, inv, fs = np.zeros(rows, np.uint8), np.zeros(rows, np.uint8), np.zeros((rows, W), np.uint64)
        rv = np.zeros(rows, np.uint8) if c.get("visited") else None
        e.step(b, first_env=5, actions=actions, next_task_ids=inp["next"][k], reward=R, terminated=term, truncated=trunc, count=cc,
               schema=sch, binding=bnd, goal=g, invalid=inv, final_states=fs, revisited=rv)
        digests.append(fx.arrays_digest(*state(), R, term, trunc, cc, sch, bnd, g, inv, fs, *([] if rv is None else [rv])))
        if rv is not None:
            totals["revisited"] = totals.get("revisited", 0) + int(rv.sum())
        cnt = cc
        if k == fx.TABLE_EXPAND_STEP and case in fx.TABLE_EXPAND_CASES:
            expansions = {}
            for drop in (False, True):
                x = ref.table_expand(ts, b["states"], b["task_ids"], drop_noops=drop)
                pads = {}
                for kp in fx.pad_ks(x["offsets"]):
                    p = ref.table_pad(ts, b["states"], b["task_ids"], kp, drop_noops=drop)
                    pads[str(kp)] = {"digest": fx.padded_digest(p), "overflow": p["overflow"]}
                expansions["drop" if drop else "all"] = {"digest": fx.expansion_digest(x), "generated": x["generated"],
                                                         "total": x["total"], "noops": int(np.asarray(x["noop"]).sum()), "pad": pads}
        for key, a in (("terminated", term), ("truncated", trunc), ("invalid", inv), ("goal", g)):
            totals[key] += int(a.sum())
        for i in range(I):
            totals["instance_rows"][i] += int((b["task_ids"] == i).sum())
    out = {"case": case, "table": table, "rows": rows, "steps": steps, "words": W, "label_width": L, "resets": resets,
           "digests": digests, "totals": totals}
    if case in fx.TABLE_EXPAND_CASES:
        out["expand"] = expansions
    return out


def make_env_table():
    out = {case: table_trajectory(case) for case in fx.TABLE_CASES}
    for case, r in out.items():
        print(case, r["totals"], flush=True)
    # the table's domain check (TaskTable::domain_mismatch, src/mymyr/rl/task_table.cpp:75-100)
    mixed = [ref.RefTask(workloads.table_files("gridworld_table", fx.TASKS)[0]), ref.RefTask(workloads.table_files("transport_table", fx.TASKS)[0])]
    try:
        ref.RefTableEnv(mixed)
        out["mismatch"] = None
    except RuntimeError as ex:
        out["mismatch"] = str(ex)
    # instance draws (rl::rng::instance_draw, include/mymyr/rl/rng.hpp:94-115): uniform and weighted
    rng = np.random.default_rng(31)
    draws = []
    for weights in (None, [1.0, 1.0], [1.0, 0.0, 3.0], [0.5, 2.0, 0.0, 1.5, 7.0]):
        thr, idx = fx.sampler_arrays(weights)
        n = 5 if weights is None else len(weights)
        for _ in range(24):
            seed, env, count = int(rng.integers(0, 2**63)), int(rng.integers(0, 2**32)), int(rng.integers(0, 2**32))
            draws.append({"weights": weights, "seed": seed, "env": env, "reset_count": count, "instances": n,
                          "draw": ref.instance_draw(seed, env, count, n, thr, idx)})
    out["instance_draws"] = draws
    dump("env_table.json", out)


def make_instance_draw_edges():
    """Instance draws whose sampler thresholds sit on the draw's own 32 bits, one below and one above them: the rule
    counts the thresholds at most the bits (include/mymyr/rl/rng.hpp:94-115), which a random draw almost never tests.
    The oracle only places the thresholds; the draws are the reference's."""
    from oracle import port

    rng = np.random.default_rng(41)
    out = []
    for _ in range(24):
        seed, env, count = int(rng.integers(0, 2**63)), int(rng.integers(0, 2**32)), int(rng.integers(0, 2**32))
        bits = port.fmix32(port.fmix32((seed & 0xFFFFFFFF) ^ port.fmix32(((seed >> 32) & 0xFFFFFFFF) ^ 0x53414D50))
                           ^ port.fmix32(env) ^ port.fmix32(count ^ 0x9E3779B9))
        for thr in ([bits], [max(bits, 1) - 1], [min(bits + 1, 0xFFFFFFFF)], [max(bits, 1) - 1, bits, min(bits + 1, 0xFFFFFFFF)]):
            t = np.array(sorted(thr), np.uint32)
            idx = np.arange(10, 10 + len(t) + 1, dtype=np.int32)
            out.append({"seed": seed, "env": env, "reset_count": count, "instances": 16, "thresholds": [int(x) for x in t],
                        "indices": [int(x) for x in idx], "draw": ref.instance_draw(seed, env, count, 16, t, idx)})
    dump("instance_draw_edges.json", out)


def make_visited_mask():
    """Visited tables filled by the reference's visited_insert (empty, short, at the 3H/4 threshold, saturated, probe
    chains of one home slot, hash 0 and its reserved key) and rl::visited_mask over queries with -1 padding, with and
    without a row mapping."""
    rng = np.random.default_rng(17)
    H, n = 16, 7
    table = np.zeros((n, H), np.uint64)
    count = np.zeros(n, np.int32)
    inserts = [[], [0, 5, 77], list(range(1, 13)), list(range(100, 120)), [16 * i + 3 for i in range(1, 9)],
               [int(x) for x in rng.integers(1, 2**63, 6, dtype=np.uint64)], [0x9E3779B97F4A7C15, 0]]
    present = []
    for r, hs in enumerate(inserts):
        hs = [int(h) for h in hs]
        p, count[r] = ref.visited_insert(table[r], 0, np.array(hs, np.uint64))
        present.append(p.tolist())
        inserts[r] = hs
    q = [0, 5, 77, 13, 6, 12, 100, 115, 119, 19, 35, 147, 3, 0x9E3779B97F4A7C15] + [h for hs in inserts for h in hs]
    q += [int(x) for x in rng.integers(0, 2**63, 20, dtype=np.uint64)]
    hashes = np.array(q * 2, np.uint64)
    parent = rng.integers(-1, n, len(hashes)).astype(np.int32)
    rows = np.array([3, -1, 0, 6, 2, 1, 5, 4, 4, -1], np.int32)
    parent_m = rng.integers(-1, len(rows), len(hashes)).astype(np.int32)
    out = {"H": H, "inserts": [[str(h) for h in hs] for hs in inserts], "present": present, "table": [[str(int(x)) for x in t] for t in table],
           "count": count.tolist(), "hashes": [str(int(h)) for h in hashes], "parent": parent.tolist(),
           "mask": ref.visited_mask(table, count, hashes, parent).tolist(), "rows": rows.tolist(), "parent_mapped": parent_m.tolist(),
           "mask_mapped": ref.visited_mask(table, count, hashes, parent_m, rows).tolist()}
    print("visited_mask", sum(out["mask"]), sum(out["mask_mapped"]), count.tolist(), flush=True)
    dump("visited_mask.json", out)


WITNESS_TASKS = {"witness_order_5": 5, "witness_order_0": 0}


def make_brfs_witness():
    """BrFS with witness pruning over schemas with several witness parameters (bound by the matcher in an order other
    than the parameter order): counts, fingerprints and the plans whose labels carry the witness choices."""
    for name, seed in WITNESS_TASKS.items():
        with open(fx.task_path(name), "w") as f:
            f.write(gen.witness_task(seed=seed))
    out = {"witness_order_5": brfs_record("witness_order_5", stop_at_goal=False),
           "witness_order_5:goal": brfs_record("witness_order_5", stop_at_goal=True),
           "witness_order_0:goal": brfs_record("witness_order_0", stop_at_goal=True),
           "witness_order_0:cut": brfs_record("witness_order_0", stop_at_goal=False, max_states=50000),
           "rovers__p02": brfs_record("rovers__p02", stop_at_goal=False),
           "rovers__p02:goal": brfs_record("rovers__p02", stop_at_goal=True),
           "rovers__p02:expanded": brfs_record("rovers__p02", stop_at_goal=False, max_expanded=20000)}
    dump("brfs_witness.json", out)


WIDE_TASKS = {"transport_w20_3": dict(locations=20, trucks=4, packages=50, goals=1, seed=3),
              "transport_w20_7": dict(locations=20, trucks=4, packages=50, goals=1, seed=7)}
# a transport task of 2208-word rows (141,312 atoms), past the 2048 words the state set keeps in registers
LONG_TASKS = {"transport_w2208": dict(locations=128, trucks=48, packages=768, goals=32, seed=5)}


def make_brfs_long():
    """BrFS over rows of more than 2048 words (the state set's long-row shape): the 2208-word transport task to a
    depth bound, a max_states cut and a goal-count beam."""
    for name, kw in LONG_TASKS.items():
        with open(fx.task_path(name), "w") as f:
            f.write(gen.transport(**kw))
    out = {"transport_w2208:depth2": brfs_record("transport_w2208", stop_at_goal=False, max_depth=2),
           "transport_w2208:cut": brfs_record("transport_w2208", stop_at_goal=False, max_states=30000),
           "transport_w2208:beam": brfs_record("transport_w2208", stop_at_goal=False, max_depth=8, layer_order="goal_count",
                                               beam_width=64)}
    for k, v in out.items():
        print(k, v["states"], v["expanded"], v["status"], flush=True)
    dump("brfs_long.json", out)


def make_brfs_wide():
    """BrFS over rows wider than 16 words (the lifted-expansion driver): typed transport instances of 20 words (plans of
    3 and 4 actions, cuts, an expansion budget), the transport workload's 176-word rows at max_states and depth cuts,
    and a 19-word task with witness parameters searched with witness pruning off."""
    for name, kw in WIDE_TASKS.items():
        with open(fx.task_path(name), "w") as f:
            f.write(gen.transport(**kw))
    with open(fx.task_path("witness_wide"), "w") as f:
        f.write(gen.witness_task(items=60, places=32, seed=2))
    out = {"transport_w20_3:goal": brfs_record("transport_w20_3", stop_at_goal=True),
           "transport_w20_7:goal": brfs_record("transport_w20_7", stop_at_goal=True),
           "transport_w20_3:cut": brfs_record("transport_w20_3", stop_at_goal=False, max_states=200000),
           "transport_w20_7:expanded": brfs_record("transport_w20_7", stop_at_goal=False, max_expanded=5000),
           "transport:cut": brfs_record("transport", stop_at_goal=False, max_depth=12, max_states=100000),
           "transport:depth2": brfs_record("transport", stop_at_goal=False, max_depth=2),
           "witness_wide:cut": brfs_record("witness_wide", "dense", stop_at_goal=False, witness_pruning=False, max_states=50000),
           "witness_wide:witness_cut": brfs_record("witness_wide", "dense", stop_at_goal=False, max_states=50000),
           "witness_wide:witness_goal": brfs_record("witness_wide", "dense", stop_at_goal=True, max_states=300000),
           "witness_wide:witness_depth": brfs_record("witness_wide", "dense", stop_at_goal=False, max_depth=2)}
    dump("brfs_wide.json", out)


def make_successors_witness():
    """Canonical successor listings with witness pruning on (the reference's Successors::generate, one successor per
    effect-relevant binding, the witness the matcher binds first) along seeded random walks of tasks with witness
    parameters: per state its schema and binding order and the successors' hash_state."""
    out = {}
    for name, atoms, steps in [("rovers__p02", "auto", 10), ("witness_wide", "dense", 10), ("witness_order_5", "auto", 10),
                               ("witness_order_0", "auto", 10)]:
        t = ref.RefTask(fx.task_path(name), atoms)
        rng = np.random.default_rng(5)
        row = t.initial_state()
        states = []
        for _ in range(steps):
            sc, bd, rs = t.successors(row, witness=True)
            full, _, frs = t.successors(row)
            states.append({"row": hex_row(row), "count": int(len(sc)), "schema": [int(x) for x in sc],
                           "binding": bd.tolist(), "succ_hash": [f"{ref.hash_state(r):016x}" for r in rs],
                           "all": int(len(full))})
            if len(full) == 0:
                break
            row = frs[int(rng.integers(len(full)))]
        out[name] = {"atoms": atoms, "states": states}
    dump("successors_witness.json", out)


def task_predicates(path):
    """(kind, arity) per predicate of a task file (its P section: "<kind> <arity> <name>" lines)."""
    preds = []
    with open(path) as f:
        lines = f.read().split("\n")
    i = next(k for k, l in enumerate(lines) if l.startswith("P "))
    for l in lines[i + 1: i + 1 + int(lines[i].split()[1])]:
        kind, ar = l.split()[:2]
        preds.append((kind, int(ar)))
    return preds


def goal_conditions(name, atoms, seed):
    """AnyOf goal conditions for a task: per random walk of 3, 5 and 8 steps from the initial state, two or three of the
    reached state's atoms that the initial state does not hold (positive) and one atom it does not hold (negative); then a condition with a false static
    literal and its negation (never holds: left out)."""
    t = ref.RefTask(fx.task_path(name), atoms)
    preds = task_predicates(fx.task_path(name))
    rng = np.random.default_rng(seed)
    rec, _ = t.slot_records()
    conds = []
    for depth in (3, 5, 8):
        row = t.initial_state()
        for _ in range(depth):
            sc, _, rs = t.successors(row)
            if len(sc) == 0:
                break
            row = rs[int(rng.integers(len(sc)))]
        t.refresh()
        rec, _ = t.slot_records()
        init = t.initial_state(len(row))
        bits = [s for s in range(len(rec)) if (int(row[s // 64]) >> (s % 64)) & 1]
        new_bits = [s for s in bits if not (int(init[s // 64]) >> (s % 64)) & 1] or bits
        off = [s for s in range(len(rec)) if s not in set(bits)]
        lits = []
        for s in rng.choice(new_bits, size=min(len(new_bits), 2 + depth % 2), replace=False):
            p = int(rec[s][0])
            lits.append([p, True, [int(x) for x in rec[s][1:1 + preds[p][1]]]])
        if off:
            s = int(rng.choice(off))
            p = int(rec[s][0])
            lits.append([p, False, [int(x) for x in rec[s][1:1 + preds[p][1]]]])
        conds.append(lits)
    # a static literal and its negation: one of them is false, so the condition never holds (left out)
    static = [p for p, (k, a) in enumerate(preds) if k == "S" and a == 1]
    if static:
        p = static[0]
        conds.append([[p, False, [0]], [p, True, [0]]] + conds[0])
    return conds


def make_brfs_goals():
    """BrfsOptions::goal as GoalSpec::AnyOf (search::any_of over ground conditions): goal stops, plans and goal states,
    counts of goal states over whole searches, a max_states cut, the lazy slots' resolution of goal atoms at the search's
    start, and the result's words, fluent_slots, threads_used, store and message."""
    out = {}
    for name, atoms, seed, kws in [
            ("gripper__prob05", "auto", 1, [dict(stop_at_goal=True), dict(stop_at_goal=False, max_states=30000)]),
            ("blocks__probBLOCKS-8-0", "auto", 2, [dict(stop_at_goal=True), dict(stop_at_goal=False, max_depth=6)]),
            ("transport_w20_3", "auto", 3, [dict(stop_at_goal=True), dict(stop_at_goal=False, max_states=60000)]),
            ("blocks__probBLOCKS-8-0", "lazy", 2, [dict(stop_at_goal=True), dict(stop_at_goal=False, max_depth=5)])]:
        conds = goal_conditions(name, "auto", seed)
        for i, kw in enumerate(kws):
            t = ref.RefTask(fx.task_path(name), atoms)
            r = ref.brfs(t, goal=conds, fingerprint=True, **kw)
            r.pop("seconds")
            r["options"] = kw
            r["goal"] = conds
            r["atoms"] = atoms
            out[f"{name}:{atoms}:{i}"] = r
            print("goals", name, atoms, kw, r["states"], r["status"], r["goal_states"], flush=True)
        # no condition can hold: every state is tested, none is a goal
        t = ref.RefTask(fx.task_path(name), atoms)
        r = ref.brfs(t, goal=[conds[-1][:2]], fingerprint=True, stop_at_goal=True, max_states=5000)
        r.pop("seconds")
        r["options"] = dict(stop_at_goal=True, max_states=5000)
        r["goal"] = [conds[-1][:2]]
        r["atoms"] = atoms
        out[f"{name}:{atoms}:never"] = r
    dump("brfs_goals.json", out)


def walk_states(t, depths, seed):
    """One state per entry of `depths`: the end of a seeded random walk of that many steps from the initial state (a walk
    that reaches a dead end stops there)."""
    rng = np.random.default_rng(seed)
    out = []
    for d in depths:
        row = t.initial_state()
        for _ in range(d):
            _, _, rows = t.successors(row)
            if len(rows) == 0:
                break
            row = rows[rng.integers(len(rows))]
        out.append(row.copy())
    return out


OPTION_CASES = {
    # key: (task, atoms, start walk depth or None, blocked walk depths, include the start among the blocked, options)
    "gripper__prob05:blocked_goal": ("gripper__prob05", "auto", None, [1, 1, 3, 3, 3, 4], False, dict(stop_at_goal=True)),
    "gripper__prob05:blocked_all": ("gripper__prob05", "auto", None, [2, 3, 4, 5, 6, 6, 8, 10], True, dict(stop_at_goal=False)),
    "gripper__prob05:start_goal": ("gripper__prob05", "auto", 4, [], False, dict(stop_at_goal=True)),
    "gripper__prob05:blocked_cut": ("gripper__prob05", "auto", None, [3, 4, 5, 5, 6, 7, 8, 9], False,
                                    dict(stop_at_goal=False, max_states=20000)),
    "gripper__prob05:start_blocked_expanded": ("gripper__prob05", "auto", 2, [3, 4, 4, 5, 6, 7], False,
                                               dict(stop_at_goal=False, max_expanded=3000)),
    "gripper__prob05:timed0": ("gripper__prob05", "auto", None, [], False, dict(stop_at_goal=False, max_seconds=0.0)),
    "blocks__probBLOCKS-8-0:blocked_goal": ("blocks__probBLOCKS-8-0", "auto", None, [1, 2, 2, 3, 4, 5, 5, 6, 8, 10], False,
                                           dict(stop_at_goal=True)),
    "logistics00__probLOGISTICS-6-1:start_blocked": ("logistics00__probLOGISTICS-6-1", "auto", 3, [1, 2, 3, 4, 5, 6], True,
                                                     dict(stop_at_goal=True)),
    "strips:blocked_cut": ("strips", "dense", None, [2, 3, 4, 5, 6, 6, 7, 7, 8, 8, 9, 10, 11, 11, 12, 12], False,
                           dict(stop_at_goal=False, max_depth=12, max_states=1 << 20)),
    "transport_w20_3:blocked_goal": ("transport_w20_3", "auto", None, [1, 1, 2, 2, 2, 3], False, dict(stop_at_goal=True)),
    "transport_w20_3:start_goal": ("transport_w20_3", "auto", 2, [], False, dict(stop_at_goal=True)),
    "transport_w20_3:blocked_cut": ("transport_w20_3", "auto", 1, [2, 3, 3, 4, 5, 6], True,
                                    dict(stop_at_goal=False, max_states=200000)),
}


def make_brfs_options():
    """BrfsOptions::start and blocked_states (and max_seconds 0) of the reference brfs(): the start state and the
    blocked states are ends of seeded random walks from the initial state; the results (counts, pruned, statuses,
    fingerprints, plans) of the reference's single-threaded search."""
    out = {}
    for i, (key, (name, atoms, start_d, blocked_d, block_start, kw)) in enumerate(OPTION_CASES.items()):
        t = ref.RefTask(fx.task_path(name), atoms)
        start = None if start_d is None else walk_states(t, [start_d], 100 + i)[0]
        blocked = walk_states(t, blocked_d, 200 + i)
        if block_start:
            blocked.append(t.initial_state() if start is None else start)
        bl = np.array(blocked, dtype=np.uint64).reshape(-1, t.table_words)
        r = ref.brfs(t, start=start, blocked_states=bl if len(bl) else None, **kw)
        r.pop("seconds")
        r["options"] = kw
        r["start"] = None if start is None else hex_row(start)
        r["blocked"] = [hex_row(b) for b in bl]
        r["atoms"] = atoms
        out[key] = r
        print(key, r["states"], r["pruned"], r["status"], len(r.get("plan", [])), flush=True)
    dump("brfs_options.json", out)


def goal_lines(text):
    lines = text.rstrip("\n").split("\n")
    gi = [i for i, l in enumerate(lines) if l.startswith("G ")][0]
    return lines[gi + 1: gi + 1 + int(lines[gi].split()[1])]


# tasks with the optional C (collapsed parameters) and EG (encoding goal) sections: a suite task's text with the sections
# appended; a collapsed parameter without a representative (-1) leaves its schema without actions
SECTION_TASKS = {
    "sections_gripper_rep": ("gripper__prob05", "C 2\n0 2 1 0\n1 0 0 5\n", True),
    "sections_gripper_norep": ("gripper__prob05", "C 1\n1 0 0 -1\n", True),
    "sections_blocks_norep": ("blocks__probBLOCKS-8-0", "C 2\n0 1 1 3\n2 0 1 -1\n", False),
    "sections_logistics_eg": ("logistics00__probLOGISTICS-6-1", "", True),
}


def make_sections():
    """BrFS of the reference on suite tasks with C and EG sections (tests/golden/tasks/sections_*.txt, written here)."""
    out = {}
    for name, (base, c, eg) in SECTION_TASKS.items():
        text = open(fx.task_path(base)).read().rstrip("\n") + "\n" + c
        if eg:
            g = goal_lines(text)
            text += "EG 1 %d\n" % len(g) + "\n".join(reversed(g)) + "\n"
        with open(fx.task_path(name), "w") as f:
            f.write(text)
        out[name + ":goal"] = brfs_record(name, stop_at_goal=True)
        out[name + ":all"] = brfs_record(name, stop_at_goal=False, max_states=200000)
        print(name, out[name + ":all"]["states"], out[name + ":goal"]["status"], flush=True)
    dump("brfs_sections.json", out)


def make_pool():
    """Digests of every batch the reference CpuEnvPool returns over each pool case's scripted calls."""
    out = {}
    for case, c in fx.POOL_CASES.items():
        t = ref.RefTask(fx.task_path(case))
        pool = ref.RefPool(t, c["num_envs"], threads=4, first_env=c["first_env"], **c["env"])
        digests = fx.run_pool_script(pool, case, max(1, t.label_width))
        assert pool.pending == 0
        out[case] = {"digests": digests, "label_width": max(1, t.label_width)}
        print("pool", case, len(digests), flush=True)
    dump("pool.json", out)


def brfs_record(name, atoms="auto", ref_threads=1, **kw):
    """The reference brfs() on a task; `options` holds the BrfsOptions a device search repeats. Cuts are recorded
    from the default single-threaded search (threads=1, the flat store for these widths): the reference's multi-threaded
    search gives the same ids and counts on whole layers (tests/cpp/search/test_brfs.cpp:113-141) but not at a
    max_states cut, where it neither records the cut layer nor stores the same states."""
    t = ref.RefTask(fx.task_path(name), atoms)
    r = ref.brfs(t, threads=ref_threads, **kw)
    r.pop("seconds")
    r["options"] = kw
    return r


def make_brfs(quick: bool):
    out = {"suite": {}, "budget": {}, "strips": {}}
    for name in fx.SUITE_COUNTS:
        if quick and fx.SUITE_COUNTS[name][0] > 200000:
            continue
        out["suite"][name] = brfs_record(name, stop_at_goal=False)
        out["budget"][name] = brfs_record(name, stop_at_goal=False, max_states=20000)
        out["budget"][name + ":goal"] = brfs_record(name, stop_at_goal=True)
        out["budget"][name + ":expanded"] = brfs_record(name, stop_at_goal=False, max_expanded=3000)
        print(name, out["suite"][name]["states"], flush=True)
    for ms in ([1 << 20] if quick else [1 << 20, 1 << 22, 1 << 24, 1 << 26]):
        out["strips"][str(ms)] = brfs_record("strips", "dense", max_depth=12, max_states=ms,
                                             stop_at_goal=False)
        print("strips", ms, flush=True)
    out["strips"]["depth3"] = brfs_record("strips", "dense", max_depth=3, stop_at_goal=False)
    out["strips"]["expanded5000"] = brfs_record("strips", "dense", max_depth=12, max_expanded=5000, stop_at_goal=False)
    out["strips"]["expanded300000"] = brfs_record("strips", "dense", max_depth=12, max_expanded=300000,
                                                  stop_at_goal=False)
    out["strips"]["goal"] = brfs_record("strips", "dense", max_depth=12, max_states=1 << 24, stop_at_goal=True)
    dump("brfs.json", out)


def make_brfs_suite_add():
    """Adds the suite, budget, goal and expanded-cut records of the suite tasks that brfs.json does not hold yet (the
    step keeps the existing records, whose strips cuts take long to regenerate)."""
    path = os.path.join(fx.GOLDEN, "brfs.json")
    with open(path) as f:
        out = json.load(f)
    for name in fx.SUITE_COUNTS:
        if name in out["suite"]:
            continue
        out["suite"][name] = brfs_record(name, stop_at_goal=False)
        out["budget"][name] = brfs_record(name, stop_at_goal=False, max_states=20000)
        out["budget"][name + ":goal"] = brfs_record(name, stop_at_goal=True)
        out["budget"][name + ":expanded"] = brfs_record(name, stop_at_goal=False, max_expanded=3000)
        print(name, out["suite"][name]["states"], flush=True)
    # the goal states of the solved budget records (auto slots) as canonical atom ids: a device search over other slots
    # (dense) compares its goal state through them
    for key, rec in out["budget"].items():
        if rec["solved"] and "goal_cids" not in rec:
            rec["goal_cids"] = goal_cids(ref.RefTask(fx.task_path(key.split(":")[0]), "auto"), rec["goal_state"])
    dump("brfs.json", out)


# small budgets at the edges (the reference's own checks: python tests/python/test_search.py:120-136), over the ground
# driver (gripper), the wide one (20-word transport rows) and lazy slots
EDGE_OPTIONS = {
    "states1": dict(max_states=1, stop_at_goal=False), "states2": dict(max_states=2, stop_at_goal=False),
    "states50": dict(max_states=50, stop_at_goal=False), "expanded0": dict(max_expanded=0, stop_at_goal=False),
    "expanded1": dict(max_expanded=1, stop_at_goal=False), "expanded5": dict(max_expanded=5, stop_at_goal=False),
    "depth0": dict(max_depth=0, stop_at_goal=False), "depth1": dict(max_depth=1, stop_at_goal=False),
    "depth2": dict(max_depth=2, stop_at_goal=False), "depth0_goal": dict(max_depth=0, stop_at_goal=True),
    "depth2_goal": dict(max_depth=2, stop_at_goal=True), "states2_goal": dict(max_states=2, stop_at_goal=True),
}
EDGE_TASKS = [("gripper__prob05", "auto"), ("transport_w20_3", "auto"), ("gripper__prob05", "lazy")]


def make_brfs_edges():
    """The reference brfs() at budgets of zero, one and a few states, expansions and layers (brfs_edges.json)."""
    out = {}
    for name, atoms in EDGE_TASKS:
        for key, kw in EDGE_OPTIONS.items():
            r = lazy_record(name, **kw) if atoms == "lazy" else brfs_record(name, atoms, **kw)
            r["atoms"] = atoms
            out[f"{name}:{atoms}:{key}"] = r
            print(name, atoms, key, r["states"], r["expanded"], r["status"], flush=True)
    dump("brfs_edges.json", out)


# BrfsOptions::goal as GoalSpec::Custom: a state is a goal iff hash_state(state) % m == r (no atom goal expresses it),
# through the ground driver (gripper) and the wide one (20-word transport rows); and, under lazy slots (whose row layout
# is the device's own), iff the state has k true atoms, a test no slot numbering changes
CUSTOM_GOAL_CASES = {
    "gripper__prob05:goal": ("gripper__prob05", "auto", {"goal_hash": (1000, 7)}, dict(stop_at_goal=True)),
    "gripper__prob05:all": ("gripper__prob05", "auto", {"goal_hash": (1000, 7)}, dict(stop_at_goal=False)),
    "gripper__prob05:cut": ("gripper__prob05", "auto", {"goal_hash": (97, 5)}, dict(stop_at_goal=False, max_states=30000)),
    "transport_w20_3:goal": ("transport_w20_3", "auto", {"goal_hash": (500, 3)}, dict(stop_at_goal=True)),
    "transport_w20_3:cut": ("transport_w20_3", "auto", {"goal_hash": (61, 2)}, dict(stop_at_goal=False, max_states=40000)),
    "blocks__probBLOCKS-8-0:lazy_goal": ("blocks__probBLOCKS-8-0", "lazy", {"goal_atoms": 10}, dict(stop_at_goal=True)),
    "blocks__probBLOCKS-8-0:lazy_cut": ("blocks__probBLOCKS-8-0", "lazy", {"goal_atoms": 12},
                                        dict(stop_at_goal=False, max_states=30000)),
}


def make_brfs_custom_goal():
    """The reference brfs() with a custom goal test (brfs_custom_goal.json)."""
    out = {}
    for key, (name, atoms, test, kw) in CUSTOM_GOAL_CASES.items():
        r = brfs_record(name, atoms, **test, **kw)
        r.update({k: list(v) if isinstance(v, tuple) else v for k, v in test.items()})
        r["atoms"] = atoms
        if atoms == "lazy" and "goal_state" in r:
            # the goal state's atoms by canonical id (the device numbers lazy slots in its own order)
            t = ref.RefTask(fx.task_path(name), "lazy")
            ref.brfs(t, **test, **kw)
            r["goal_cids"] = goal_cids(t, r["goal_state"])
        out[key] = r
        print(key, r["states"], r["expanded"], r["goal_states"], r["status"], len(r.get("plan", [])), flush=True)
    dump("brfs_custom_goal.json", out)


def make_brfs_strips_large():
    """Adds the strips workload's cut at max_states = 2^28 to brfs.json (the single-threaded reference search: about
    1.2 G successors and 25 GB of host memory, some 20 minutes), keeping the existing records."""
    path = os.path.join(fx.GOLDEN, "brfs.json")
    with open(path) as f:
        out = json.load(f)
    ms = 1 << 28
    out["strips"][str(ms)] = brfs_record("strips", "dense", max_depth=12, max_states=ms, stop_at_goal=False)
    print("strips", ms, flush=True)
    dump("brfs.json", out)


LAYER_CASES = [
    ("gripper__prob05", "auto", dict(layer_order="in_order", beam_width=50)),
    ("gripper__prob05", "auto", dict(layer_order="reverse")),
    ("gripper__prob05", "auto", dict(layer_order="randomized", seed=5)),
    ("gripper__prob05", "auto", dict(layer_order="randomized", seed=5, stop_at_goal=True)),
    ("gripper__prob05", "auto", dict(layer_order="goal_count")),
    ("gripper__prob05", "auto", dict(layer_order="goal_count", prefer_more_satisfied_goals=False, randomize_ties=True, seed=11,
                                     beam_width=100)),
    ("gripper__prob05", "auto", dict(layer_order="in_order", max_next_layer_states=300)),
    ("gripper__prob05", "auto", dict(layer_order="randomized", seed=9, max_next_layer_states=1000, stop_at_goal=True)),
    ("gripper__prob05", "auto", dict(layer_order="popcount", beam_width=40)),
    ("blocks__probBLOCKS-8-0", "auto", dict(layer_order="goal_count", beam_width=200, stop_at_goal=True)),
    ("blocks__probBLOCKS-8-0", "auto", dict(layer_order="reverse", max_states=20000)),
    ("blocks__probBLOCKS-8-0", "auto", dict(layer_order="neg_popcount_mod3", randomize_ties=True, seed=2, max_next_layer_states=5000)),
    ("logistics00__probLOGISTICS-6-1", "auto", dict(layer_order="goal_count", beam_width=1000, stop_at_goal=True)),
    ("depot__p02", "auto", dict(layer_order="goal_count", randomize_ties=True, seed=4, max_next_layer_states=2000, max_expanded=30000)),
    ("transport_w20_3", "auto", dict(layer_order="goal_count", beam_width=64, stop_at_goal=True)),
    ("transport_w20_3", "auto", dict(layer_order="randomized", seed=3, max_next_layer_states=2000, max_depth=6)),
    ("transport_w20_3", "auto", dict(layer_order="reverse", max_depth=4)),
    ("blocks__probBLOCKS-8-0", "lazy", dict(layer_order="goal_count", beam_width=200, stop_at_goal=True)),
    ("gripper__prob05", "lazy", dict(layer_order="randomized", seed=7, max_next_layer_states=800)),
]


def make_brfs_layers():
    """The reference brfs() under BrfsOptions::layers (ordered layers, randomized orders, goal-count and scored ranks,
    beams and max_next_layer_states) on ground, wide-row and lazy tasks: counts, layer counts, fingerprints, plans."""
    out = {}
    for name, atoms, kw in LAYER_CASES:
        opts = dict(kw)
        opts.setdefault("stop_at_goal", False)
        ref_kw = dict(opts)
        if ref_kw["layer_order"] in fx.LAYER_SCORERS:
            ref_kw["layer_order"] = fx.LAYER_SCORERS[ref_kw["layer_order"]]
        t = ref.RefTask(fx.task_path(name), atoms)
        r = ref.brfs(t, witness_pruning=atoms != "lazy", **ref_kw)
        r.pop("seconds")
        if atoms == "lazy" and r["solved"]:
            r["goal_cids"] = goal_cids(t, r["goal_state"])
        r["options"] = opts
        r["atoms"] = atoms
        key = f"{name}:{atoms}:" + ",".join(f"{k}={v}" for k, v in sorted(opts.items()))
        out[key] = r
        print(key, r["states"], r["expanded"], r["status"], flush=True)
    dump("brfs_layers.json", out)


EVENT_CASES = [
    ("gripper__prob05", dict(stop_at_goal=False, max_states=3000)),
    ("caldera-split-opt18-adl__p04", dict(stop_at_goal=True)),
    ("parcprinter-opt11-strips__p03", dict(stop_at_goal=True)),
    ("transport_w20_3", dict(stop_at_goal=True)),
    ("blocks__probBLOCKS-8-0", dict(stop_at_goal=False, max_states=2000, blocked=3)),
    ("gripper__prob05", dict(stop_at_goal=False, layer_order="reverse", beam_width=30, max_depth=6)),
    ("depot__p02", dict(stop_at_goal=False, layer_order="in_order", max_next_layer_states=200, max_depth=5)),
    ("miconic-simpleadl__s10-2", dict(stop_at_goal=False, max_states=2000)),
]


def make_brfs_events():
    """The reference observer's events (search::SearchObserver, include/mymyr/search/control.hpp:157-186) of small
    searches, as the harness records them (7-word records: start, expand, generate, prune, pass, solution, end; states
    by hash_state, bindings by a polynomial hash): per case the count of each kind, the sha256 of all records and the
    first 60 records. blocked=k blocks the first k successors of the initial state."""
    out = {}
    for name, kw in EVENT_CASES:
        kw = dict(kw)
        t = ref.RefTask(fx.task_path(name), "auto")
        blocked = None
        if "blocked" in kw:
            k = kw.pop("blocked")
            _, _, rows = t.successors(t.initial_state())
            blocked = rows[:k]
        r = ref.brfs(t, record_events=True, blocked_states=blocked, **kw)
        ev = r["events"]
        key = f"{name}:" + ",".join(f"{a}={b}" for a, b in sorted(kw.items())) + (f",blocked={len(blocked)}" if blocked is not None else "")
        out[key] = {"options": kw, "blocked": None if blocked is None else [hex_row(x) for x in blocked],
                    "counts": {str(int(k)): int((ev[:, 0] == k).sum()) for k in range(7)},
                    "sha256": hashlib.sha256(np.ascontiguousarray(ev).astype("<u8").tobytes()).hexdigest(),
                    "head": [[f"{int(x):x}" for x in row] for row in ev[:60]],
                    "states": r["states"], "expanded": r["expanded"], "generated": r["generated"], "status": r["status"]}
        print(key, out[key]["counts"], flush=True)
    dump("brfs_events.json", out)


LAZY_TASKS = ["gripper__prob05", "blocks__probBLOCKS-8-0", "depot__p02", "pegsol-08-strips__p22", "visitall__visitall_x-6_y-3_r-100",
              "miconic__s7-4", "logistics00__probLOGISTICS-6-1", "driverlog__p03", "rovers__p02"]


def goal_cids(t, words_hex):
    """The canonical ids of a goal state's atoms (its words as hex strings) under the task's current slots, ascending."""
    _, cid = t.slot_records()
    out = []
    for w, x in enumerate(words_hex):
        v = int(x, 16)
        while v:
            b = (v & -v).bit_length() - 1
            v &= v - 1
            out.append(int(cid[w * 64 + b]))
    return sorted(out)


def lazy_record(name, **kw):
    """The reference brfs() over a task loaded with lazy slots (witness pruning off, as the lifted expansion runs it):
    counts, fingerprint and plan, plus what does not depend on the order the slots were numbered in: the number of
    slots the search left, the sha256 of their canonical ids sorted, and the goal state's atoms by canonical id."""
    t = ref.RefTask(fx.task_path(name), "lazy")
    r = ref.brfs(t, witness_pruning=False, **kw)
    r.pop("seconds")
    _, cid = t.slot_records()
    r["slots"] = t.fluent_slots
    r["slot_cids_sha"] = hashlib.sha256(np.sort(cid.astype(np.uint64)).tobytes()).hexdigest()
    if "goal_state" in r:
        r["goal_cids"] = goal_cids(t, r.pop("goal_state"))
    r["options"] = dict(kw, witness_pruning=False)
    return r


def make_lazy():
    """Lazy atom slots: the slot table right after loading (the initial state's atoms in its atom order), and BrFS runs
    whose states' atoms intern as the search meets them (exhaustive, to the first goal, and a max_states cut)."""
    out = {"initial": {}, "brfs": {}}
    for name in LAZY_TASKS + ["transport_w20_3", "transport"]:
        t = ref.RefTask(fx.task_path(name), "lazy")
        rec, cid = t.slot_records()
        out["initial"][name] = {"words": t.words, "slots": t.fluent_slots, "cid": [int(x) for x in cid],
                                "rec_sha": hashlib.sha256(rec.astype(np.uint32).tobytes()).hexdigest(),
                                "initial": hex_row(t.initial_state(t.words))}
    for name in LAZY_TASKS:
        out["brfs"][name] = lazy_record(name, stop_at_goal=False, fingerprint=True)
        out["brfs"][name + ":goal"] = lazy_record(name, stop_at_goal=True, fingerprint=True)
        print("lazy", name, out["brfs"][name]["states"], out["brfs"][name]["slots"], flush=True)
    out["brfs"]["transport_w20_3:goal"] = lazy_record("transport_w20_3", stop_at_goal=True, fingerprint=True)
    out["brfs"]["gripper__prob05:cut"] = lazy_record("gripper__prob05", stop_at_goal=False, fingerprint=True, max_states=20000)
    out["brfs"]["blocks__probBLOCKS-8-0:depth"] = lazy_record("blocks__probBLOCKS-8-0", stop_at_goal=False, fingerprint=True, max_depth=6)
    dump("lazy.json", out)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--quick", action="store_true")
    ap.add_argument("--only", default="")
    a = ap.parse_args()
    workload_tasks()
    steps = {"hash": make_hash, "philox": make_philox, "slots": make_slots, "successors": make_successors, "env": make_env,
             "env_small": make_env_small, "env_long": make_env_long, "env_tail": make_env_tail, "pool": make_pool,
             "brfs_witness": make_brfs_witness, "brfs_wide": make_brfs_wide, "successors_witness": make_successors_witness, "brfs_goals": make_brfs_goals, "brfs_options": make_brfs_options, "sections": make_sections, "env_table": make_env_table, "visited_mask": make_visited_mask, "lazy": make_lazy, "brfs": lambda: make_brfs(a.quick),
             "brfs_suite_add": make_brfs_suite_add, "brfs_layers": make_brfs_layers, "brfs_long": make_brfs_long,
             "brfs_events": make_brfs_events, "brfs_strips_large": make_brfs_strips_large,
             "brfs_edges": make_brfs_edges, "env_batch": make_env_batch,
             "instance_draw_edges": make_instance_draw_edges,
             "brfs_custom_goal": make_brfs_custom_goal}
    for k, f in steps.items():
        if not a.only or k in a.only.split(","):
            f()


if __name__ == "__main__":
    main()
