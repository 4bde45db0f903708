"""Lazy atom slots on the device (TaskOptions::Atoms::Lazy, include/mymyr/task/atom_index.hpp:19-22; the device side:
include/mymyr/cuda/generator.hpp:20-24 and the arena widening of cuda/src/brfs.cpp:130-152): a task starts with the
initial state's atoms, and the BrFS, the flat expansion and the successor listing intern the atoms their successors
add without a slot (ascending canonical id per device launch), widening the rows as the slots outgrow them.

The slot numbering depends on the order searches meet the atoms (the reference's CPU search numbers them as its thread
meets them), so what is compared is what does not depend on it: counts, statuses, fingerprints (over canonical ids),
plans, the goal state's atoms and, for searches that ran to their end, the set of atoms that got slots, all against
the compiled reference's brfs() over the same task loaded with lazy slots (tests/golden/lazy.json), and expansions
against the same task with frozen slots, atom for atom."""

import hashlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

KEYS = ["states", "expanded", "generated", "goal_states", "layers", "fingerprint", "layer_counts", "exhausted", "solved"]
STATUS = {0: "solved", 1: "exhausted", 2: "out_of_states", 3: "out_of_time", 4: "cancelled"}


def atoms_of(cid, rows):
    """Per row, the sorted canonical ids of its set bits (cid: the task's slot -> canonical id table)."""
    out = []
    for r in np.asarray(rows, dtype=np.uint64).reshape(len(rows), -1):
        ids = []
        for w, x in enumerate(r):
            x = int(x)
            while x:
                b = (x & -x).bit_length() - 1
                x &= x - 1
                ids.append(int(cid[w * 64 + b]))
        out.append(sorted(ids))
    return out


def lazy_keys():
    from tests.golden import fixtures

    return sorted(fixtures.load("lazy.json")["brfs"])


@pytest.mark.parametrize("key", lazy_keys())
def test_lazy_brfs_equals_reference(golden, key):
    from mymyr_amd import search
    from mymyr_amd.task import Task

    exp = golden.load("lazy.json")["brfs"][key]
    name = key.split(":")[0]
    print(f"lazy brfs: {key}", flush=True)
    t = Task.from_text_file(golden.task_path(name), "lazy")
    words0 = t.words
    r = search.brfs(t, **exp["options"])
    got = {"states": r.states, "expanded": r.expanded, "generated": r.generated, "goal_states": r.num_goal_states,
           "layers": r.layers, "fingerprint": r.fingerprint, "layer_counts": r.layer_counts, "exhausted": r.exhausted,
           "solved": r.solved}
    bad = {k: (got[k], exp[k]) for k in KEYS if got[k] != exp[k]}
    assert not bad, (key, bad)
    assert r.status == STATUS[exp["status"]]
    rec, cid = t.slot_records()
    assert t.words == max(1, (t.fluent_slots + 63) // 64) and len(set(cid.tolist())) == t.fluent_slots
    assert [int(x) for x in cid[: len(golden.load("lazy.json")["initial"][name]["cid"])]] == \
        golden.load("lazy.json")["initial"][name]["cid"]  # the initial state's atoms keep the first slots
    if exp["solved"]:
        assert [[a.schema, *a.binding] for a in r.plan] == exp["plan"] and r.cost == exp["cost"]
        assert atoms_of(cid, [r.goal_state])[0] == exp["goal_cids"]
    if exp["status"] != 2:
        # a search that ran to its end (or to its goal) met the same atoms as the reference's
        assert t.fluent_slots == exp["slots"]
        assert hashlib.sha256(np.sort(cid.astype(np.uint64)).tobytes()).hexdigest() == exp["slot_cids_sha"]
    if t.words > words0:
        print(f"  rows widened {words0} -> {t.words} words", flush=True)


@pytest.mark.parametrize("name", ["blocks__probBLOCKS-8-0", "depot__p02", "transport_w20_3"])
def test_lazy_expansion_equals_frozen(golden, name):
    """rl.expand over a lazy task, layer after layer from the initial state: the same successor counts, labels and goal
    flags as over the task with frozen slots, and successors with the same atoms; the rows widen as atoms intern."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task

    lazy = Task.from_text_file(golden.task_path(name), "lazy")
    frozen = Task.from_text_file(golden.task_path(name), "auto")
    dev = torch.device("cuda:0")
    fl = torch.from_numpy(frozen.initial_state().view(np.int64)).reshape(1, -1).to(dev)
    lz = torch.from_numpy(lazy.initial_state().view(np.int64)).reshape(1, -1).to(dev)
    _, fcid = frozen.slot_records()
    for depth in range(5):
        a = rl.expand(frozen, fl, goal=True)
        b = rl.expand(lazy, lz, goal=True)
        print(f"lazy expand {name} depth {depth}: {fl.shape[0]} rows, {a['total']} successors, lazy rows {b['succ'].shape[1]} words",
              flush=True)
        assert not a["overflow"] and not b["overflow"]
        for k in ("offsets", "parent", "schema", "binding", "goal"):
            assert torch.equal(a[k].cpu(), b[k].cpu()), (name, depth, k)
        _, lcid = lazy.slot_records()
        assert atoms_of(fcid, a["succ"].cpu().numpy().view(np.uint64)) == atoms_of(lcid, b["succ"].cpu().numpy().view(np.uint64))
        assert b["succ"].shape[1] >= lazy.words
        # the next layer: up to 256 successors, the same ones on both sides
        take = torch.arange(0, a["succ"].shape[0], max(1, a["succ"].shape[0] // 256), device=dev)[:256]
        fl, lz = a["succ"][take].contiguous(), b["succ"][take].contiguous()


def test_lazy_successor_listing_equals_frozen(golden):
    """rl.successors (the canonical listing) over a lazy task: the frozen task's labels, successors with its atoms."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task

    name = "depot__p02"
    lazy = Task.from_text_file(golden.task_path(name), "lazy")
    frozen = Task.from_text_file(golden.task_path(name), "auto")
    dev = torch.device("cuda:0")
    W = max(frozen.words, (lazy.dense_fluent + 63) // 64)
    f0 = np.zeros((1, W), np.uint64)
    f0[0, : frozen.words] = frozen.initial_state()
    l0 = np.zeros((1, W), np.uint64)
    l0[0, : lazy.words] = lazy.initial_state()
    fc, fs, fb, fr = rl.successors(frozen, torch.from_numpy(f0.view(np.int64)).to(dev), cap=256)
    lc, ls, lb, lr = rl.successors(lazy, torch.from_numpy(l0.view(np.int64)).to(dev), cap=256)
    n = int(fc[0])
    assert int(lc[0]) == n and n > 0
    assert torch.equal(fs[:, :n].cpu(), ls[:, :n].cpu()) and torch.equal(fb[:, :n].cpu(), lb[:, :n].cpu())
    _, fcid = frozen.slot_records()
    _, lcid = lazy.slot_records()
    assert atoms_of(fcid, fr[0, :n].cpu().numpy().view(np.uint64)) == atoms_of(lcid, lr[0, :n].cpu().numpy().view(np.uint64))


def test_lazy_task_searched_again(golden):
    """A second search over a lazy task starts with the slots the first left (wider rows from the start) and finds the
    same counts, fingerprint and plan; a search after an expansion that interned atoms too."""
    from mymyr_amd import rl, search
    from mymyr_amd.task import Task

    exp = golden.load("lazy.json")["brfs"]["blocks__probBLOCKS-8-0:goal"]
    t = Task.from_text_file(golden.task_path("blocks__probBLOCKS-8-0"), "lazy")
    first = search.brfs(t, **exp["options"])
    words = t.words
    again = search.brfs(t, **exp["options"])
    assert t.words == words and t.fluent_slots == exp["slots"]
    for r in (first, again):
        assert (r.states, r.expanded, r.generated, r.fingerprint, r.layer_counts) == \
            (exp["states"], exp["expanded"], exp["generated"], exp["fingerprint"], exp["layer_counts"])
        assert [[a.schema, *a.binding] for a in r.plan] == exp["plan"]
    # an expansion first: its atoms take slots in another order, which changes nothing the search reports
    t2 = Task.from_text_file(golden.task_path("blocks__probBLOCKS-8-0"), "lazy")
    s0 = torch.from_numpy(t2.initial_state().view(np.int64)).reshape(1, -1).to("cuda:0")
    x = rl.expand(t2, s0)
    rl.expand(t2, x["succ"].contiguous())
    r = search.brfs(t2, **exp["options"])
    assert (r.states, r.generated, r.fingerprint) == (exp["states"], exp["generated"], exp["fingerprint"])
    _, cid = t2.slot_records()
    assert atoms_of(cid, [r.goal_state])[0] == exp["goal_cids"]


@pytest.mark.parametrize("key", ["rovers__p02", "rovers__p02:goal", "rovers__p02:expanded", "witness_order_5:goal",
                                 "witness_order_0:goal", "witness_order_0:cut"])
def test_lazy_search_with_witness_pruning(golden, key):
    """A lazy task's search runs over the lifted expansion, which prunes witness parameters as the reference's matcher
    does (the reference's default options): over rovers and tasks whose two witness parameters the matcher binds in an
    order other than the parameter order, counts, statuses, fingerprints and plans (whose labels carry the witness
    objects found first) equal the compiled reference's over the frozen task (tests/golden/brfs_witness.json)."""
    from mymyr_amd import search
    from mymyr_amd.task import Task

    exp = golden.load("brfs_witness.json")[key]
    name = key.split(":")[0]
    print(f"lazy witness brfs: {key}", flush=True)
    t = Task.from_text_file(golden.task_path(name), "lazy")
    r = search.brfs(t, fingerprint=True, **exp["options"])
    got = {"states": r.states, "expanded": r.expanded, "generated": r.generated, "goal_states": r.num_goal_states,
           "layers": r.layers, "fingerprint": r.fingerprint, "layer_counts": r.layer_counts, "exhausted": r.exhausted,
           "solved": r.solved}
    bad = {k: (got[k], exp[k]) for k in KEYS if got[k] != exp[k]}
    assert not bad, (key, bad)
    assert r.status == STATUS[exp["status"]]
    if exp["solved"]:
        assert [[a.schema, *a.binding] for a in r.plan] == exp["plan"] and r.cost == exp["cost"]
    # the same search with witness pruning off generates every binding: at least as many successors
    if key == "rovers__p02:expanded":
        off = search.brfs(Task.from_text_file(golden.task_path(name), "lazy"), fingerprint=True, witness_pruning=False,
                          **exp["options"])
        assert off.generated >= r.generated


@pytest.mark.parametrize("key", ["transport:cut", "transport:depth2", "transport_w20_3:cut", "transport_w20_7:expanded",
                                 "transport_w20_7:goal"])
def test_lazy_wide_rows_equal_the_frozen_reference(golden, key):
    """Transport tasks of 20 and 176 words loaded with lazy slots: the rows start at 1 to 4 words and widen several times
    (every stored state moved to the wider set in id order) while the search runs to a max_states cut, a depth bound,
    an expansion budget or a goal. Counts, fingerprints and plans do not depend on the slots, so they equal the
    compiled reference's over the frozen task (tests/golden/brfs_wide.json), and the goal state holds the same atoms."""
    from mymyr_amd import search
    from mymyr_amd.task import Task

    exp = golden.load("brfs_wide.json")[key]
    name = key.split(":")[0]
    print(f"lazy wide brfs: {key}", flush=True)
    t = Task.from_text_file(golden.task_path(name), "lazy")
    words0 = t.words
    r = search.brfs(t, fingerprint=True, **exp["options"])
    got = {"states": r.states, "expanded": r.expanded, "generated": r.generated, "goal_states": r.num_goal_states,
           "layers": r.layers, "fingerprint": r.fingerprint, "layer_counts": r.layer_counts, "exhausted": r.exhausted,
           "solved": r.solved}
    bad = {k: (got[k], exp[k]) for k in KEYS if got[k] != exp[k]}
    assert not bad, (key, bad)
    assert r.status == STATUS[exp["status"]]
    assert t.words > words0
    if exp["solved"]:
        assert [[a.schema, *a.binding] for a in r.plan] == exp["plan"] and r.cost == exp["cost"]
        frozen = Task.from_text_file(golden.task_path(name), "auto")
        _, fcid = frozen.slot_records()
        _, lcid = t.slot_records()
        want = np.array([int(x, 16) for x in exp["goal_state"]], dtype=np.uint64)
        assert atoms_of(lcid, [r.goal_state])[0] == atoms_of(fcid, [want])[0]
