"""The device flat expansion (rl.expand, include/mymyr/rl/expand.hpp:1-130) against the reference's successor
listings (counts, schemas, bindings and successor hashes written by the compiled reference), the oracle's expansion
(goal and no-op flags, the no-op filter) and the properties the reference's own tests check
(tests/python/test_rl_noops.py: the kept rows are the full expansion's rows at the kept positions, index is the
position in the parent's full order, succ_hash is the hash of succ)."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def host(t):
    return t.cpu().numpy()


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int64)).cuda()


def load(golden, name):
    from mymyr_amd.task import Task
    from oracle import port

    atoms = "dense" if name == "strips" else "auto"
    text = open(golden.task_path(name)).read()
    return Task.from_text(text, atoms), port.Task(text, atoms)


@pytest.mark.parametrize("name", ["gripper__prob05", "blocks__probBLOCKS-8-0", "depot__p02", "gridworld", "transport",
                                  "strips"])
def test_expand_matches_reference_listing(golden, name):
    from mymyr_amd import rl
    from oracle import port

    g = golden.load("successors.json")[name]
    t, pt = load(golden, name)
    rows = np.array([[int(x, 16) for x in s["row"]][: t.words] for s in g], dtype=np.uint64)
    x = rl.expand(t, dev(rows), goal=True, hashes=True, noops=True, index=True)
    off = host(x["offsets"])
    assert list(np.diff(off)) == [s["count"] for s in g] and x["generated"] == x["total"] == off[-1]
    succ = host(x["succ"]).view(np.uint64)
    sch, bnd, hsh = host(x["schema"]), host(x["binding"]), host(x["succ_hash"]).view(np.uint64)
    for i, s in enumerate(g):
        a, b = off[i], off[i + 1]
        assert list(sch[a:b]) == s["schema"]
        if b > a:
            assert bnd[a:b, : len(s["binding"][0])].tolist() == s["binding"]
        assert [f"{int(h):016x}" for h in hsh[a:b]] == s["succ_hash"]
        assert list(host(x["parent"])[a:b]) == [i] * (b - a) and list(host(x["index"])[a:b]) == list(range(b - a))
    # flags against the oracle: goal tests and no-ops of the successor rows
    assert list(host(x["goal"]).astype(bool)) == [port.is_goal(pt, r) for r in succ]
    assert np.array_equal(host(x["noop"]).astype(bool), np.all(succ == rows[host(x["parent"])], axis=1))


def random_rows(pt, n, seed):
    rng = np.random.default_rng(seed)
    rows = np.zeros((n, pt.words), np.uint64)
    for i in range(n):
        for s in rng.choice(pt.slots, size=pt.slots // 2, replace=False):
            rows[i, s >> 6] |= np.uint64(1) << np.uint64(s & 63)
    return rows


@pytest.mark.parametrize("name", ["noop_switches", "strips"])
def test_drop_noops(golden, name):
    """Dropping no-ops keeps exactly the oracle's rows; they are the full expansion's rows at the kept positions."""
    from mymyr_amd import rl
    from oracle import port

    t, pt = load(golden, name)
    if name == "noop_switches":
        rows = np.array([[1], [3], [0], [2]], np.uint64)  # live; live and p (idle only); dead; p only
    else:
        rows = random_rows(pt, 24, seed=5)
    full = rl.expand(t, dev(rows), goal=True, hashes=True, noops=True, index=True)
    kept = rl.expand(t, dev(rows), goal=True, hashes=True, noops=True, drop_noops=True)
    exp = port.expand(pt, list(rows), drop_noops=True)
    assert kept["generated"] == full["total"] and kept["total"] == exp["total"] and not kept["overflow"]
    assert list(host(kept["offsets"])) == exp["offsets"]
    assert list(host(kept["index"])) == exp["index"] and list(host(kept["schema"])) == exp["schema"]
    assert list(host(kept["succ_hash"]).view(np.uint64)) == exp["succ_hash"]
    assert list(host(kept["noop"]).astype(bool)) == exp["noop"] and list(host(kept["goal"]).astype(bool)) == exp["goal"]
    # the kept rows are the full rows at offsets[parent] + index
    foff = host(full["offsets"])
    at = foff[host(kept["parent"])] + host(kept["index"])
    for key in ("succ", "schema", "binding", "succ_hash", "noop", "goal"):
        assert np.array_equal(host(kept[key]), host(full[key])[at]), key
    if name == "strips":
        assert 0 < exp["total"] < exp["generated"]  # the random states do have no-op successors


def test_capacity_overflow(golden):
    """Rows past the capacity are counted, not written; offsets keep the true counts. With drop_noops the overflow
    reports the counts before dropping."""
    from mymyr_amd import rl
    from oracle import port

    t, pt = load(golden, "transport")
    g = golden.load("successors.json")["transport"]
    rows = np.array([[int(x, 16) for x in s["row"]][: t.words] for s in g], dtype=np.uint64)
    full = rl.expand(t, dev(rows), hashes=True)
    cap = full["total"] // 2
    part = rl.expand(t, dev(rows), capacity=cap, hashes=True)
    assert part["overflow"] and part["generated"] == part["total"] == full["total"]
    assert np.array_equal(host(part["offsets"]), host(full["offsets"]))
    assert np.array_equal(host(part["succ"]), host(full["succ"])[:cap])
    assert np.array_equal(host(part["succ_hash"]), host(full["succ_hash"])[:cap])
    over = rl.expand(t, dev(rows), capacity=cap, drop_noops=True)
    assert over["overflow"] and over["total"] == over["generated"] == full["total"]
    assert np.array_equal(host(over["offsets"]), host(full["offsets"]))


def test_narrow_successor_rows(golden):
    """Successor rows narrower than the task: the successors that do not fit are zero rows and words_needed is the
    widest trimmed successor among them; the hashes stay exact."""
    from mymyr_amd import rl

    t, pt = load(golden, "transport")
    g = golden.load("successors.json")["transport"]
    rows = np.array([[int(x, 16) for x in s["row"]][: t.words] for s in g], dtype=np.uint64)
    full = rl.expand(t, dev(rows), hashes=True)
    fs = host(full["succ"]).view(np.uint64)
    width = np.array([max([k + 1 for k in range(fs.shape[1]) if r[k]] or [0]) for r in fs])
    w = int(np.median(width))
    narrow = rl.expand(t, dev(rows), hashes=True, words=w)
    ns = host(narrow["succ"]).view(np.uint64)
    fit = width <= w
    assert np.array_equal(ns[fit], fs[fit, :w]) and not ns[~fit].any()
    assert narrow["words_needed"] == (width[~fit].max() if (~fit).any() else 0)
    assert np.array_equal(host(narrow["succ_hash"]), host(full["succ_hash"]))


def test_expand_argument_errors(golden):
    from mymyr_amd import _lib, rl
    from mymyr_amd._lib import MyaError, lib

    t, pt = load(golden, "gridworld")
    rows = torch.zeros((4, t.words), dtype=torch.int64, device="cuda")
    wide = torch.zeros((4, t.words + 1), dtype=torch.int64, device="cuda")
    wide[2, -1] = 1  # an atom past the task's words
    with pytest.raises(MyaError, match="atoms past the task's slots"):
        rl.expand(t, wide)
    assert t.words > 1
    with pytest.raises(MyaError, match="the task needs"):
        rl.expand(t, rows[:, : t.words - 1].contiguous())
    # drop_noops without index, through the C ABI
    opts = _lib.ExpandOptions(1, 0, 1, 1)
    x = _lib.Expansion()
    x.capacity = 8
    assert lib.mya_expand(t.handle, rows.data_ptr(), 4, t.words, ctypes.byref(opts), ctypes.byref(x), None) != 0
    assert b"drop_noops requires index" in lib.mya_last_error()


@pytest.mark.parametrize("name", ["witness_wide", "rovers__p02", "witness_order_5", "witness_order_0"])
def test_expand_with_witness_pruning_matches_reference_listing(golden, name):
    """rl.expand with witness_pruning (the reference's ExpandOptions::witness_pruning, include/mymyr/rl/expand.hpp:81):
    along a seeded walk, per state the count, schemas, bindings (whose witness objects are the ones the reference's
    matcher binds first) and successor hashes equal the compiled reference's Successors::generate with witness pruning
    on; the 19-word task's listings are shorter than its full ones."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task

    g = golden.load("successors_witness.json")[name]
    t = Task.from_text_file(golden.task_path(name), g["atoms"])
    states = g["states"]
    rows = np.array([[int(x, 16) for x in s["row"]][: t.words] + [0] * max(0, t.words - len(s["row"])) for s in states],
                    dtype=np.uint64)
    print(f"witness expand: {name} rows {len(rows)}", flush=True)
    x = rl.expand(t, dev(rows), hashes=True, witness_pruning=True)
    off = host(x["offsets"])
    assert list(np.diff(off)) == [s["count"] for s in states]
    sch, bnd, hsh = host(x["schema"]), host(x["binding"]), host(x["succ_hash"]).view(np.uint64)
    for i, s in enumerate(states):
        a, b = off[i], off[i + 1]
        assert list(sch[a:b]) == s["schema"], (i, list(sch[a:b])[:8], s["schema"][:8])
        if b > a:
            assert bnd[a:b, : len(s["binding"][0])].tolist() == s["binding"], i
        assert [f"{int(h):016x}" for h in hsh[a:b]] == s["succ_hash"], i
    full = rl.expand(t, dev(rows))
    assert list(np.diff(host(full["offsets"]))) == [s["all"] for s in states]
    if name == "witness_wide":
        assert all(s["count"] < s["all"] for s in states)
