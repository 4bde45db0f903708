"""The oracle's CPU restatement (oracle/port.py) pinned against the reference: the golden vectors the compiled
reference wrote (tests/golden/*.json), the reference's own fixtures (Random123 vectors, determinism digests, suite
counts) and closed forms. When oracle/_ref is built here, it is also compared directly on fresh inputs."""

import numpy as np
import pytest

from mymyr_amd import gen, workloads
from oracle import port


def test_hash_golden(golden):
    g = golden.load("hash.json")
    for c in g["cases"]:
        w = [int(x, 16) for x in c["words"]]
        assert port.hash_words(w, int(c["seed"], 16)) == int(c["hash_words"], 16)
        assert port.hash_state(w) == int(c["hash_state"], 16)
    for m in g["mix64"]:
        assert port.mix64(int(m["x"], 16)) == int(m["mix64"], 16)


def test_hash_properties():
    # the state hash ignores trailing zero words and separates single-bit states (tests/cpp/core/test_hash.cpp:12-75)
    w = [0x1234, 0, 0xFFFF, 0, 0]
    assert port.hash_state(w) == port.hash_state(w[:3])
    assert port.hash_words(w) != port.hash_words(w[:3])
    seen = {port.hash_state([1 << b if i == k else 0 for i in range(4)]) for k in range(4) for b in range(64)}
    assert len(seen) == 256


def test_philox_known_answers(golden):
    g = golden.load("philox.json")
    for k in g["kats"]:
        assert port.philox4x32_10(k["ctr"], *k["key"]) == k["out"]
    # the draw layout: counter (draw lo, draw hi, env, purpose), key (seed lo, seed hi) (test_env.cpp:190-193)
    assert port.philox_block(0x0123456789ABCDEF, 7, 0x100000002, 0) == port.philox4x32_10([2, 1, 7, 0], 0x89ABCDEF, 0x01234567)
    for d in g["draws"]:
        assert port.philox_block(d["seed"], d["env"], d["draw"], 0) == d["block"]
        assert port.successor_index(d["seed"], d["env"], d["draw"], d["count"]) == d["index"]


def test_below_is_the_high_word_of_the_product():
    """rng::below takes the high 64 bits of the 128-bit product x * n from 32x32 partial products (rng.hpp:73-78): the
    mathematics fixes it as floor(x * n / 2^64). The golden draws' counts (< 5000) leave the low partial product's
    carry almost never visible, so random and extreme x and n pin it here."""
    rng = np.random.default_rng(17)
    xs = [int(x) for x in rng.integers(0, 2**63, size=2000, dtype=np.int64)] + [2**64 - 1, 2**63, 2**32 - 1, 2**32, 1, 0]
    ns = [int(n) for n in rng.integers(1, 2**32, size=2000, dtype=np.int64)] + [2**32 - 1, 2**31, 65536, 3, 1, 2]
    for x in xs:
        x2 = x | ((x & 1) << 63)  # top bit set for half of them
        for n in ns[:: 97]:
            assert port.below(x2, n) == (x2 * n) >> 64
    for x, n in zip(xs, ns):
        assert port.below(x, n) == (x * n) >> 64


def test_index_in_range():
    for n in (1, 2, 3, 7, 1000, 0xFFFFFFFF):
        for d in range(50):
            assert port.successor_index(42, d % 13, d, n) < n


SMALL_LAYOUTS = ["gripper__prob05", "blocks__probBLOCKS-8-0", "depot__p02", "driverlog__p03", "rovers__p02",
                 "sokoban-opt08-strips__p14", "snake-opt18-strips__p05", "gridworld", "strips", "transport"]


@pytest.mark.parametrize("name", SMALL_LAYOUTS)
def test_layout_golden(golden, name):
    import hashlib

    slots = golden.load("slots.json")
    text = open(golden.task_path(name)).read()
    for atoms in ["auto", "dense", "reachable"]:
        t = port.Task(text, atoms)
        g = slots[f"{name}:{atoms}"]
        assert t.words == g["words"] and t.mode == g["mode"] and t.slots == g["slots"], (name, atoms)
        assert t.fluent_count == g["dense_fluent"]
        assert hashlib.sha256(np.array(t.slot_cid, dtype=np.uint64).tobytes()).hexdigest() == g["cid_sha"]
        assert [f"{int(x):016x}" for x in t.initial] == g["initial"]


@pytest.mark.parametrize("name", ["gripper__prob05", "blocks__probBLOCKS-8-0", "depot__p02", "gridworld", "transport", "strips"])
def test_successors_golden(golden, name):
    g = golden.load("successors.json")[name]
    t = port.Task(open(golden.task_path(name)).read(), "dense" if name == "strips" else "auto")
    for s in g:
        row = np.array([int(x, 16) for x in s["row"]], dtype=np.uint64)[: t.words]
        succ = port.successors(t, row)
        assert len(succ) == s["count"]
        assert [x[0] for x in succ] == s["schema"]
        assert [list(x[1]) + [-1] * (len(s["binding"][0]) - len(x[1])) for x in succ] == s["binding"] if succ else True
        assert [f"{port.hash_state(x[2]):016x}" for x in succ] == s["succ_hash"]
        assert port.is_goal(t, row) == s["goal"]


def test_env_golden_small(golden):
    """The restated HostEnv step against the reference's trajectory (first rows of the truncating gridworld)."""
    g = golden.load("env_gridworld_small.json")
    t = port.Task(open(golden.task_path("gridworld")).read())
    e = port.Env(t, **g["env"])
    b = e.reset(g["rows"])
    for k in range(g["steps"]):
        o = e.step(b)
        assert golden.step_digest(g["rows"], b["states"], o["reward"], o["terminated"], o["truncated"], o["count"],
                                  o["schema"], o["binding"], o["goal"]) == g["digests"][k], k


def test_brfs_determinism_digests(golden):
    """The reference's own determinism fixture (tests/data/determinism.json) for two suite tasks."""
    for name in ["gripper__prob05", "depot__p02"]:
        t = port.Task(open(golden.task_path(name)).read())
        r = port.brfs(t, max_states=20000, stop_at_goal=False)
        d = golden.determinism_digest(r["states"], r["expanded"], r["generated"], r["layers"], r["fingerprint"])
        assert d == golden.DETERMINISM_BRFS[name], name


def test_brfs_golden_budget(golden):
    g = golden.load("brfs.json")["budget"]
    for name in ["depot__p02", "miconic__s7-4"]:
        t = port.Task(open(golden.task_path(name)).read())
        r = port.brfs(t, max_states=20000, stop_at_goal=False)
        exp = g[name]
        for k in ["states", "expanded", "generated", "goal_states", "layers", "fingerprint", "status", "layer_counts"]:
            assert r[k] == exp[k], (name, k)


def test_dedup_workload_unique_count_closed_form():
    """The dedup workload's unique count at its full size (2^26 rows): the generator's fresh rows, counted in chunks."""
    from tests.golden import fixtures as fx

    w = fx.DEDUP_WORKLOAD
    fresh = 0
    for b in range(0, w["rows"], 1 << 22):
        fresh += int(gen.dedup_is_fresh(np.arange(b, b + (1 << 22), dtype=np.uint64), seed=w["seed"], dup=w["dup"]).sum())
    assert fresh == w["unique"]


def test_dedup_stream_against_reference_store():
    """The reference FlatStateStore stores exactly the stream's fresh rows (2^18 rows of the workload's stream)."""
    from oracle import ref

    if not ref.available():
        pytest.skip("reference build missing")
    rows = gen.dedup_rows(0, 1 << 18, 16, seed=0)
    unique, _ = ref.dedup_flat(rows)
    assert unique == int(gen.dedup_is_fresh(np.arange(1 << 18, dtype=np.uint64), seed=0).sum())


def test_dedup_closed_form():
    rows = gen.dedup_rows(0, 4000, 16, seed=5)
    n, ids = port.dedup_unique(rows)
    assert n == int(gen.dedup_is_fresh(np.arange(4000, dtype=np.uint64), seed=5).sum())
    # an exact duplicate maps to the id of its source's first occurrence
    assert all(ids[i] <= i for i in range(len(ids)))


def test_encode_closed_form():
    t = port.Task(workloads.TASKS["transport"]())
    row = t.initial
    idx = port.encode_atoms(row, 200)
    ones = [s for s in range(t.slots) if (int(row[s >> 6]) >> (s & 63)) & 1]
    assert list(idx[: len(ones)]) == ones and (idx[len(ones):] == -1).all()
    m = port.schema_masks(t, row)
    assert list(m) == [1 if any(x[0] == s for x in port.successors(t, row)) else 0 for s in range(len(t.schemas))]


ref = pytest.importorskip("oracle.ref")


@pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (make -C oracle)")
def test_port_against_reference_random_rows():
    rng = np.random.default_rng(99)
    for n in range(0, 40):
        w = rng.integers(0, 2**63, size=n, dtype=np.int64).view(np.uint64)
        if n > 3:
            w[-2:] = 0
        assert port.hash_state(w) == ref.hash_state(w)
        assert port.hash_words(w) == ref.hash_words(w)
    for _ in range(200):
        s, e, d, c = (int(x) for x in rng.integers(1, 2**31, size=4))
        assert port.successor_index(s, e, d, c) == ref.successor_index(s, e, d, c)
    # the whole-batch row hash the env batch fixtures are written with: hash_state row by row, zero tails trimmed
    rows = rng.integers(0, 2**63, size=(64, 9), dtype=np.int64).view(np.uint64)
    rows[5:20, 6:] = 0
    rows[30] = 0
    h = ref.hash_rows(rows)
    assert all(int(h[i]) == port.hash_state(rows[i]) for i in range(len(rows)))
    assert all(int(x) == port.hash_state(rows[i, :7]) for i, x in enumerate(ref.hash_rows(rows, 7)))


def test_expand_noop_filter_closed_form(golden):
    """The switches task (two idle schemas, stop, set; the reference's no-op test domain, tests/python/test_rl_noops.py)
    from its initial state: four successors in schema order, the idle ones no-ops; dropping them keeps stop and set at
    their full-order positions 2 and 3; a state whose successors are all no-ops keeps them all."""
    t = port.Task(open(golden.task_path("noop_switches")).read())
    row = np.zeros(t.words, np.uint64)
    row[0] = 1  # live
    full = port.expand(t, [row])
    assert full["schema"] == [0, 1, 2, 3] and full["noop"] == [True, True, False, False]
    assert full["offsets"] == [0, 4] and full["generated"] == full["total"] == 4
    assert [port.hash_state(r) for r in full["succ"]][:2] == [port.hash_state(row)] * 2
    kept = port.expand(t, [row], drop_noops=True)
    assert kept["schema"] == [2, 3] and kept["index"] == [2, 3] and kept["offsets"] == [0, 2] and kept["total"] == 2
    assert kept["generated"] == 4 and kept["goal"] == [False, True]
    # live and p: only the idle schemas apply, all no-ops, so all are kept
    both = np.array([3], np.uint64)
    k2 = port.expand(t, [both], drop_noops=True)
    assert k2["schema"] == [0, 1] and k2["noop"] == [True, True] and k2["offsets"] == [0, 2]
    # an overflow with drop_noops reports the counts before dropping
    k3 = port.expand(t, [row, row], capacity=5, drop_noops=True)
    assert k3["generated"] == 8 and k3["total"] == 8 and k3["offsets"] == [0, 4, 8]
