"""The checks that pin the oracle (oracle/port.py) catch plausible mistakes: each test plants one mistake at a time
in the oracle on the CPU (a dropped term, a wrong constant, shift or index, a transposed operand, a reversed order)
and asserts that the golden vectors, the reference's fixtures or the closed form that pin that function no longer
pass, after checking that they pass unmutated."""

import numpy as np
import pytest

from mymyr_amd import gen
from oracle import port

M32, M64 = port.M32, port.M64


def passes(check, golden) -> bool:
    try:
        return bool(check(golden))
    except (AssertionError, IndexError, KeyError, ValueError):
        return False


def assert_pins(golden, monkeypatch, check, mutants):
    assert passes(check, golden), "the check fails on the unmutated oracle"
    for name, attr, fn in mutants:
        with monkeypatch.context() as m:
            m.setattr(port, attr, fn)
            assert not passes(check, golden), f"mutant {name} of port.{attr} passes the check"


# ------------------------------------------------------------------------------------------------- hashing
def hash_check(golden):
    g = golden.load("hash.json")
    ok = all(port.hash_words([int(x, 16) for x in c["words"]], int(c["seed"], 16)) == int(c["hash_words"], 16)
             and port.hash_state([int(x, 16) for x in c["words"]]) == int(c["hash_state"], 16) for c in g["cases"])
    return ok and all(port.mix64(int(m["x"], 16)) == int(m["mix64"], 16) for m in g["mix64"])


_mix64, _mulfold, _hash_words = port.mix64, port.mulfold, port.hash_words


def mix64_shift(x):
    x &= M64
    x ^= x >> 31  # 30
    x = (x * 0xBF58476D1CE4E5B9) & M64
    x ^= x >> 27
    x = (x * 0x94D049BB133111EB) & M64
    return x ^ (x >> 31)


def hash_words_no_length(w, seed=port.HASH_SEED):
    return _hash_words(w, seed ^ (len(list(w)) * port.HASH_P1) & M64)  # cancels the n * P1 term


def hash_words_swapped_primes(w, seed=port.HASH_SEED):
    w = [int(x) for x in w]
    h = (seed ^ (len(w) * port.HASH_P1)) & M64
    i = 0
    while i + 1 < len(w):
        h = _mulfold(h ^ w[i] ^ port.HASH_P2, w[i + 1] ^ port.HASH_P1)
        i += 2
    if i < len(w):
        h = _mulfold(h ^ w[i] ^ port.HASH_P1, port.HASH_P2)
    return _mix64(h)


def test_hash_pins(golden, monkeypatch):
    assert_pins(golden, monkeypatch, hash_check, [
        ("low half of the product only", "mulfold", lambda a, b: ((a & M64) * (b & M64)) & M64),
        ("first shift 31", "mix64", mix64_shift),
        ("no length term", "hash_words", hash_words_no_length),
        ("primes swapped", "hash_words", hash_words_swapped_primes),
        ("untrimmed words", "hash_state", lambda w: _hash_words(list(w))),
    ])


# ------------------------------------------------------------------------------------------------- Philox and draws
def philox_check(golden):
    g = golden.load("philox.json")
    ok = all(port.philox4x32_10(k["ctr"], *k["key"]) == k["out"] for k in g["kats"])
    ok = ok and all(port.philox_block(d["seed"], d["env"], d["draw"], 0) == d["block"]
                    and port.successor_index(d["seed"], d["env"], d["draw"], d["count"]) == d["index"] for d in g["draws"])
    # below's closed form (the high word of the 128-bit product), as tests/test_oracle.py pins it
    rng = np.random.default_rng(17)
    xs = [int(x) for x in rng.integers(0, 2**63, size=500, dtype=np.int64)]
    ns = [int(n) for n in rng.integers(1, 2**32, size=500, dtype=np.int64)]
    return ok and all(port.below(x, n) == (x * n) >> 64 for x, n in zip(xs, ns))


def philox_rounds(rounds, k0_step=0x9E3779B9, k1_step=0xBB67AE85):
    def f(c, k0, k1):
        c = [x & M32 for x in c]
        k0 &= M32
        k1 &= M32
        for _ in range(rounds):
            p0 = 0xD2511F53 * c[0]
            p1 = 0xCD9E8D57 * c[2]
            c = [((p1 >> 32) ^ c[1] ^ k0) & M32, p1 & M32, ((p0 >> 32) ^ c[3] ^ k1) & M32, p0 & M32]
            k0 = (k0 + k0_step) & M32
            k1 = (k1 + k1_step) & M32
        return c
    return f


_philox, _below = port.philox4x32_10, port.below


def test_philox_and_draw_pins(golden, monkeypatch):
    assert_pins(golden, monkeypatch, philox_check, [
        ("nine rounds", "philox4x32_10", philox_rounds(9)),
        ("key steps swapped", "philox4x32_10", philox_rounds(10, 0xBB67AE85, 0x9E3779B9)),
        ("env and purpose words swapped", "philox_block",
         lambda seed, env, draw, purpose: _philox([draw & M32, (draw >> 32) & M32, purpose, env & M32], seed & M32, (seed >> 32) & M32)),
        ("seed halves swapped", "philox_block",
         lambda seed, env, draw, purpose: _philox([draw & M32, (draw >> 32) & M32, env & M32, purpose], (seed >> 32) & M32, seed & M32)),
        ("low product bits", "below", lambda x, n: ((x & M32) * n) >> 32),
        ("high word alone", "below", lambda x, n: ((x >> 32) * n) >> 32),
    ])


# ------------------------------------------------------------------------------------------------- env step
def env_check(golden):
    g = golden.load("env_gridworld_small.json")
    t = port.Task(open(golden.task_path("gridworld")).read())
    e = port.Env(t, **g["env"])
    b = e.reset(g["rows"])
    for k in range(g["steps"]):
        o = e.step(b)
        if golden.step_digest(g["rows"], b["states"], o["reward"], o["terminated"], o["truncated"], o["count"], o["schema"],
                              o["binding"], o["goal"]) != g["digests"][k]:
            return False
    return True


_successors, _successor_index, _is_goal = port.successors, port.successor_index, port.is_goal


def test_env_step_pins(golden, monkeypatch):
    assert_pins(golden, monkeypatch, env_check, [
        ("successors in reverse order", "successors", lambda task, row, witness=False: _successors(task, row, witness)[::-1]),
        ("draw counter off by one", "successor_index", lambda seed, env, draw, count: _successor_index(seed, env, draw + 1, count)),
        ("env ids off by one", "successor_index", lambda seed, env, draw, count: _successor_index(seed, env + 1, draw, count)),
        ("goal test negated", "is_goal", lambda task, row: not _is_goal(task, row)),
    ])


# ------------------------------------------------------------------------------------------------- BrFS
def brfs_check(golden):
    """The reference's searches of gripper to depth 2 and to a 50-state cut (brfs_edges.json): counts and fingerprints."""
    t = port.Task(open(golden.task_path("gripper__prob05")).read())
    edges = golden.load("brfs_edges.json")
    for key in ("gripper__prob05:auto:depth2", "gripper__prob05:auto:states50"):
        exp = edges[key]
        opts = {k: v for k, v in exp["options"].items() if k in ("max_depth", "max_states", "stop_at_goal")}
        r = port.brfs(t, **opts)
        if any(r[k] != exp[k] for k in ("states", "expanded", "generated", "layers", "fingerprint", "layer_counts")):
            return False
    return True


_canonical_hash, _mix = port.canonical_hash, port.mix64


def canonical_hash_offset(task, row):
    x = 0
    for wi, w in enumerate(row):
        w = int(w)
        while w:
            b = (w & -w).bit_length() - 1
            w &= w - 1
            x ^= _mix(task.slot_cid[wi * 64 + b] + 0x1234568)  # 0x1234567
    return x


def canonical_hash_sum(task, row):
    x = 0
    for wi, w in enumerate(row):
        w = int(w)
        while w:
            b = (w & -w).bit_length() - 1
            w &= w - 1
            x = (x + _mix(task.slot_cid[wi * 64 + b] + 0x1234567)) & M64  # x ^= ...
    return x


def test_brfs_pins(golden, monkeypatch):
    assert_pins(golden, monkeypatch, brfs_check, [
        ("canonical hash offset", "canonical_hash", canonical_hash_offset),
        ("sum for xor", "canonical_hash", canonical_hash_sum),
        ("successors in reverse order", "successors", lambda task, row, witness=False: _successors(task, row, witness)[::-1]),
    ])


# ------------------------------------------------------------------------------------------------- dedup and encoding
def dedup_check(golden):
    rows = gen.dedup_rows(0, 4000, 16, seed=5)
    n, ids = port.dedup_unique(rows)
    src = gen.dedup_sources(0, 4000, seed=5)
    fresh = src == np.arange(4000, dtype=np.uint64)
    return n == int(fresh.sum()) and np.array_equal(ids, (np.cumsum(fresh) - 1)[src.astype(np.int64)])


def dedup_row_index_ids(rows):
    seen = {}
    ids = np.zeros(rows.shape[0], np.int64)
    for i in range(rows.shape[0]):
        ids[i] = seen.setdefault(rows[i].tobytes(), i)  # the row index, not the rank
    return len(seen), ids


def dedup_last_occurrence(rows):
    n, ids = _dedup(rows)
    last = {}
    for i in range(len(ids)):
        last[ids[i]] = i
    order = {k: r for r, k in enumerate(sorted(last, key=lambda k: last[k]))}
    return n, np.array([order[x] for x in ids], np.int64)


_dedup, _encode = port.dedup_unique, port.encode_atoms


def encode_check(golden):
    from mymyr_amd import workloads

    t = port.Task(workloads.TASKS["transport"]())
    row = t.initial
    idx = port.encode_atoms(row, 200)
    bits = np.unpackbits(np.asarray(row, np.uint64).view(np.uint8), bitorder="little")
    ones = np.flatnonzero(bits)
    return list(idx[: len(ones)]) == list(ones) and bool((idx[len(ones):] == -1).all())


def test_dedup_and_encoding_pins(golden, monkeypatch):
    assert_pins(golden, monkeypatch, dedup_check, [
        ("row indices for ids", "dedup_unique", dedup_row_index_ids),
        ("ids by last occurrence", "dedup_unique", dedup_last_occurrence),
    ])
    assert_pins(golden, monkeypatch, encode_check, [
        ("descending slots", "encode_atoms", lambda row, k: np.concatenate([np.sort(_encode(row, k)[_encode(row, k) >= 0])[::-1],
                                                                            _encode(row, k)[_encode(row, k) < 0]]).astype(np.int32)),
        ("zero padding", "encode_atoms", lambda row, k: np.where(_encode(row, k) < 0, 0, _encode(row, k)).astype(np.int32)),
    ])


# ------------------------------------------------------------------------------------------------- task tables
def table_check(*cases):
    def check(golden):
        from tests.test_table_oracle import replay_oracle

        for d in golden.load("env_table.json")["instance_draws"]:
            thr, idx = golden.sampler_arrays(d["weights"])
            if port.instance_draw(d["seed"], d["env"], d["reset_count"], d["instances"], thr, idx) != d["draw"]:
                return False
        for d in golden.load("instance_draw_edges.json"):
            if port.instance_draw(d["seed"], d["env"], d["reset_count"], d["instances"], d["thresholds"], d["indices"]) != d["draw"]:
                return False
        for case in cases:
            replay_oracle(golden, case)
        return True
    return check


_instance_draw, _fmix32, _visited_insert, _mask_goal, _pad = (port.instance_draw, port.fmix32, port.visited_insert,
                                                              port.mask_goal, port.pad)


def fmix32_constant(x):
    x &= M32
    x = ((x ^ (x >> 16)) * 0x85EBCA6C) & M32  # 0x85EBCA6B
    x = ((x ^ (x >> 13)) * 0xC2B2AE35) & M32
    return x ^ (x >> 16)


def instance_draw_strict(seed, env, reset_count, instances, thresholds=(), indices=()):
    # thresholds compared with < where the draw counts those at most its bits
    if len(indices) == 0:
        return _instance_draw(seed, env, reset_count, instances)
    value = _fmix32((seed & M32) ^ _fmix32(((seed >> 32) & M32) ^ 0x53414D50))
    bits = _fmix32(value ^ _fmix32(env & M32) ^ _fmix32((reset_count & M32) ^ 0x9E3779B9))
    return int(indices[sum(1 for t in thresholds if int(t) < bits)])


def visited_insert_late_overflow(table, count, h):
    H = len(table)
    key = h if h else port.VISITED_ZERO
    at = key & (H - 1)
    for _ in range(H):
        if int(table[at]) == key:
            return True, count
        if int(table[at]) == 0:
            if count >= (H * 3) // 4 + 1:  # (H * 3) // 4
                return False, H
            table[at] = np.uint64(key)
            return False, count + 1
        at = (at + 1) & (H - 1)
    return False, H


def test_task_table_pins(golden, monkeypatch):
    assert_pins(golden, monkeypatch, table_check("gridworld_sampled", "transport_weighted"), [
        ("fmix32 constant", "fmix32", fmix32_constant),
        ("thresholds compared strictly", "instance_draw", instance_draw_strict),
        ("env and reset count swapped", "instance_draw",
         lambda seed, env, rc, n, thr=(), idx=(): _instance_draw(seed, rc, env, n, thr, idx)),
    ])
    assert_pins(golden, monkeypatch, table_check("gridworld_visited"), [
        ("overflow one entry late", "visited_insert", visited_insert_late_overflow),
    ])
    assert_pins(golden, monkeypatch, table_check("gridworld_goals"), [
        ("goal masks transposed", "mask_goal", lambda row, gp, gn: _mask_goal(row, gn, gp)),
    ])
    assert_pins(golden, monkeypatch, table_check("gridworld_ids"), [
        ("one slot fewer", "pad", lambda flat, rows, k, *a, **kw: _pad(flat, rows, max(0, k - 1), *a, **kw)),
    ])


@pytest.mark.parametrize("attr", ["mix64", "mulfold", "hash_words", "hash_state", "philox4x32_10", "philox_block", "below",
                                  "successor_index", "successors", "is_goal", "canonical_hash", "dedup_unique",
                                  "encode_atoms", "fmix32", "instance_draw", "visited_insert", "mask_goal", "pad"])
def test_every_pinned_function_has_a_mutant(attr):
    """Each function named here is mutated by at least one of the tests above."""
    import inspect
    import sys

    src = inspect.getsource(sys.modules[__name__])
    assert f'"{attr}"' in src.split("def test_every_pinned_function_has_a_mutant")[0]
