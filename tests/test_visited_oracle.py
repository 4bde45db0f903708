"""The oracle's visited tables (rl/visited.hpp) against the compiled reference's: tables filled by visited_insert and
rl::visited_mask over queries with padding and a row mapping (tests/golden/visited_mask.json), and membership against
what linear probing must give for tables below their load limit."""

import numpy as np

from oracle import port


def _u64(xs):
    return np.array([int(x) for x in xs], np.uint64)


def test_visited_tables_and_mask_match_reference(golden):
    g = golden.load("visited_mask.json")
    H = g["H"]
    table = np.zeros((len(g["inserts"]), H), np.uint64)
    count = np.zeros(len(g["inserts"]), np.int32)
    for r, hs in enumerate(g["inserts"]):
        present = []
        for h in hs:
            p, count[r] = port.visited_insert(table[r], int(count[r]), int(h))
            present.append(int(p))
        assert present == g["present"][r], f"row {r}: present flags"
    assert (table == np.array([_u64(t) for t in g["table"]])).all()
    assert count.tolist() == g["count"]
    hashes = _u64(g["hashes"])
    assert port.visited_mask(table, count, hashes, g["parent"]).tolist() == g["mask"]
    rows = np.array(g["rows"], np.int32)
    assert port.visited_mask(table, count, hashes, g["parent_mapped"], rows).tolist() == g["mask_mapped"]


def test_visited_contains_is_set_membership():
    """Below the 3H/4 limit every inserted key is stored, so membership is plain set membership (hash 0 standing for
    its reserved key); an emptied count hides every key."""
    rng = np.random.default_rng(3)
    H = 32
    for trial in range(20):
        table = np.zeros(H, np.uint64)
        n = int(rng.integers(0, 24))
        keys = [int(x) for x in rng.integers(0, 4 * H, n)]  # small keys: long probe chains
        count = 0
        for k in keys:
            _, count = port.visited_insert(table, count, k)
        stored = {k if k else port.VISITED_ZERO for k in keys}
        assert count == len(stored)
        for q in list(range(4 * H)) + [port.VISITED_ZERO]:
            want = (q if q else port.VISITED_ZERO) in stored
            assert port.visited_contains(table, count, q) == want, (trial, q)
        if keys:
            assert not port.visited_contains(table, 0, keys[0])
