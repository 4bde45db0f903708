"""Device hashing and the device state set against the golden hash vectors, the oracle and closed forms."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def dev(a: np.ndarray) -> "torch.Tensor":
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int64)).cuda()


def host(t) -> np.ndarray:
    return t.cpu().numpy().view(np.uint64)


def test_hash_rows_golden(golden):
    from mymyr_amd import hip

    g = golden.load("hash.json")
    by_len = {}
    for c in g["cases"]:
        by_len.setdefault(len(c["words"]), []).append(c)
    for n, cases in by_len.items():
        if n == 0:
            continue
        rows = np.array([[int(x, 16) for x in c["words"]] for c in cases], dtype=np.uint64)
        h = host(hip.hash_rows(dev(rows)))
        assert [f"{int(x):016x}" for x in h] == [c["hash_state"] for c in cases], n


def test_hash_rows_random_vs_oracle():
    from mymyr_amd import hip
    from oracle import port

    rng = np.random.default_rng(1)
    for words in (1, 3, 8, 13, 16, 176, 2049, 3000):
        rows = rng.integers(0, 2**63, size=(257, words), dtype=np.int64).view(np.uint64)
        rows[::4, words // 2:] = 0
        rows[7] = 0
        h = host(hip.hash_rows(dev(rows)))
        assert all(int(h[i]) == port.hash_state(rows[i]) for i in range(0, 257, 16))


def test_dedup_stream_matches_generator():
    from mymyr_amd import gen, hip

    d = host(hip.dedup_rows(1000, 3000, 16, seed=9))
    assert np.array_equal(d, gen.dedup_rows(1000, 3000, 16, seed=9))


def test_state_set_ids_and_unique_count():
    from mymyr_amd import gen, hip
    from oracle import port

    rows = gen.dedup_rows(0, 20000, 16, seed=4)
    s = hip.StateSet(40000, 16, 0.5, batch=4096)  # several batches
    n, ids, is_new = s.insert(dev(rows))
    exp_n, exp_ids = port.dedup_unique(rows)
    assert n == exp_n == len(s)
    assert np.array_equal(ids.cpu().numpy(), exp_ids)
    first = np.zeros(len(rows), np.uint8)
    first[np.unique(exp_ids, return_index=True)[1]] = 1
    assert np.array_equal(is_new.cpu().numpy(), first)
    # a second insert of the same rows adds nothing and returns the same ids
    n2, ids2, _ = s.insert(dev(rows))
    assert n2 == 0 and np.array_equal(ids2.cpu().numpy(), exp_ids)


def test_state_set_ids_across_epoch_settling():
    """Batches of 128 rows use up the state set's 64 epochs several times: the passes that settle candidate-coded
    entries to ids keep every id and the unique count equal to the oracle's, and rows inserted again later find them."""
    from mymyr_amd import gen, hip
    from oracle import port

    rows = gen.dedup_rows(0, 30000, 8, seed=6)
    s = hip.StateSet(30000, 8, 0.5, batch=128)  # 235 batches: 3 settling passes
    n, ids, _ = s.insert(dev(rows))
    exp_n, exp_ids = port.dedup_unique(rows)
    assert n == exp_n == len(s)
    assert np.array_equal(ids.cpu().numpy(), exp_ids)
    # rows from the start and the end of the stream again, in one more batch sequence
    again = np.concatenate([rows[:5000], rows[-5000:]])
    n2, ids2, is_new2 = s.insert(dev(again))
    assert n2 == 0 and not is_new2.any()
    assert np.array_equal(ids2.cpu().numpy(), np.concatenate([exp_ids[:5000], exp_ids[-5000:]]))
    # the stored rows are the first occurrences in id order
    stored = torch.from_dlpack(s.rows()).cpu().numpy().view(np.uint64)
    assert np.array_equal(stored, rows[np.unique(exp_ids, return_index=True)[1]])


def test_state_set_dedup_closed_form_large():
    """2^22 rows of 1024 bits in 2^20-row batches at load 0.5: the unique count is the generator's fresh-row count."""
    from mymyr_amd import gen, hip

    total, batch = 1 << 22, 1 << 20
    s = hip.StateSet(total, 16, 0.5, batch=batch)
    new = 0
    for b in range(0, total, batch):
        n, _, _ = s.insert(hip.dedup_rows(b, batch, 16, seed=0), want_ids=False)
        new += n
    fresh = int(gen.dedup_is_fresh(np.arange(total, dtype=np.uint64), seed=0).sum())
    assert new == fresh == len(s)


def test_state_set_dedup_workload_full_size():
    """The dedup workload at its stated size: 2^26 rows of 1024 bits, about 30% duplicates, in 2^20-row batches into a
    table at load 0.5 (a 1 GiB table and an 8.6 GB arena, so row and slot offsets pass 2^32 bytes). The unique count is
    exact (the stream's fresh rows), and so is every row's id: the stream makes each duplicate a copy of an earlier
    fresh row, so a row's id is that fresh row's rank among the fresh rows (ids are first-occurrence ranks). Inserting
    a batch again adds nothing and finds the ids of its first insert."""
    from mymyr_amd import gen, hip
    from tests.golden import fixtures as fx

    w = fx.DEDUP_WORKLOAD
    total, batch = w["rows"], w["batch"]
    print(f"dedup workload: {total} rows in batches of {batch}", flush=True)
    src = gen.dedup_sources(0, total, seed=w["seed"], dup=w["dup"])
    fresh = src == np.arange(total, dtype=np.uint64)
    exp_ids = (np.cumsum(fresh, dtype=np.int64) - 1)[src.astype(np.int64)]
    del fresh
    s = hip.StateSet(total, w["words"], 0.5, batch=batch)
    new = 0
    again = {}
    for b in range(0, total, batch):
        n, ids, _ = s.insert(hip.dedup_rows(b, batch, w["words"], seed=w["seed"], dup=w["dup"]))
        got = ids.cpu().numpy()
        assert np.array_equal(got, exp_ids[b:b + batch]), b
        if b in (0, total // 2, total - batch):
            again[b] = got
        new += n
    assert new == w["unique"] == len(s)
    for b, ids in again.items():
        n2, ids2, is_new2 = s.insert(hip.dedup_rows(b, batch, w["words"], seed=w["seed"], dup=w["dup"]))
        assert n2 == 0 and not bool(is_new2.any())
        assert np.array_equal(ids2.cpu().numpy(), ids)
        assert ids.min() >= 0 and ids.max() < w["unique"]


def test_state_set_errors():
    from mymyr_amd import hip
    from mymyr_amd._lib import MyaError

    s = hip.StateSet(10, 4, 0.5, batch=16)
    with pytest.raises(ValueError):
        s.insert(torch.zeros((3, 5), dtype=torch.int64, device="cuda"))
    with pytest.raises(MyaError, match="state set full"):
        s.insert(torch.arange(64, dtype=torch.int64, device="cuda").view(16, 4))
    with pytest.raises(MyaError, match="load"):
        hip.StateSet(10, 4, 1.5)


@pytest.mark.parametrize("words", [2049, 3000])
def test_state_set_rows_beyond_2048_words(words):
    """Rows wider than 2048 words stay in memory (a 64-lane group compares, hashes and copies them): ids, unique count and
    stored rows equal the oracle's first occurrences over several batches, and rows that differ only in their last
    or a middle word stay apart."""
    from mymyr_amd import gen, hip
    from oracle import port

    rows = gen.dedup_rows(0, 3000, words, seed=8)
    a = rows[0].copy()
    b = a.copy()
    b[-1] ^= 1
    c = a.copy()
    c[words // 2] ^= 1 << 63
    rows = np.concatenate([rows, np.stack([a, b, a, c, b])])
    s = hip.StateSet(4000, words, 0.5, batch=700)
    n, ids, _ = s.insert(dev(rows))
    exp_n, exp_ids = port.dedup_unique(rows)
    assert n == exp_n == len(s)
    assert np.array_equal(ids.cpu().numpy(), exp_ids)
    got = ids.cpu().numpy()[-5:]
    assert got[0] == got[2] and got[1] == got[4] and len({got[0], got[1], got[3]}) == 3
    stored = torch.from_dlpack(s.rows()).cpu().numpy().view(np.uint64)
    assert np.array_equal(stored, rows[np.unique(exp_ids, return_index=True)[1]])


def test_state_set_ids_at_4m_rows():
    """Ids at 2^22 rows of 1,024 bits in 2^20-row batches (four batches, 7% of the 2^26-row workload), against the ids
    numpy derives from the rows themselves: each distinct row's id is the rank of its first occurrence."""
    from mymyr_amd import gen, hip

    total, batch = 1 << 22, 1 << 20
    rows = gen.dedup_rows(0, total, 16, seed=12)
    _, first, inverse = np.unique(np.ascontiguousarray(rows).view(np.dtype((np.void, 128))).reshape(-1), return_index=True,
                                  return_inverse=True)
    rank = np.empty(len(first), np.int64)
    rank[np.argsort(first, kind="stable")] = np.arange(len(first))
    exp = rank[inverse.reshape(-1)]
    s = hip.StateSet(total, 16, 0.5, batch=batch)
    got = np.empty(total, np.int64)
    for b in range(0, total, batch):
        _, ids, _ = s.insert(dev(rows[b:b + batch]))
        got[b:b + batch] = ids.cpu().numpy()
    assert len(s) == len(first)
    assert np.array_equal(got, exp)
