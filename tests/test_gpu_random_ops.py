"""The random-access microbenchmark entry point (mya_random_ops) against closed forms of its seeded operations: op i
acts on word mix64(seed + i * golden gamma) & (words - 1) of the table; folded over all threads, the loads' and the
atomics' old values and the atomics' final table do not depend on the order the operations run in."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GAMMA = 0x9E3779B97F4A7C15
THREADS = 1 << 20  # MYA_RANDOM_OPS_THREADS


def mix64_np(x: np.ndarray) -> np.ndarray:
    """The splitmix64 finalizer over a uint64 array (wrapping products)."""
    x = x.copy()
    x ^= x >> np.uint64(30)
    x *= np.uint64(0xBF58476D1CE4E5B9)
    x ^= x >> np.uint64(27)
    x *= np.uint64(0x94D049BB133111EB)
    x ^= x >> np.uint64(31)
    return x


def addresses(seed: int, n: int, words: int) -> np.ndarray:
    with np.errstate(over="ignore"):
        i = np.arange(n, dtype=np.uint64)
        return mix64_np(np.uint64(seed) + i * np.uint64(GAMMA)) & np.uint64(words - 1)


def run(kind: int, table: "torch.Tensor", n: int, seed: int) -> np.ndarray:
    from mymyr_amd._lib import check, lib

    sink = torch.full((THREADS,), 0x5A5A, dtype=torch.int64, device="cuda")
    check(lib.mya_random_ops(table.data_ptr(), table.numel(), n, kind, seed, sink.data_ptr(),
                             torch.cuda.current_stream().cuda_stream))
    torch.cuda.synchronize()
    return sink.cpu().numpy().view(np.uint64)


def xor_all(a: np.ndarray) -> int:
    return int(np.bitwise_xor.reduce(a, initial=np.uint64(0)))


def test_addresses_follow_the_oracle_mix64():
    from oracle import port

    a = addresses(77, 1000, 1 << 16)
    for i in (0, 1, 2, 3, 499, 999):
        assert int(a[i]) == port.mix64((77 + i * GAMMA) & ((1 << 64) - 1)) & 0xFFFF


@pytest.mark.parametrize("n", [0, 3, 50001])
def test_loads_fold_to_the_table_words(n):
    words, seed = 1 << 16, 11
    vals = mix64_np(np.arange(words, dtype=np.uint64) + np.uint64(7))
    table = torch.from_numpy(vals.view(np.int64)).cuda()
    sink = run(0, table, n, seed)
    assert xor_all(sink) == xor_all(vals[addresses(seed, n, words)])
    assert np.array_equal(table.cpu().numpy().view(np.uint64), vals)


def test_cas_table_and_old_values():
    words, seed, n = 1 << 16, 12, 50001
    table = torch.zeros(words, dtype=torch.int64, device="cuda")
    sink = run(1, table, n, seed)
    a = addresses(seed, n, words)
    hits = np.bincount(a.astype(np.int64), minlength=words)
    idx = np.arange(words, dtype=np.uint64)
    want = np.where(hits > 0, idx | np.uint64(1), np.uint64(0))
    assert np.array_equal(table.cpu().numpy().view(np.uint64), want)
    # per word hit k times: the first CAS reads 0, the k - 1 others read the stored value
    odd = (hits > 0) & ((hits - 1) % 2 == 1)
    assert xor_all(sink) == xor_all((idx | np.uint64(1))[odd])


def test_atomic_min_table_and_old_values():
    words, seed, n = 1 << 16, 13, 50001
    table = torch.full((words,), -1, dtype=torch.int64, device="cuda")
    sink = run(2, table, n, seed)
    a = addresses(seed, n, words)
    hits = np.bincount(a.astype(np.int64), minlength=words)
    idx = np.arange(words, dtype=np.uint64)
    ones = np.uint64(0xFFFFFFFFFFFFFFFF)
    want = np.where(hits > 0, ~idx, ones)
    assert np.array_equal(table.cpu().numpy().view(np.uint64), want)
    # per word hit k times: the first reads all ones, the k - 1 others read ~word
    first = xor_all(np.full(int((hits > 0).sum()), ones, dtype=np.uint64))
    odd = (hits > 0) & ((hits - 1) % 2 == 1)
    assert xor_all(sink) == first ^ xor_all((~idx)[odd])


def test_stores_hold_an_operation_of_their_word():
    words, seed, n = 1 << 16, 14, 50001
    table = torch.zeros(words, dtype=torch.int64, device="cuda")
    sink = run(3, table, n, seed)
    assert np.all(sink == 0x5A5A)  # stores leave the sink alone
    a = addresses(seed, n, words)
    got = table.cpu().numpy().view(np.uint64)
    hits = np.bincount(a.astype(np.int64), minlength=words)
    assert np.all(got[hits == 0] == 0)
    nz = np.nonzero(got)[0]
    assert np.all(got[nz] < n)
    assert np.array_equal(a[got[nz].astype(np.int64)], nz.astype(np.uint64))
    # every hit word holds one of its operations (operation 0 stores 0)
    assert len(nz) >= int((hits > 0).sum()) - 1


def test_rejects_bad_arguments():
    from mymyr_amd._lib import lib

    table = torch.zeros(100, dtype=torch.int64, device="cuda")
    sink = torch.zeros(THREADS, dtype=torch.int64, device="cuda")
    s = torch.cuda.current_stream().cuda_stream
    assert lib.mya_random_ops(table.data_ptr(), 100, 10, 0, 1, sink.data_ptr(), s) != 0  # not a power of two
    assert lib.mya_random_ops(table.data_ptr(), 64, 10, 4, 1, sink.data_ptr(), s) != 0  # no such kind
    assert lib.mya_random_ops(None, 64, 10, 0, 1, sink.data_ptr(), s) != 0
