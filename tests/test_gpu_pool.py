"""The pool's asynchronous API on the device (rl.EnvPool and DeviceEnvPool: send / recv / recv_ticket / reset(env_ids) /
recycle, the reference's CpuEnvPool, include/mymyr/rl/pool.hpp:114-172) against the compiled reference pool: over each case's
scripted calls (subsets of shuffled env ids, given actions with invalid ones, the random policy, several sends received
together and by ticket, resets of some envs) every returned batch is digest-equal to the reference's."""

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


class Calls:
    """The reference pool's call shapes over an EnvPool."""

    def __init__(self, pool):
        self.pool = pool

    def reset(self, ids):
        return self.pool.reset(ids)

    def send(self, ids, actions):
        return self.pool.send(ids, None if actions is None else torch.from_numpy(actions))

    def recv(self, min_rows):
        return self.pool.recv(min_rows)

    def recv_ticket(self, t):
        return self.pool.recv_ticket(t)


def make_pool(golden, case, cls="EnvPool"):
    from mymyr_amd import rl
    from mymyr_amd.task import Task

    c = golden.POOL_CASES[case]
    t = Task.from_text_file(golden.task_path(case))
    return getattr(rl, cls)(t, c["num_envs"], first_env=c["first_env"], **c["env"]), t


@pytest.mark.parametrize("case", ["gridworld", "transport"])
def test_pool_calls_match_reference(golden, case):
    g = golden.load("pool.json")[case]
    pool, t = make_pool(golden, case)
    print(f"pool calls: {case}", flush=True)
    digests = golden.run_pool_script(Calls(pool), case, g["label_width"])
    assert len(digests) == len(g["digests"])
    for k, (a, b) in enumerate(zip(digests, g["digests"])):
        assert a == b, f"{case}: batch {k} differs from the reference pool's"
    assert pool.pending == 0
    pool.check()


def test_pool_send_errors_and_recycle(golden):
    pool, t = make_pool(golden, "gridworld")
    pool.reset()
    with pytest.raises(ValueError, match="repeated"):
        pool.send([1, 2, 1])
    with pytest.raises(ValueError, match="out of range"):
        pool.send([pool.num_envs])
    t1 = pool.send([3, 4, 5])
    with pytest.raises(ValueError, match="in flight"):
        pool.send([5, 6])
    with pytest.raises(ValueError, match="in flight"):
        pool.step()
    with pytest.raises(ValueError, match="ticket"):
        pool.recv_ticket(t1 + 7)
    b = pool.recv_ticket(t1)
    assert b.rows == 3 and b.step and b.env_ids.tolist() == [3, 4, 5]
    with pytest.raises(ValueError, match="pending"):
        pool.recv()
    # a recycled batch's arrays are filled by the next send of as many rows
    reward = b.reward
    pool.recycle(b)
    b2 = pool.step([7, 8, 9])
    assert b2.reward.data_ptr() == reward.data_ptr() and b2.env_ids.tolist() == [7, 8, 9]
    # a send of every env equals an in-place step of a twin pool
    twin, _ = make_pool(golden, "gridworld", "DeviceEnvPool")
    twin.reset()
    twin.step(env_ids=[3, 4, 5])
    twin.step(env_ids=[7, 8, 9])
    a = pool.recv_ticket(pool.send())
    w = twin.step()
    for k in ("states", "reward", "terminated", "truncated", "count", "schema", "goal"):
        assert torch.equal(a[k], w[k]), k


def test_env_pool_samples_instances_like_the_reference_default(golden):
    """EnvPool over a table with the default sampler ("auto": uniform) places every env in a sampled instance and a reset
    without task ids draws the next one, the draw of (seed, env id, reset counter) of the reference pool
    (rl::rng::instance_draw); with sampler=None every env stays in instance 0."""
    from mymyr_amd import rl
    from mymyr_amd.task import Task
    from mymyr_amd import workloads
    from oracle import port

    paths = workloads.table_files("gridworld_table", golden.TASKS)
    ts = [Task.from_text_file(p) for p in paths]
    pool = rl.EnvPool(ts, 64, seed=5, first_env=2)
    b = pool.reset()
    ids = b.task_ids.cpu().numpy()
    exp = [port.instance_draw(5, 2 + e, 1, len(ts)) for e in range(64)]
    assert ids.tolist() == exp and len(set(exp)) > 1
    assert pool.reset_counts.cpu().numpy().tolist() == [2] * 64
    still = rl.EnvPool(ts, 64, seed=5, first_env=2, sampler=None)
    assert still.reset().task_ids.cpu().numpy().tolist() == [0] * 64
    # the reference pool's read-only properties (python/src/rl_bindings.cpp:2465-2600)
    assert (pool.num_envs, pool.first_env, pool.seed, pool.threads, pool.goals, pool.dead_end) == (64, 2, 5, 1, False, "no_successors")
    assert (pool.framework, pool.numeric_words, pool.max_steps, pool.pending) == (None, 0, None, 0)
