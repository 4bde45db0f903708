"""Label-mode steps of the compiled reference (HostEnv::step with Labels, src/mymyr/rl/env.cpp:376-426) against its
index-mode steps: a label step equals the index step at the label's position in the row's canonical successor order
(rl::expand's order, no witness pruning), an inapplicable or out-of-range label equals an invalid index, and the
reported counts are clamped to 0/1 (ActionSpace::Label, include/mymyr/rl/env.hpp:69-74). The device label step is
built on this equivalence."""

import numpy as np
import pytest

from oracle import ref

pytestmark = pytest.mark.skipif(not ref.available(), reason="oracle/_ref not built (make -C oracle)")


def _outputs(rows, L, W):
    return {"reward": np.zeros(rows, np.float32), "terminated": np.zeros(rows, np.uint8), "truncated": np.zeros(rows, np.uint8),
            "count": np.zeros(rows, np.int32), "schema": np.zeros(rows, np.int32), "binding": np.zeros((rows, L), np.int32),
            "goal": np.zeros(rows, np.uint8), "invalid": np.zeros(rows, np.uint8), "final_states": np.zeros((rows, W), np.uint64)}


@pytest.mark.parametrize("table", ["gridworld_table", "transport_table"])
def test_label_step_is_the_index_step_at_the_label(golden, table):
    from mymyr_amd import workloads

    ts = [ref.RefTask(p) for p in workloads.table_files(table, golden.TASKS)]
    I, rows = len(ts), 48
    W = max(t.words for t in ts)
    L = max(1, max(t.label_width for t in ts))
    kw = dict(seed=7, max_steps=9)
    envs = {m: ref.RefTableEnv(ts, labels=(m == "label"), **kw) for m in ("index", "label")}
    rng = np.random.default_rng(11)
    ids = (np.arange(rows) % I).astype(np.int32)
    moved = invalid = 0
    batches = {}
    for m, e in envs.items():
        b = {"states": np.zeros((rows, W), np.uint64), "steps": np.zeros(rows, np.int32), "draws": np.zeros(rows, np.uint64),
             "at_goal": np.zeros(rows, np.uint8), "task_ids": ids.copy()}
        cnt = np.zeros(rows, np.int32)
        e.reset(b, cnt)
        batches[m] = (b, cnt)
    for k in range(12):
        bi, ci = batches["index"]
        bl, _ = batches["label"]
        assert all(np.array_equal(bi[n], bl[n]) for n in bi), f"step {k}: batches differ"
        x = ref.table_expand(ts, bi["states"], bi["task_ids"])
        off = np.asarray(x["offsets"], np.int64)
        c = off[1:] - off[:-1]
        idx = np.where(c > 0, (rng.random(rows) * np.maximum(c, 1)).astype(np.int64), 0)
        lab_s = np.full(rows, -1, np.int32)
        lab_b = rng.integers(-1, 6, (rows, L)).astype(np.int32)
        for i in range(rows):
            if c[i]:
                lab_s[i] = x["schema"][off[i] + idx[i]]
                lab_b[i] = np.where(x["binding"][off[i] + idx[i]] >= 0, x["binding"][off[i] + idx[i]], lab_b[i])
        garbage = rng.random(rows) < 0.3
        lab_s[garbage] = rng.integers(-1, 8, int(garbage.sum()))
        # the index of each label in the row's canonical order (-1: not among the successors)
        act = np.full(rows, -1, np.int64)
        for i in range(rows):
            for j in range(off[i], off[i + 1]):
                bj = x["binding"][j]
                if x["schema"][j] == lab_s[i] and np.all((bj < 0) | (bj == lab_b[i])):
                    act[i] = j - off[i]
                    break
        oi, ol = _outputs(rows, L, W), _outputs(rows, L, W)
        envs["index"].step(bi, actions=act, **oi)
        envs["label"].step(bl, labels=(lab_s, lab_b), **ol)
        oi["count"] = np.minimum(oi["count"], 1)
        for n in oi:
            assert np.array_equal(oi[n], ol[n]), f"{table} step {k}: {n}"
        moved += int((ol["schema"] >= 0).sum())
        invalid += int(ol["invalid"].sum())
    assert moved > 0 and invalid > 0, (moved, invalid)
