"""mya_expand_noalloc (the flat expansion whose scratch is a static device array) against mya_expand on the same
inputs, through the C ABI: every output array bit-equal, on two calls in a row with the second on fewer rows (the
static scratch keeps the first call's contents), for a lifted and a ground task and the no-op filter; and the
library's allocation count (mya_memory_usage_get) unchanged across every no-alloc call."""

import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def walk_states(task, rows, steps, seed):
    """Device rows of `rows` envs of the task after `steps` random-policy steps."""
    from mymyr_amd import rl

    pool = rl.DeviceEnvPool(task, rows, seed=seed)
    pool.reset()
    for _ in range(steps):
        pool.step()
    return pool.states.clone()


def run(fn, task, states, drop_noops, cap=None):
    """One expansion through `fn` (mya_expand or mya_expand_noalloc) into fresh buffers sized by a counting call."""
    from mymyr_amd import _lib
    from mymyr_amd._lib import check

    s = states.contiguous()
    rows, w = s.shape
    opts = _lib.ExpandOptions(1, 0, 1, int(drop_noops))
    stream = torch.cuda.current_stream().cuda_stream
    if cap is None:
        probe = _lib.Expansion()
        check(fn(task.handle, s.data_ptr(), rows, w, ctypes.byref(opts), ctypes.byref(probe), stream))
        cap = probe.generated
    L = max(1, task.label_width)
    dev = s.device
    out = {
        "succ": torch.zeros((cap, task.words), dtype=torch.int64, device=dev),
        "parent": torch.full((cap,), -7, dtype=torch.int32, device=dev),
        "schema": torch.full((cap,), -7, dtype=torch.int32, device=dev),
        "binding": torch.full((cap, L), -7, dtype=torch.int32, device=dev),
        "goal": torch.full((cap,), 7, dtype=torch.uint8, device=dev),
        "offsets": torch.full((rows + 1,), -7, dtype=torch.int32, device=dev),
        "succ_hash": torch.zeros(cap, dtype=torch.int64, device=dev),
        "noop": torch.full((cap,), 7, dtype=torch.uint8, device=dev),
        "index": torch.full((cap,), -7, dtype=torch.int32, device=dev),
    }
    p = {k: v.data_ptr() for k, v in out.items()}
    x = _lib.Expansion(cap, task.words, L, p["succ"], p["parent"], p["schema"], p["binding"], p["goal"], p["offsets"], p["succ_hash"],
                       p["noop"], p["index"], 0, 0, 0, 0)
    check(fn(task.handle, s.data_ptr(), rows, w, ctypes.byref(opts), ctypes.byref(x), stream))
    torch.cuda.synchronize()
    res = {k: v.cpu().numpy() for k, v in out.items()}
    res["counts"] = (x.generated, x.total, x.words_needed)
    return res


@pytest.mark.parametrize("name,atoms,rows,steps", [("transport", "auto", 6000, 9), ("strips", "dense", 3000, 3),
                                                   ("gridworld", "auto", 5000, 17)])
def test_noalloc_expand_equals_expand(golden, name, atoms, rows, steps):
    from mymyr_amd._lib import MyaError, lib
    from mymyr_amd.task import Task

    print(f"noalloc expand: {name} rows {rows}", flush=True)
    task = Task.from_text_file(golden.task_path(name), atoms)
    states = walk_states(task, rows, steps, seed=11)
    # the task's device image goes up with the first allocating call
    _ = run(lib.mya_expand, task, states[:0], False, cap=0)
    from mymyr_amd._lib import memory_usage

    for drop in (False, True):
        for n in (rows, rows // 3 + 1):  # the second call on fewer rows: the static scratch holds the first call's data
            a = run(lib.mya_expand, task, states[:n], drop)
            before = memory_usage()
            b = run(lib.mya_expand_noalloc, task, states[:n], drop)
            after = memory_usage()
            # no device block handed out (from the driver or the library's cache) and none taken from the driver
            assert (after["allocations"], after["driver_allocations"]) == (before["allocations"], before["driver_allocations"]), (n, drop)
            assert a["counts"] == b["counts"], (n, drop)
            for k in a:
                if k != "counts":
                    assert np.array_equal(a[k], b[k]), (k, n, drop)
    # rows past the static scratch's maximum are refused with a clear error
    big = torch.zeros((lib_max() + 1, task.words), dtype=torch.int64, device="cuda")
    from mymyr_amd import _lib

    x = _lib.Expansion()
    opts = _lib.ExpandOptions(1, 0, 1, 0)
    rc = lib.mya_expand_noalloc(task.handle, big.data_ptr(), big.shape[0], task.words, ctypes.byref(opts), ctypes.byref(x), None)
    assert rc != 0 and "static scratch" in lib.mya_last_error().decode()
    with pytest.raises(MyaError):
        from mymyr_amd._lib import check

        check(rc)


def lib_max():
    return 262144


def test_noalloc_refuses_a_task_without_device_image(golden):
    """The no-alloc call never uploads a task: a task that no earlier call took to the device is refused."""
    from mymyr_amd import _lib
    from mymyr_amd._lib import lib
    from mymyr_amd.task import Task

    task = Task.from_text_file(golden.task_path("gridworld"))
    states = torch.zeros((4, task.words), dtype=torch.int64, device="cuda")
    x = _lib.Expansion()
    opts = _lib.ExpandOptions(1, 0, 1, 0)
    rc = lib.mya_expand_noalloc(task.handle, states.data_ptr(), 4, task.words, ctypes.byref(opts), ctypes.byref(x), None)
    assert rc != 0 and "device image" in lib.mya_last_error().decode()
