"""Host-side checks of the product library (no GPU needed): the C ABI loads and exports every symbol that
include/mymyr_amd.h declares, the task compiler reproduces the reference's atom slots, host hash / Philox functions
match the golden vectors, and argument errors surface as MyaError with the reference's messages."""

import ctypes
import hashlib
import os
import re

import numpy as np
import pytest

from mymyr_amd import _lib, gen, workloads
from mymyr_amd._lib import MyaError, lib
from mymyr_amd.task import Task

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_symbols():
    text = open(os.path.join(ROOT, "include", "mymyr_amd.h")).read()
    return sorted(set(re.findall(r"\b(mya_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    syms = declared_symbols()
    assert len(syms) >= 25
    missing = [s for s in syms if not hasattr(lib, s)]
    assert not missing, missing
    assert lib.mya_abi_version() == _lib.ABI_VERSION


def test_symbols_are_plain_c():
    # no C++ types cross the boundary: the exported names are unmangled
    dll = ctypes.CDLL(_lib.LIB_PATH)
    for s in declared_symbols():
        assert getattr(dll, s) is not None


ALL_TASKS = ["gripper__prob05", "blocks__probBLOCKS-8-0", "depot__p02", "driverlog__p03", "logistics00__probLOGISTICS-6-1",
             "miconic__s7-4", "parcprinter-opt11-strips__p03", "pathways__p02", "pegsol-08-strips__p22", "rovers__p02",
             "snake-opt18-strips__p05", "sokoban-opt08-strips__p14", "transport-opt08-strips__p23",
             "visitall__visitall_x-6_y-3_r-100", "zenotravel__p05", "gridworld", "strips", "transport", "transport_xl",
             "freecell__p02", "folding-opt23-adl__p01", "miconic-simpleadl__s10-2", "caldera-split-opt18-adl__p04"]


@pytest.mark.parametrize("name", ALL_TASKS)
def test_slot_tables_match_reference(golden, name):
    slots = golden.load("slots.json")
    for atoms in ["auto", "dense", "reachable"]:
        t = Task.from_text_file(golden.task_path(name), atoms)
        g = slots[f"{name}:{atoms}"]
        assert (t.words, t.atom_mode, t.fluent_slots, t.dense_fluent) == (g["words"], g["mode"], g["slots"], g["dense_fluent"])
        rec, cid = t.slot_records()
        assert hashlib.sha256(cid.astype(np.uint64).tobytes()).hexdigest() == g["cid_sha"]
        assert hashlib.sha256(rec.astype(np.uint32).tobytes()).hexdigest() == g["rec_sha"]
        assert [f"{int(x):016x}" for x in t.initial_state()] == g["initial"]


def test_workload_task_files_are_reproducible(golden):
    for name in workloads.TASKS:
        assert open(golden.task_path(name)).read() == workloads.TASKS[name](), name


def test_host_hash_and_philox(golden):
    g = golden.load("hash.json")
    for c in g["cases"]:
        w = np.array([int(x, 16) for x in c["words"]], dtype=np.uint64)
        assert lib.mya_hash_words(w.ctypes.data, w.size, int(c["seed"], 16)) == int(c["hash_words"], 16)
        assert lib.mya_hash_state(w.ctypes.data, w.size) == int(c["hash_state"], 16)
    p = golden.load("philox.json")
    out = np.zeros(4, np.uint32)
    for d in p["draws"]:
        lib.mya_philox(d["seed"], d["env"], d["draw"], 0, out.ctypes.data)
        assert list(out) == d["block"]
        assert lib.mya_successor_index(d["seed"], d["env"], d["draw"], d["count"]) == d["index"]


def test_successor_index_large_counts():
    """The library's successor index at counts up to 2^32 - 1: the high word of the 128-bit product of the draw's 64
    Philox bits and the count (rng.hpp:73-84), whose low partial product's carry small counts almost never show."""
    from oracle import port

    rng = np.random.default_rng(23)
    for _ in range(3000):
        seed, env, draw = (int(x) for x in rng.integers(0, 2**63, size=3, dtype=np.int64))
        count = int(rng.integers(1, 2**32, dtype=np.int64))
        b = port.philox_block(seed, env & 0xFFFFFFFF, draw, 0)
        assert lib.mya_successor_index(seed, env & 0xFFFFFFFF, draw, count) == ((b[0] | (b[1] << 32)) * count) >> 64


def test_task_errors():
    with pytest.raises(MyaError, match="expected"):
        Task.from_text("O 1\nQ 0\n")
    with pytest.raises(MyaError, match="numeric"):
        Task.from_text("O 0\nP 0\nN 0\n")
    with pytest.raises(MyaError, match="cannot open"):
        Task.from_text_file("/nonexistent/task.txt")
    with pytest.raises(MyaError, match="object out of range"):
        Task.from_text("O 1\nP 1\nF 1 p\nSI 0\nFI 1\n0 3\nG 0\nA 0\n")
    with pytest.raises(MyaError, match="parameters; the device path supports at most"):
        Task.from_text("O 2\nP 1\nF 1 p\nSI 0\nFI 0\nG 0\nA 1\nbig 33\nL 0\nE 1\n0\nL 0\nF 1\n0 1 0\n")


def test_conditional_effects_load_frozen_and_refuse_lazy():
    """A schema with a conditional effect (one effect with a condition) loads with frozen slots; lazy slots refuse it,
    as the lifted entry points do (the ground search is the one path that evaluates conditional effects)."""
    txt = "O 1\nP 1\nF 1 p\nSI 0\nFI 0\nG 0\nA 1\nx 1\nL 0\nE 1\n0\nL 1\n0 1 0\nF 1\n0 1 0\n"
    for atoms in ("auto", "dense", "reachable"):
        assert Task.from_text(txt, atoms).words == 1
    with pytest.raises(MyaError, match="conditional effects"):
        Task.from_text(txt, "lazy")


def test_generators_deterministic():
    assert gen.gridworld(8, 8, 0.2, seed=1) == gen.gridworld(8, 8, 0.2, seed=1)
    assert gen.gridworld(8, 8, 0.2, seed=1) != gen.gridworld(8, 8, 0.2, seed=2)
    a = gen.dedup_rows(100, 50, 16, seed=3)
    b = gen.dedup_rows(0, 150, 16, seed=3)[100:]
    assert np.array_equal(a, b)


def test_pool_sampler_resolution():
    """sampler="auto" (the reference pool's default) and "uniform" sample every instance uniformly over a table of several
    instances and nothing over one; other strings and mismatched samplers are refused (python/mymyr/rl/_sampling.py)."""
    import pytest

    from mymyr_amd.rl import InstanceSampler, resolve_sampler

    assert resolve_sampler("auto", 1) is None
    s = resolve_sampler("auto", 3)
    assert isinstance(s, InstanceSampler) and s.num_instances == 3 and s.weights is None
    assert isinstance(resolve_sampler("uniform", 2), InstanceSampler)
    assert resolve_sampler(None, 4) is None
    with pytest.raises(ValueError):
        resolve_sampler("weighted", 2)
    with pytest.raises(ValueError):
        resolve_sampler(InstanceSampler(2), 3)


def test_brfs_option_arguments_checked_on_the_host(golden):
    """search.brfs checks start / blocked_states widths, max_seconds and the cancel type before any device call, and a
    CancelToken behaves as the reference's (request() once, requested stays True)."""
    import numpy as np

    from mymyr_amd import search

    tok = search.CancelToken()
    assert not tok.requested and repr(tok) == "CancelToken(requested=False)"
    tok.request()
    tok.request()
    assert tok.requested and repr(tok) == "CancelToken(requested=True)"
    t = Task.from_text_file(golden.task_path("gripper__prob05"))
    with pytest.raises(ValueError, match="words per state"):
        search.brfs(t, start=np.zeros(t.words + 1, np.uint64))
    with pytest.raises(ValueError, match="one state"):
        search.brfs(t, start=np.zeros((2, t.words), np.uint64))
    with pytest.raises(ValueError, match="words per state"):
        search.brfs(t, blocked_states=np.zeros((3, t.words + 2), np.uint64))
    with pytest.raises(ValueError, match="max_seconds"):
        search.brfs(t, max_seconds=-1.0)
    with pytest.raises(TypeError, match="CancelToken"):
        search.brfs(t, cancel=True)
    with pytest.raises(ValueError, match="custom goal test needs threads == 1"):
        search.brfs(t, goal=lambda row: False, threads=2)


def test_brfs_result_stats_and_status():
    """BrfsResult.stats (the reference's result.stats: expanded, generated, states, pruned, seconds, memory_bytes) and
    search.Status, whose members equal the result's status strings (mymyr.search.Status)."""
    from mymyr_amd import search

    r = search.BrfsResult("out_of_states", 50, 4, 61, 0, 2, False, False, 0, 0, 0.25, 0.2, pruned=3, memory_bytes=4096)
    st = r.stats
    assert (st.expanded, st.generated, st.states, st.pruned, st.seconds, st.memory_bytes) == (4, 61, 50, 3, 0.25, 4096)
    assert r.status == search.Status.OUT_OF_STATES and r.status != search.Status.EXHAUSTED
    assert [s.name for s in search.Status] == ["SOLVED", "EXHAUSTED", "OUT_OF_STATES", "OUT_OF_TIME", "CANCELLED", "FAILED",
                                               "UNSOLVABLE"]
    assert all(search.Status(v) == v for v in search.STATUS.values())


def test_visited_mask_is_a_registered_torch_op():
    """rl.visited_mask is the torch op mymyr::visited_mask, with a fake implementation (bool [size]) for tracing."""
    torch = pytest.importorskip("torch")
    from torch._subclasses.fake_tensor import FakeTensorMode

    from mymyr_amd import rl  # noqa: F401  (registers the op)

    assert hasattr(torch.ops.mymyr, "visited_mask")
    with FakeTensorMode():
        tab, cnt = torch.empty((4, 8), dtype=torch.int64), torch.empty(4, dtype=torch.int32)
        h, par = torch.empty(10, dtype=torch.int64), torch.empty(10, dtype=torch.int32)
        out = torch.ops.mymyr.visited_mask(tab, cnt, h, par, None)
        assert out.shape == (10,) and out.dtype == torch.bool


SECTION_ERRORS = [
    ("C 1\n0 5 1 0\n", "ascend"),           # a position past the parameters before collapsing
    ("C 2\n0 1 1 0\n0 0 1 0\n", "ascend"),  # positions of one schema not ascending
    ("C 1\n9 0 1 0\n", "unknown schema"),
    ("C 1\n0 0 1 999\n", "representative"),
    ("EG 1 1\n99 1 0\n", "predicate"),
    ("EG 1 1\n6 1 999 1\n", "object"),
    ("C 0\nX 0\n", "unexpected section"),  # the sections' order is X, C, EG (what follows EG is not read)
    ("Z 1\n", "unexpected section"),
]


@pytest.mark.parametrize("appendix,match", SECTION_ERRORS)
def test_malformed_c_and_eg_sections_are_refused_as_the_reference_does(golden, appendix, match, tmp_path):
    """The reader checks the C and EG sections as the reference's reader and validator do (text_format.cpp:140-187,
    task_data.cpp:129-147): both refuse each of these appendices to a valid task."""
    from mymyr_amd._lib import MyaError
    from oracle import ref

    text = open(golden.task_path("gripper__prob05")).read().rstrip("\n") + "\n" + appendix
    with pytest.raises(MyaError, match=match):
        Task.from_text(text)
    if ref.available():
        p = tmp_path / "t.txt"
        p.write_text(text)
        with pytest.raises(Exception):
            ref.RefTask(str(p))


def test_c_and_eg_sections_are_read(golden):
    """Valid C and EG sections load; a schema whose collapsed parameter has no representative has no successors."""
    from mymyr_amd import gen  # noqa: F401

    for name in ("sections_gripper_rep", "sections_gripper_norep", "sections_blocks_norep", "sections_logistics_eg"):
        Task.from_text_file(golden.task_path(name))


def test_lazy_slots_after_load_equal_the_reference(golden):
    """atoms="lazy": the slots start with the initial state's atoms, in its atom order (src/mymyr/task/task.cpp:214-224),
    record for record the reference's lazy AtomIndex right after loading."""
    init = golden.load("lazy.json")["initial"]
    for name, g in init.items():
        t = Task.from_text_file(golden.task_path(name), "lazy")
        assert (t.atom_mode, t.words, t.fluent_slots, t.frozen) == ("lazy", g["words"], g["slots"], False), name
        rec, cid = t.slot_records()
        assert [int(x) for x in cid] == g["cid"], name
        assert hashlib.sha256(rec.astype(np.uint32).tobytes()).hexdigest() == g["rec_sha"], name
        assert [f"{int(x):016x}" for x in t.initial_state()] == g["initial"], name


def test_lazy_tasks_refused_by_env_tables(golden):
    """Environments and task tables need a fixed slot layout (src/mymyr/rl/task_table.cpp:120-123): the refusal comes
    before any device work."""
    t = Task.from_text_file(golden.task_path("gripper__prob05"), "lazy")
    cfg = _lib.EnvConfig(0, 0, 0.0, 1.0, 0.0, 0, 1, 1, 1, 0, 0)
    h = ctypes.c_void_p()
    assert lib.mya_env_create(t.handle, ctypes.byref(cfg), ctypes.byref(h)) != 0
    assert "lazy atom slots" in lib.mya_last_error().decode()
    with pytest.raises(MyaError, match="atoms 'auto', 'reachable' or 'dense'"):
        from mymyr_amd import rl

        rl.TaskTable([Task.from_text_file(golden.task_path("gripper__prob05")), t])
    with pytest.raises(MyaError, match="atoms must be"):
        _lib.check(lib.mya_task_load_file(golden.task_path("gripper__prob05").encode(), 4, ctypes.byref(h)))
