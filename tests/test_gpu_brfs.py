"""The device BrFS against the reference: the suite's published exhaustive counts (tests/cpp/support/suite.hpp:33-56),
the reference's own determinism digests (tests/data/determinism.json), and the compiled reference's layer counts,
fingerprints and statuses (tests/golden/brfs.json), including the strips workload's max_states cuts."""

import pytest

pytestmark = pytest.mark.gpu

pytest.importorskip("torch")

KEYS = ["states", "expanded", "generated", "goal_states", "layers", "fingerprint", "status", "layer_counts", "exhausted", "solved"]
STATUS = {0: "solved", 1: "exhausted", 2: "out_of_states", 3: "out_of_time", 4: "cancelled"}


def device(golden, name, atoms="auto", full=False, **kw):
    from mymyr_amd import search
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path(name), atoms)
    r = search.brfs(t, fingerprint=True, **kw)
    out = {"states": r.states, "expanded": r.expanded, "generated": r.generated, "goal_states": r.num_goal_states,
           "layers": r.layers, "fingerprint": r.fingerprint, "status": r.status, "layer_counts": r.layer_counts,
           "exhausted": r.exhausted, "solved": r.solved}
    if full:
        out["result"] = r
    return out


def trimmed_hex(words):
    w = [int(x, 16) if isinstance(x, str) else int(x) for x in words]
    while w and w[-1] == 0:
        w.pop()
    return w


def goal_cids(task, words):
    """The canonical atom ids of a state's set slots under the task's slots, ascending."""
    _, cid = task.slot_records()
    return sorted(int(cid[w * 64 + b]) for w, x in enumerate(words) for b in range(64) if (int(x) >> b) & 1)


def same_plan(r, exp, task=None):
    """The device's plan, cost and goal state against the reference's (BrfsResult::plan, cost, goal_state). With `task`
    (loaded with other slots than the reference's auto ones), the goal states are compared as canonical atom ids."""
    res = r["result"]
    if not exp["solved"]:
        return res.plan == [] and res.cost == 0.0 and res.goal_state is None
    if task is not None:
        same_goal = goal_cids(task, res.goal_state) == exp["goal_cids"]
    else:
        same_goal = trimmed_hex(res.goal_state) == trimmed_hex(exp["goal_state"])
    return [[a.schema, *a.binding] for a in res.plan] == exp["plan"] and res.cost == exp["cost"] and same_goal


def same(r, exp):
    bad = {k: (r[k], exp[k] if k != "status" else STATUS.get(exp[k], exp[k])) for k in KEYS
           if (r[k] != (STATUS.get(exp[k], exp[k]) if k == "status" else exp[k]))}
    return bad


# the host's relaxed-reachability fixpoint (the auto mode's choice of slots) takes about two minutes on
# organic-synthesis, whose schemas have up to 31 parameters; its search does not depend on the slots, so it is loaded
# with dense slots (47 words; the auto mode's reachable slots take 21), and goal states compare as canonical atoms
SUITE_ATOMS = {"organic-synthesis-opt18-strips__p20": "dense"}


@pytest.mark.parametrize("name", ["gripper__prob05", "blocks__probBLOCKS-8-0", "depot__p02", "miconic__s7-4", "pegsol-08-strips__p22",
                                  "parcprinter-opt11-strips__p03", "visitall__visitall_x-6_y-3_r-100", "sokoban-opt08-strips__p14",
                                  "driverlog__p03", "logistics00__probLOGISTICS-6-1", "pathways__p02", "zenotravel__p05",
                                  "transport-opt08-strips__p23", "snake-opt18-strips__p05", "freecell__p02",
                                  "folding-opt23-adl__p01", "organic-synthesis-opt18-strips__p20",
                                  "miconic-simpleadl__s10-2", "caldera-split-opt18-adl__p04"])
def test_suite_exhaustive(golden, name):
    states, generated, goals = golden.SUITE_COUNTS[name]
    print(f"suite: {name}", flush=True)
    r = device(golden, name, SUITE_ATOMS.get(name, "auto"), stop_at_goal=False)
    assert (r["states"], r["generated"], r["goal_states"]) == (states, generated, goals)
    exp = golden.load("brfs.json")["suite"].get(name)
    if exp:
        assert not same(r, exp), same(r, exp)


@pytest.mark.parametrize("name", list(__import__("tests.golden.fixtures", fromlist=["x"]).DETERMINISM_BRFS))
def test_reference_determinism_digests(golden, name):
    r = device(golden, name, stop_at_goal=False, max_states=20000)
    assert golden.determinism_digest(r["states"], r["expanded"], r["generated"], r["layers"], r["fingerprint"]) == \
        golden.DETERMINISM_BRFS[name]


def test_budget_and_goal_stops(golden):
    """max_states and max_expanded cuts and goal stops of the suite: counts, statuses and fingerprints, and for the
    solved searches the plan (the first discoveries from the start state to the first goal state), its cost and the
    goal state, all equal to the reference's."""
    from mymyr_amd.task import Task

    g = golden.load("brfs.json")["budget"]
    solved = 0
    for key, exp in g.items():
        name = key.split(":")[0]
        kw = dict(exp["options"])
        r = device(golden, name, SUITE_ATOMS.get(name, "auto"), full=True, **kw)
        assert not same(r, exp), (key, same(r, exp))
        other = Task.from_text_file(golden.task_path(name), SUITE_ATOMS[name]) if name in SUITE_ATOMS else None
        assert same_plan(r, exp, other), (key, r["result"].plan[:4], exp.get("plan", [])[:4])
        solved += bool(exp["solved"])
    assert solved >= 10


def test_plan_replays_to_the_goal_state(golden):
    """A device plan applied step by step with the oracle's successor function from the initial state reaches the
    reported goal state, which satisfies the goal; every step is an applicable action of the state before it."""
    from mymyr_amd.task import Task
    from oracle import port

    for name in ("gripper__prob05", "depot__p02", "logistics00__probLOGISTICS-6-1"):
        text = open(golden.task_path(name)).read()
        r = device(golden, name, full=True, stop_at_goal=True)["result"]
        assert r.solved and len(r.plan) == r.cost > 0
        pt = port.Task(text)
        row = pt.initial
        for a in r.plan:
            nxt = [s for (sc, b, s) in port.successors(pt, row) if sc == a.schema and tuple(b[: len(a.binding)]) == a.binding]
            assert len(nxt) == 1, (name, a)
            row = nxt[0]
        assert trimmed_hex(row) == trimmed_hex(r.goal_state)
        assert port.is_goal(pt, row)


def test_strips_workload_cuts(golden):
    """The strips workload's searches (512 fluents, 4096 actions) at max_states 2^20, 2^22, 2^24, 2^26 and 2^28 (1.18 G
    successors, a 4 GiB table), its depth, expansion and goal cuts: counts, layers and fingerprints equal to the
    reference's single-threaded search."""
    g = golden.load("brfs.json")["strips"]
    for key, exp in g.items():
        r = device(golden, "strips", "dense", **exp["options"])
        assert not same(r, exp), (key, same(r, exp))


def custom_goal_keys():
    from tests.golden import fixtures

    return sorted(fixtures.load("brfs_custom_goal.json"))


@pytest.mark.parametrize("key", custom_goal_keys())
def test_custom_goal_test(golden, key):
    """BrfsOptions::goal as a callable (GoalSpec::Custom): a state is a goal iff its hash_state % m == r, which no atom
    goal expresses, through the ground driver (gripper) and the wide one (20-word rows), and under lazy slots iff it has
    k true atoms (a test the device's own slot numbering leaves alone); with the goal stop, over the whole space and at
    a cut: counts, fingerprints, statuses and plans equal to the reference's with the same test."""
    from mymyr_amd.task import Task
    from oracle import port

    exp = golden.load("brfs_custom_goal.json")[key]
    calls = [0]
    if "goal_hash" in exp:
        m, res = exp["goal_hash"]

        def goal(row):
            calls[0] += 1
            return port.hash_state(row) % m == res
    else:
        k = exp["goal_atoms"]

        def goal(row):
            calls[0] += 1
            return sum(bin(int(w)).count("1") for w in row) == k

    print(f"custom goal: {key}", flush=True)
    opts = {o: v for o, v in exp["options"].items() if o not in ("goal_hash", "goal_atoms")}  # the reference's form of the test
    name, atoms = key.split(":")[0], exp["atoms"]
    if atoms == "lazy":
        # lazy slots number the atoms in the order the search meets them: the goal state compares by canonical ids
        from mymyr_amd import search

        t = Task.from_text_file(golden.task_path(name), "lazy")
        res = search.brfs(t, fingerprint=True, goal=goal, **opts)
        got = {"states": res.states, "expanded": res.expanded, "generated": res.generated, "goal_states": res.num_goal_states,
               "layers": res.layers, "fingerprint": res.fingerprint, "status": res.status, "layer_counts": res.layer_counts,
               "exhausted": res.exhausted, "solved": res.solved, "result": res}
        assert not same(got, exp), (key, same(got, exp))
        assert same_plan(got, exp, t)
    else:
        r = device(golden, name, atoms, full=True, goal=goal, **opts)
        assert not same(r, exp), (key, same(r, exp))
        assert same_plan(r, exp)
    assert calls[0] >= exp["expanded"]  # every expanded state was tested


def test_custom_goal_test_errors(golden):
    """An exception in the goal test stops the search and is raised again; the threads check is the reference's."""
    from mymyr_amd import search
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path("gripper__prob05"))

    class Stop(Exception):
        pass

    def goal(row):
        raise Stop()

    with pytest.raises(Stop):
        search.brfs(t, goal=goal, stop_at_goal=False, max_states=5000)
    # the search runs again afterwards
    assert search.brfs(t, goal=lambda row: False, stop_at_goal=False, max_states=5000).states == 5000


def edge_keys():
    from tests.golden import fixtures

    return sorted(fixtures.load("brfs_edges.json"))


@pytest.mark.parametrize("key", edge_keys())
def test_budgets_at_the_edges(golden, key):
    """max_states of 1, 2 and 50, max_expanded of 0, 1 and 5 and max_depth of 0, 1 and 2 (with and without the goal
    stop) through the ground driver, the wide one (20-word rows) and lazy slots: counts, layers, statuses and
    fingerprints equal to the reference's (its own checks of these budgets: tests/python/test_search.py:120-136)."""
    exp = golden.load("brfs_edges.json")[key]
    name, atoms = key.split(":")[:2]
    print(f"edge budget: {key}", flush=True)
    r = device(golden, name, atoms, **exp["options"])
    assert not same(r, exp), (key, same(r, exp))
    if "max_states" in exp["options"]:
        assert r["states"] == exp["options"]["max_states"]


def test_small_chunks_do_not_change_results(golden):
    """Chunked layers (tiny candidate buffers) give the same ids and counts."""
    a = device(golden, "gripper__prob05", stop_at_goal=False)
    b = device(golden, "gripper__prob05", stop_at_goal=False, chunk=64)
    assert a == b




@pytest.mark.parametrize("key", ["witness_order_5", "witness_order_5:goal", "witness_order_0:goal", "witness_order_0:cut",
                                 "rovers__p02", "rovers__p02:goal", "rovers__p02:expanded"])
def test_several_witness_parameters(golden, key):
    """Witness pruning over schemas with two witness parameters, which the reference's matcher binds in its own order
    (here not the parameter order): counts, fingerprints, statuses and, for solved searches, plans (whose labels carry
    the witness objects the matcher finds first) equal to the reference's."""
    exp = golden.load("brfs_witness.json")[key]
    name = key.split(":")[0]
    r = device(golden, name, full=True, **exp["options"])
    assert not same(r, exp), (key, same(r, exp))
    assert same_plan(r, exp), (key, r["result"].plan[:6], exp.get("plan", [])[:6])


WIDE_ATOMS = {"witness_wide": "dense"}


@pytest.mark.parametrize("key", ["transport_w20_3:goal", "transport_w20_7:goal", "transport_w20_3:cut", "transport_w20_7:expanded",
                                 "transport:cut", "transport:depth2", "witness_wide:cut", "witness_wide:witness_cut",
                                 "witness_wide:witness_depth", "witness_wide:witness_goal"])
def test_wide_rows(golden, key):
    """Rows wider than 16 words (typed transport of 20 and of 176 words, a 19-word dense task) take the driver over the
    lifted expansion: layer counts, fingerprints, statuses, cuts and plans equal to the reference's. The 19-word task's
    schemas have witness parameters: with witness pruning on (the reference's default) the expansion keeps one
    successor per effect-relevant binding, with the witnesses the reference's matcher binds first."""
    exp = golden.load("brfs_wide.json")[key]
    name = key.split(":")[0]
    print(f"wide brfs: {key}", flush=True)
    r = device(golden, name, WIDE_ATOMS.get(name, "auto"), full=True, **exp["options"])
    assert not same(r, exp), (key, same(r, exp))
    assert same_plan(r, exp), (key, r["result"].plan[:6], exp.get("plan", [])[:6])


def _rows(words, hexrows):
    import numpy as np

    out = np.zeros((len(hexrows), words), np.uint64)
    for i, r in enumerate(hexrows):
        w = trimmed_hex(r)
        assert len(w) <= words
        out[i, : len(w)] = w
    return out


OPTION_KEYS = [
    "gripper__prob05:blocked_goal", "gripper__prob05:blocked_all", "gripper__prob05:start_goal", "gripper__prob05:blocked_cut",
    "gripper__prob05:start_blocked_expanded", "gripper__prob05:timed0", "blocks__probBLOCKS-8-0:blocked_goal",
    "logistics00__probLOGISTICS-6-1:start_blocked", "strips:blocked_cut", "transport_w20_3:blocked_goal",
    "transport_w20_3:start_goal", "transport_w20_3:blocked_cut"]


@pytest.mark.parametrize("key", OPTION_KEYS)
def test_start_and_blocked_states(golden, key):
    """BrfsOptions::start and blocked_states (and max_seconds 0): a successor equal to a blocked state counts as
    generated and pruned and is never stored (the start state is exempt, a successor equal to it and blocked is
    pruned), the search and its plan start at `start`; counts, pruned, statuses, fingerprints and plans equal to the
    reference's, on the ground-action driver and on the wide-row driver, at goal stops and at max_states and
    max_expanded cuts."""
    from mymyr_amd import search
    from mymyr_amd.task import Task

    exp = golden.load("brfs_options.json")[key]
    name = key.split(":")[0]
    t = Task.from_text_file(golden.task_path(name), exp["atoms"])
    kw = dict(exp["options"])
    if exp["start"] is not None:
        kw["start"] = _rows(t.words, [exp["start"]])[0]
    if exp["blocked"]:
        kw["blocked_states"] = _rows(t.words, exp["blocked"])
    print(f"brfs options: {key}", flush=True)
    for chunk in ((0, 4096) if name == "strips" else (0,)):
        r = search.brfs(t, fingerprint=True, chunk=chunk, **kw)
        got = {"states": r.states, "expanded": r.expanded, "generated": r.generated, "goal_states": r.num_goal_states,
               "layers": r.layers, "fingerprint": r.fingerprint, "status": r.status, "layer_counts": r.layer_counts,
               "exhausted": r.exhausted, "solved": r.solved, "result": r}
        assert not same(got, exp), (key, chunk, same(got, exp))
        assert r.pruned == exp["pruned"], (key, chunk, r.pruned, exp["pruned"])
        assert same_plan(got, exp), (key, r.plan[:6], exp.get("plan", [])[:6])


def _consistent(r):
    lc = r.layer_counts
    return (sum(x[0] for x in lc) == r.expanded and sum(x[1] for x in lc) == r.generated and
            sum(x[2] for x in lc) + 1 == r.states and len(lc) == r.layers)


def test_cancel_and_time_stop_between_batches(golden):
    """A CancelToken requested before the search stops it before the first expansion; one requested from another thread
    and a max_seconds budget stop a long search between device batches: status "cancelled" / "out_of_time", the
    layers before the last equal to the uncut search's, and counts that add up."""
    import threading
    import time

    from mymyr_amd import search
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path("strips"), "dense")
    full = golden.load("brfs.json")["strips"][str(1 << 24)]
    tok = search.CancelToken()
    tok.request()
    r = search.brfs(t, max_depth=12, max_states=1 << 24, stop_at_goal=False, cancel=tok)
    assert (r.status, r.states, r.expanded, r.layers) == ("cancelled", 1, 0, 0)

    r = search.brfs(t, max_depth=12, max_states=1 << 24, stop_at_goal=False, max_seconds=0.02, chunk=1 << 16)
    assert r.status == "out_of_time" and r.states < full["states"] and _consistent(r), (r.status, r.states)
    assert r.layer_counts[:-1] == full["layer_counts"][: max(0, r.layers - 1)]

    tok = search.CancelToken()
    timer = threading.Timer(0.02, tok.request)
    t0 = time.perf_counter()
    timer.start()
    r = search.brfs(t, max_depth=12, max_states=1 << 24, stop_at_goal=False, cancel=tok, chunk=1 << 16)
    timer.join()
    if r.status != "cancelled":
        # the whole search finished inside the timer's delay: nothing to stop
        assert r.status == "out_of_states" and time.perf_counter() - t0 < 0.5
    else:
        assert r.states < full["states"] and _consistent(r)
        assert r.layer_counts[:-1] == full["layer_counts"][: max(0, r.layers - 1)]


@pytest.mark.parametrize("key", ["sections_gripper_rep:goal", "sections_gripper_rep:all", "sections_gripper_norep:goal",
                                 "sections_gripper_norep:all", "sections_blocks_norep:goal", "sections_blocks_norep:all",
                                 "sections_logistics_eg:goal", "sections_logistics_eg:all"])
def test_tasks_with_collapsed_parameters_and_encoding_goal(golden, key):
    """Tasks with the C (collapsed parameters) and EG (encoding goal) sections: a collapsed parameter without a
    representative leaves its schema without actions (src/mymyr/task/compile.cpp:1171-1181), one with a representative
    changes nothing, and the encoding goal does not touch the search; counts, fingerprints and plans equal to the
    reference's on the same text."""
    exp = golden.load("brfs_sections.json")[key]
    name = key.split(":")[0]
    r = device(golden, name, full=True, **exp["options"])
    assert not same(r, exp), (key, same(r, exp))
    assert same_plan(r, exp), (key, r["result"].plan[:4], exp.get("plan", [])[:4])


GOAL_KEYS = sorted(__import__("json").load(open(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                                                          "brfs_goals.json"))))


@pytest.mark.parametrize("key", GOAL_KEYS)
def test_any_of_goals(golden, key):
    """BrfsOptions::goal as GoalSpec::AnyOf over ground conditions (search::any_of: static literals decided, fluent atoms
    resolved to slots, interned at the search's start under lazy slots; impossible conditions left out): goal stops with
    their plans and goal states, goal-state counts over whole searches, a max_states cut and conditions that can never
    hold, on the ground-action driver (gripper, blocks), the wide-row driver (20-word transport) and lazy slots; and the
    result's words, fluent_slots, threads_used and message, all equal to the compiled reference's (words as its flat
    store reports them)."""
    from mymyr_amd import search
    from mymyr_amd.task import Task

    exp = golden.load("brfs_goals.json")[key]
    name = key.split(":")[0]
    print(f"any-of goals: {key}", flush=True)
    t = Task.from_text_file(golden.task_path(name), exp["atoms"])
    goal = [[(p, pos, objs) for p, pos, objs in cond] for cond in exp["goal"]]
    r = search.brfs(t, fingerprint=True, goal=goal, **exp["options"])
    got = {"states": r.states, "expanded": r.expanded, "generated": r.generated, "goal_states": r.num_goal_states,
           "layers": r.layers, "fingerprint": r.fingerprint, "status": r.status, "layer_counts": r.layer_counts,
           "exhausted": r.exhausted, "solved": r.solved, "result": r}
    assert not same(got, exp), (key, same(got, exp))
    assert same_plan(got, exp), (key, r.plan[:6], exp.get("plan", [])[:6])
    assert (r.fluent_slots, r.threads_used, r.message) == (exp["fluent_slots"], exp["threads_used"], exp["message"])
    # words: the fluent width of the stored rows at the end; the reference's flat store reports the same, its chunked
    # store (rows above 8 words) its width rounded up to whole 8-word chunks
    assert r.words == t.words
    assert r.words == exp["words"] if exp["store"] == "flat" else exp["words"] == (r.words + 7) // 8 * 8
    assert r.store == "device"


def test_any_of_goal_errors(golden):
    """Invalid goal literals are refused with the reference's GroundCondition::validate messages."""
    from mymyr_amd import search
    from mymyr_amd._lib import MyaError
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path("gripper__prob05"))
    with pytest.raises(MyaError, match="predicate index 99 out of range"):
        search.brfs(t, goal=[[(99, True, [0])]])
    with pytest.raises(MyaError, match="takes 2 arguments, got 1"):
        search.brfs(t, goal=[[(6, True, [0])]])
    with pytest.raises(MyaError, match="object index 1000 out of range"):
        search.brfs(t, goal=[[(6, True, [0, 1000])]])


def test_conditional_effects_refused_by_lifted_entry_points(golden):
    """The ground search evaluates conditional effects (test_suite_exhaustive covers miconic-simpleadl and caldera);
    the lifted expansion, the successor listing and the environment refuse such a task with an error."""
    import torch

    from mymyr_amd import rl
    from mymyr_amd._lib import MyaError
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path("miconic-simpleadl__s10-2"))
    rows = torch.from_numpy(t.initial_state().view("int64")).reshape(1, -1).cuda()
    with pytest.raises(MyaError, match="conditional effects"):
        rl.expand(t, rows)
    with pytest.raises(MyaError, match="conditional effects"):
        rl.successors(t, rows)
    with pytest.raises(MyaError, match="conditional effects"):
        rl.EnvPool(t, 4)


def test_observer_events(golden):
    """BrfsOptions::observer (include/mymyr/search/control.hpp:157-186) on the device search: on_start with the start
    state, on_pass per layer with the reference-pinned layer counts, on_solution with the plan and on_end with the
    result's status and totals (Control::finish, src/mymyr/search/brfs.cpp:193-211); on_progress every
    progress_interval expansions, False stopping the search as cancelled; an exception in an event stops the search and
    is raised; per-state events are refused."""
    from mymyr_amd import search
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path("gripper__prob05"))

    class Rec(search.Observer):
        def __init__(self):
            self.ev = []

        def on_start(self, state):
            self.ev.append(("start", [int(x) for x in state]))

        def on_pass(self, width, stats):
            self.ev.append(("pass", width, stats.expanded, stats.generated, stats.states))

        def on_progress(self, stats):
            self.ev.append(("progress", stats.expanded, stats.generated, stats.states))
            return True

        def on_solution(self, plan, cost):
            self.ev.append(("solution", plan, cost))

        def on_end(self, status, stats):
            self.ev.append(("end", status, stats.expanded, stats.generated, stats.states, stats.pruned))

    # gripper over the ground driver (to its goal and exhaustively), a 20-word transport task over the lifted one
    for name, stop in (("gripper__prob05", True), ("gripper__prob05", False), ("transport_w20_3", True)):
        t = Task.from_text_file(golden.task_path(name))
        o = Rec()
        r = search.brfs(t, stop_at_goal=stop, observer=o, progress_interval=5000)
        assert o.ev[0] == ("start", [int(x) for x in t.initial_state()])
        passes = [e for e in o.ev if e[0] == "pass"]
        assert [p[1] for p in passes] == list(range(len(r.layer_counts)))
        assert [list(p[2:]) for p in passes] == r.layer_counts
        prog = [e for e in o.ev if e[0] == "progress"]
        assert (prog or r.expanded < 100000) and all(b[1] - a[1] >= 5000 for a, b in zip(prog, prog[1:]))
        assert all(p[1] >= 5000 and p[1] <= r.expanded for p in prog)
        sol = [e for e in o.ev if e[0] == "solution"]
        assert (len(sol) == 1 and sol[0][1] == r.plan and sol[0][2] == r.cost) if r.solved else not sol
        assert o.ev[-1] == ("end", r.status, r.expanded, r.generated, r.states, r.pruned)

    class Stop(search.Observer):
        def __init__(self):
            self.calls = 0

        def on_progress(self, stats):
            self.calls += 1
            return False

    t = Task.from_text_file(golden.task_path("gripper__prob05"))
    o = Stop()
    r = search.brfs(t, stop_at_goal=False, observer=o, progress_interval=1)
    full = search.brfs(t, stop_at_goal=False)
    assert r.status == "cancelled" and o.calls == 1 and r.expanded < full.expanded

    class Boom(search.Observer):
        def on_pass(self, width, stats):
            if width == 3:
                raise RuntimeError("boom")

    with pytest.raises(RuntimeError, match="boom"):
        search.brfs(t, stop_at_goal=False, observer=Boom())

    class Boom2(search.Observer):
        def on_generate(self, parent, action, child, state, is_new):
            if child is not None and child > 100:
                raise KeyError("late")

    with pytest.raises(KeyError, match="late"):
        search.brfs(t, stop_at_goal=False, observer=Boom2())


@pytest.mark.parametrize("key", list(__import__("json").load(open(__import__("os").path.join(
    __import__("os").path.dirname(__file__), "golden", "brfs_layers.json")))))
def test_layer_orders(golden, key):
    """BrfsOptions::layers (include/mymyr/search/layer_ordering.hpp; src/mymyr/search/brfs.cpp:300-382 with
    layer_order_detail.hpp): in-order, reverse and SplitMix64-randomized layers, goal-count ranks (most or fewest
    satisfied first, random tie tokens) and scored ranks, beams and max_next_layer_states cuts, over ground, wide-row
    and lazy tasks: counts, layer counts, fingerprints, statuses and plans equal to the compiled reference's."""
    from mymyr_amd.task import Task

    exp = golden.load("brfs_layers.json")[key]
    name = key.split(":")[0]
    kw = dict(exp["options"])
    if kw["layer_order"] in golden.LAYER_SCORERS:
        kw["layer_order"] = golden.LAYER_SCORERS[kw["layer_order"]]
    print(f"layers: {key}", flush=True)
    if exp["atoms"] != "lazy":
        r = device(golden, name, exp["atoms"], full=True, **kw)
        assert not same(r, exp), same(r, exp)
        assert same_plan(r, exp)
        return
    # lazy slots: the plan and the goal state's atoms by canonical id (the slots the search interned are the task's)
    from mymyr_amd import search

    t = Task.from_text_file(golden.task_path(name), "lazy")
    res = search.brfs(t, fingerprint=True, witness_pruning=False, **kw)
    r = {"states": res.states, "expanded": res.expanded, "generated": res.generated, "goal_states": res.num_goal_states,
         "layers": res.layers, "fingerprint": res.fingerprint, "status": res.status, "layer_counts": res.layer_counts,
         "exhausted": res.exhausted, "solved": res.solved}
    assert not same(r, exp), same(r, exp)
    assert [[a.schema, *a.binding] for a in res.plan] == exp.get("plan", [])
    if exp["solved"]:
        assert goal_cids(t, res.goal_state) == exp["goal_cids"]


def test_layer_order_errors(golden):
    """The reference's check_layers messages (include/mymyr/search/layer_ordering.hpp:117-134) and the device's refusal of
    the relaxed survivors-only beam."""
    from mymyr_amd import search
    from mymyr_amd._lib import MyaError
    from mymyr_amd.task import Task

    t = Task.from_text_file(golden.task_path("gripper__prob05"))
    for kw, msg in [(dict(max_next_layer_states=10), "needs an ordered layer order"),
                    (dict(beam_width=10), "needs an ordered layer order"),
                    (dict(layer_order="in_order", beam_width=10, max_next_layer_states=10), "exclude each other"),
                    (dict(layer_order="in_order", beam_novelty="survivors_only"), "needs a beam"),
                    (dict(layer_order="reverse", randomize_ties=True), "randomize_ties needs"),
                    (dict(layer_order="in_order", beam_width=5, beam_novelty="relaxed_survivors_only"), "needs the goal-count"),
                    (dict(layer_order="goal_count", beam_width=5, beam_novelty="relaxed_survivors_only"), "not supported")]:
        with pytest.raises(MyaError, match=msg):
            search.brfs(t, **kw)
    for kw in (dict(layer_order="sideways"), dict(layer_order="in_order", beam_width=0),
               dict(layer_order="in_order", max_next_layer_states=0), dict(beam_novelty="none")):
        with pytest.raises(ValueError):
            search.brfs(t, **kw)
    with pytest.raises(MyaError, match="NaN"):
        search.brfs(t, stop_at_goal=False, layer_order=lambda rows: [float("nan")] * len(rows))

    class Fail(RuntimeError):
        pass

    def bad(rows):
        raise Fail("scorer")

    with pytest.raises(Fail):
        search.brfs(t, stop_at_goal=False, layer_order=bad)


@pytest.mark.parametrize("key", ["transport_w2208:depth2", "transport_w2208:cut", "transport_w2208:beam"])
def test_rows_beyond_2048_words(golden, key):
    """A transport task of 2208-word rows (141,312 atoms), past the rows the state set keeps in registers: the lifted
    driver's probe, compaction and blocked test compare, hash and copy them from memory (the reference's set takes any
    width, cuda/src/state_set.cu:456-464). Counts, layer counts, fingerprints and statuses equal the reference's."""
    exp = golden.load("brfs_long.json")[key]
    print(f"long rows: {key}", flush=True)
    r = device(golden, "transport_w2208", **exp["options"])
    assert not same(r, exp), same(r, exp)


class EventLog:
    """The observer's events as the reference harness records them (tests/golden/make_golden.py, make_brfs_events):
    7-word records, states by hash_state, bindings by h = arity, then h * 1000003 + object (mod 2^64)."""

    M = (1 << 64) - 1
    CODES = {"solved": 0, "exhausted": 1, "out_of_states": 2, "out_of_time": 3, "cancelled": 4, "failed": 5, "unsolvable": 6}

    def __init__(self):
        from mymyr_amd._lib import lib

        self.lib = lib
        self.ev = []

    def sh(self, row):
        import numpy as np

        r = np.ascontiguousarray(row, dtype=np.uint64)
        return int(self.lib.mya_hash_state(r.ctypes.data, r.size))

    def bh(self, a):
        h = len(a.binding)
        for o in a.binding:
            h = (h * 1000003 + o) & self.M
        return h

    def rec(self, *v):
        self.ev.append(list(v) + [0] * (7 - len(v)))

    def on_start(self, state):
        self.rec(0, self.sh(state))

    def on_expand(self, sid, state):
        self.rec(1, sid, self.sh(state))

    def on_generate(self, parent, action, child, state, is_new):
        self.rec(2, parent, action.schema, self.bh(action), self.M if child is None else child, self.sh(state), int(is_new))

    def on_prune(self, parent, action, state):
        self.rec(3, parent, action.schema, self.bh(action), 0, self.sh(state))

    def on_pass(self, layer, st):
        self.rec(4, layer, st.expanded, st.generated, st.states)

    def on_solution(self, plan, cost):
        h = len(plan)
        for a in plan:
            h = (h * 1000003 + a.schema * 7919 + self.bh(a)) & self.M
        self.rec(5, len(plan), h, int(cost))

    def on_end(self, status, st):
        self.rec(6, self.CODES[status], st.expanded, st.generated, st.states, st.pruned)


@pytest.mark.parametrize("key", list(__import__("json").load(open(__import__("os").path.join(
    __import__("os").path.dirname(__file__), "golden", "brfs_events.json")))))
def test_observer_per_state_events(golden, key):
    """Every observer event of a search, on_expand, on_generate (child ids, new flags, successor states) and on_prune
    included, in order, equal to the compiled reference's (src/mymyr/search/brfs.cpp:274-404): ground, conditional-effect,
    wide-row, blocked-state, beam and layer-cut searches, compared by the sha256 of their event records."""
    import hashlib

    import numpy as np

    from mymyr_amd import search
    from mymyr_amd.task import Task

    exp = golden.load("brfs_events.json")[key]
    name = key.split(":")[0]
    t = Task.from_text_file(golden.task_path(name))
    kw = dict(exp["options"])
    if exp["blocked"]:
        kw["blocked_states"] = np.array([[int(x, 16) for x in r][: t.words] + [0] * max(0, t.words - len(r)) for r in exp["blocked"]],
                                        dtype=np.uint64)
    log = EventLog()
    print(f"events: {key}", flush=True)
    search.brfs(t, observer=log, **kw)
    ev = np.array(log.ev, dtype=np.uint64)
    counts = {str(k): int((ev[:, 0] == k).sum()) for k in range(7)}
    head = [[f"{int(x):x}" for x in row] for row in ev[:60]]
    assert counts == exp["counts"], (counts, exp["counts"])
    assert head == exp["head"]
    assert hashlib.sha256(np.ascontiguousarray(ev).astype("<u8").tobytes()).hexdigest() == exp["sha256"]
