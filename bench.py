"""Benchmark of the state-expansion path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--only strips,gridworld,...] [--no-cpu] [--no-larger-budget]

Prints ONE JSON line. The headline (`value`) is the strips workload: BrFS expanded states per second of a random
ground STRIPS task (512 fluents, 4096 actions) from its initial state, depth bound 12, stopped by max_states = 2^26
(the frontier grows ~40x per layer, so the depth bound is never reached; the stop is the reference's own max_states
rule). One step = one whole BrFS; `detail.larger_budget` times the same search once at max_states = 2^28. The other
workloads (gridworld / transport / transport_xl env pools, dedup) are reported under "workloads", each with
env-steps/s (or rows/s) and the achieved HBM bandwidth of its dominant kernel.

roofline: the dominant kernel class of the BrFS (by summed HIP-event time on the search's own stream): its
algorithmic bytes (per launch, summed) / its summed duration, against the 8 TB/s HBM peak of MI355X.
cpu_baseline: the reference's own CPU code (oracle/_ref, compiled from the reference's sources) on a bounded sample of
the same workload, on every core allotted to this job (the CPU share of one GPU: OMP_NUM_THREADS when set, else the
process's CPU affinity); `host` reports nproc, the affinity and the CPU model beside it. BrFS: ParallelBrfs with
deterministic ids; env pools: CpuEnvPool; dedup: ConcurrentStateStore (and FlatStateStore on one core).
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
METRIC = "env steps/sec + BrFS expanded states/sec on 1 GPU; % of HBM roofline"


def affinity() -> int:
    try:
        return len(os.sched_getaffinity(0))
    except AttributeError:
        return os.cpu_count() or 1


def cpu_threads() -> int:
    """The cores allotted to this job: OMP_NUM_THREADS when the launcher sets it (the host's CPU share of one GPU), else
    every core of the process's affinity."""
    try:
        n = int(os.environ.get("OMP_NUM_THREADS", "0"))
    except ValueError:
        n = 0
    return max(1, min(n, affinity()) if n > 0 else affinity())


def host_info() -> dict:
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"nproc": os.cpu_count(), "affinity": affinity(), "threads_used": cpu_threads(), "cpu_model": model,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def load_traffic(kernel: str):
    """HBM bytes per launch of a kernel, measured by rocprofv3 PMC counters (FETCH_SIZE, WRITE_SIZE, each scaled by what
    it reads for a kernel of known traffic and the same access pattern: a plain copy for streaming kernels, the
    random 8-byte loads of bench.py --random-ops for the state set's probes) and committed in
    profiles/pmc_traffic.json; None if not measured."""
    p = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        k = json.load(f).get("kernels", {}).get(kernel)
    return k.get("traffic_bytes_per_launch") if k else None


def load_traffic_copy_scaled(kernel: str):
    """The same kernel's traffic with every FETCH_SIZE byte scaled by the plain copy's factor (an upper bound for the
    probes, whose random reads the copy's 128-byte streaming requests overstate); None if not measured."""
    p = os.path.join(ROOT, "profiles", "pmc_traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        k = json.load(f).get("kernels", {}).get(kernel)
    return k.get("traffic_upper_bytes_per_launch", k.get("traffic_bytes_per_launch")) if k else None


def load_bound(kernel: str):
    """The counter evidence of what bounds a kernel, committed in profiles/pmc_bounds.json (from rocprofv3 PMC runs of
    this bench): for the state set's probes the share of the measured random-access capacity their reads and atomics
    use, for the env steps the share of the VALU issue slots; None if not measured."""
    p = os.path.join(ROOT, "profiles", "pmc_bounds.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f).get("kernels", {}).get(kernel)


def bench_strips(steps: int, warmup: int, cpu: bool, larger: bool = True):
    import torch

    from mymyr_amd import search, workloads
    from mymyr_amd.task import Task

    w = workloads.STRIPS
    path = workloads.task_file("strips", os.path.join(ROOT, "tests", "golden", "tasks"))
    t = Task.from_text_file(path, w.atoms)
    kw = dict(max_depth=w.max_depth, max_states=w.max_states, stop_at_goal=False)
    for _ in range(warmup):
        search.brfs(t, **kw)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    results = [search.brfs(t, timings=True, **kw) for _ in range(steps)]
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    r = results[0]
    expanded = sum(x.expanded for x in results)
    value = expanded / wall
    # the dominant kernel class over the timed region
    classes = ["count", "emit", "insert", "rank", "compact", "other"]
    ms = {c: sum(x.kernels[c]["ms"] for x in results) for c in classes}
    by = {c: sum(x.kernels[c]["bytes"] for x in results) for c in classes}
    launches = {c: sum(x.kernels[c]["launches"] for x in results) for c in classes}
    dom = max(classes, key=lambda c: ms[c])
    achieved = by[dom] / (ms[dom] * 1e-3) / 1e9 if ms[dom] > 0 else 0.0
    traffic = load_traffic(f"brfs_{dom}")
    roofline = {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": round(achieved / HBM_PEAK_GBS, 4), "traffic": traffic,
                "traffic_copy_scaled": load_traffic_copy_scaled(f"brfs_{dom}"), "kernel": f"brfs {dom}",
                "bytes_per_launch": int(by[dom] / max(1, launches[dom])), "ms_per_launch": round(ms[dom] / max(1, launches[dom]), 4),
                "bound_evidence": load_bound(f"brfs_{dom}")}
    out = {
        "value": value, "unit": "expanded states/s", "ms_per_step": wall * 1e3 / steps, "roofline": roofline,
        "detail": {"states": r.states, "expanded": r.expanded, "generated": r.generated, "layers": r.layers, "status": r.status,
                   "layer_counts": r.layer_counts, "generated_per_s": sum(x.generated for x in results) / wall,
                   "kernel_ms_per_step": {c: round(ms[c] / steps, 3) for c in classes},
                   "kernel_gbs": {c: round(by[c] / (ms[c] * 1e-3) / 1e9, 1) if ms[c] else None for c in classes},
                   "whole_search_gbs": round(sum(by.values()) / wall / 1e9, 1),
                   "search_ms": round(sum(x.search_s for x in results) * 1e3 / steps, 3),
                   "device_ms": round(sum(x.device_s for x in results) * 1e3 / steps, 3)},
    }
    # the same search at four times the budget (max_states 2^28: a 4 GiB table, a 16 GiB arena, the cut late in the
    # fifth layer), one untimed and one timed search: how the rate holds as the table outgrows the caches' reach
    if not larger:
        if cpu:
            out["cpu_baseline"] = cpu_strips(path, w)
        return out
    big = dict(kw, max_states=w.max_states << 2)
    search.brfs(t, **big)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    rb = search.brfs(t, timings=True, **big)
    torch.cuda.synchronize()
    wb = time.perf_counter() - t0
    out["detail"]["larger_budget"] = {
        "max_states": big["max_states"], "ms": round(wb * 1e3, 2), "expanded_per_s": rb.expanded / wb,
        "generated_per_s": rb.generated / wb, "expanded": rb.expanded, "generated": rb.generated, "states": rb.states,
        "layer_counts": rb.layer_counts, "kernel_ms": {c: round(rb.kernels[c]["ms"], 3) for c in classes},
        "insert_candidates_per_s": rb.generated / (rb.kernels["insert"]["ms"] * 1e-3)}
    if cpu:
        out["cpu_baseline"] = cpu_strips(path, w)
    return out


def cpu_strips(path, w):
    from oracle import ref

    if not ref.available():
        return None
    T = cpu_threads()
    rt = ref.RefTask(path, w.atoms)
    sample = 1 << 22
    r = ref.brfs(rt, threads=T, max_depth=w.max_depth, max_states=sample, stop_at_goal=False, fingerprint=False)
    return {"value": r["expanded"] / r["seconds"], "unit": "expanded states/s", "cores": T, "kind": "reference",
            "sample": f"reference ParallelBrfs (deterministic ids) on the strips task, depth 12, max_states 2^22: "
                      f"{r['expanded']} expanded, {r['generated']} generated in {r['seconds']:.2f} s", "host": host_info()}


def bench_env(name: str, steps: int, warmup: int, cpu: bool, num_envs: int | None = None):
    import numpy as np
    import torch

    from mymyr_amd import rl, workloads
    from mymyr_amd.task import Task

    w = {"gridworld": workloads.GRIDWORLD, "transport": workloads.TRANSPORT, "transport_xl": workloads.TRANSPORT_XL}[name]
    path = workloads.task_file(name, os.path.join(ROOT, "tests", "golden", "tasks"))
    t = Task.from_text_file(path, w.atoms)
    N = num_envs or w.num_envs
    # the encoding's width: the task's true-atom count per state (transport: one position per truck and package; every
    # state of the task holds the initial state's count)
    encode = int(np.unpackbits(t.initial_state().view(np.uint8)).sum()) if w.encode else 0
    pool = rl.DeviceEnvPool(t, N, **w.env)
    pool.reset()
    for _ in range(warmup):
        pool.step(encode=encode, labels=False)
    # the rate: the workload's whole horizon from reset, back-to-back steps, synchronized on both sides
    pool.reset()
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for _ in range(steps):
        pool.step(encode=encode, labels=False)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    # the step kernel's duration: HIP events around each of the same number of further steps (the event records add
    # their own gaps, so these steps are not part of the rate)
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for a, b in evs:
        a.record()
        pool.step(encode=encode, labels=False)
        b.record()
    torch.cuda.synchronize()
    pool.check()
    kms = sum(a.elapsed_time(b) for a, b in evs) / steps
    R = t.words * 8
    per_step = 2 * R + 36 + (encode * 4 + t.num_schemas if encode else 0)
    achieved = per_step * N / (kms * 1e-3) / 1e9
    out = {"env_steps_per_s": N * steps / wall, "num_envs": N, "steps_timed": steps, "ms_per_step": wall * 1e3 / steps,
           "timed": f"the whole horizon from reset: {steps} steps of {N} envs", "words": t.words,
           "bytes_per_env_step": per_step, "encode_atoms": encode,
           "roofline": {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(achieved / HBM_PEAK_GBS, 4), "kernel": "env step", "ms_per_launch": round(kms, 4),
                        "traffic": load_traffic(f"env_{name}"), "bound_evidence": load_bound(f"env_{name}")}}
    if cpu:
        out["cpu_baseline"] = cpu_env(path, w)
    return out


def cpu_env(path, w):
    from oracle import ref

    if not ref.available():
        return None
    T = cpu_threads()
    rt = ref.RefTask(path, w.atoms)
    n, k = {"gridworld": (1024, 256), "transport": (16384, 16), "transport_xl": (4096, 4)}[w.name]
    secs, _ = ref.pool_run(rt, n, T, k, **w.env)
    return {"value": n * k / secs, "unit": "env steps/s", "cores": T, "kind": "reference",
            "sample": f"reference CpuEnvPool, {n} envs x {k} steps, {T} worker threads", "host": host_info()}


def bench_dedup(steps: int, warmup: int, cpu: bool):
    import torch

    from mymyr_amd import gen, hip, workloads

    total, batch, words = workloads.DEDUP_ROWS, workloads.DEDUP_BATCH, workloads.DEDUP_WORDS
    rows = hip.dedup_rows(0, total, words, seed=workloads.SEED, dup=workloads.DEDUP_DUP)
    times = []
    unique = 0
    for it in range(warmup + steps):
        s = hip.StateSet(total, words, 0.5, batch=batch)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for b in range(0, total, batch):
            s.insert(rows[b: b + batch], want_ids=False, count=False)
        unique = len(s)
        torch.cuda.synchronize()
        if it >= warmup:
            times.append(time.perf_counter() - t0)
        del s
    wall = sum(times) / len(times)
    R = words * 8
    alg = total * (R + 8) + unique * (R + 8) + (total - unique) * R
    nb = total // batch
    out = {"rows_per_s": total / wall, "unique": unique, "rows": total, "ms_per_step": wall * 1e3,
           "roofline": {"bound": "hbm", "achieved": round(alg / wall / 1e9, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
                        "frac": round(alg / wall / 1e9 / HBM_PEAK_GBS, 4),
                        "kernel": "state-set batch insert (probe, winner scan, compaction) per 2^20-row batch",
                        "bytes_per_launch": int(alg / nb), "ms_per_launch": round(wall * 1e3 / nb, 4),
                        "traffic": load_traffic("dedup_batch"), "bound_evidence": load_bound("dedup_probe")}}
    if cpu:
        out["cpu_baseline"] = cpu_dedup(words)
    return out


def cpu_dedup(words: int):
    """The reference's concurrent store (the store of its multi-threaded searches) on the workload's first 2^23 rows in
    2^20-row batches, on the job's cores; the single-threaded flat store on the first 2^21 rows beside it."""
    from mymyr_amd import gen, workloads
    from oracle import ref

    if not ref.available():
        return None
    T = cpu_threads()
    sample = 1 << 23
    rows = gen.dedup_rows(0, sample, words, seed=workloads.SEED, dup=workloads.DEDUP_DUP)
    unique, secs = ref.dedup_concurrent(rows, T, workloads.DEDUP_BATCH)
    flat_n = 1 << 21
    flat_unique, flat_secs = ref.dedup_flat(rows[:flat_n])
    return {"value": sample / secs, "unit": "rows/s", "cores": T, "kind": "reference",
            "sample": f"reference ConcurrentStateStore, the dedup stream's first {sample} rows of {words} words in 2^20-row "
                      f"batches on {T} threads: {unique} unique in {secs:.3f} s; reference FlatStateStore on one core, "
                      f"first {flat_n} rows: {flat_n / flat_secs:.4g} rows/s", "host": host_info()}


def copy_calibration(steps: int):
    """A plain device copy of a known size (1 GiB read, 1 GiB written per launch): the PMC counters FETCH_SIZE and
    WRITE_SIZE read on it give the scale factor between counter units and bytes."""
    import torch

    n = 1 << 28
    x = torch.ones(n, dtype=torch.int32, device="cuda")
    y = torch.empty_like(x)
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record()
    for _ in range(steps):
        y.copy_(x)
    b.record()
    torch.cuda.synchronize()
    ms = a.elapsed_time(b) / steps
    print(json.dumps({"copy_bytes_read": n * 4, "copy_bytes_written": n * 4, "ms_per_launch": ms,
                      "gbs": 2 * n * 4 / (ms * 1e-3) / 1e9}))


def random_ops(steps: int):
    """The random 8-byte operation rates that bound the state set's probes (mya_random_ops): loads, compare-and-swaps,
    atomic mins and stores at seeded random addresses of a 1 GiB table (in HBM), of a 256 MiB one (the Infinity Cache's
    size) and of 4 GiB and 16 GiB ones (the strips search's table and arena at 2^28 states), 2^28 operations each,
    HIP-event timed; one JSON line."""
    import torch

    from mymyr_amd._lib import check, lib

    n = 1 << 28
    sink = torch.empty(1 << 20, dtype=torch.int64, device="cuda")
    out = {}
    for label, words in (("1 GiB", 1 << 27), ("256 MiB", 1 << 25), ("4 GiB", 1 << 29), ("16 GiB", 1 << 31)):
        table = torch.zeros(words, dtype=torch.int64, device="cuda")
        rates = {}
        for kind, name in enumerate(("load", "cas", "atomic_min", "store")):
            best = None
            for it in range(steps + 1):
                a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                a.record()
                check(lib.mya_random_ops(table.data_ptr(), words, n, kind, 12345 + it, sink.data_ptr(),
                                         torch.cuda.current_stream().cuda_stream))
                b.record()
                torch.cuda.synchronize()
                if it:
                    ms = a.elapsed_time(b)
                    best = ms if best is None else min(best, ms)
            rates[name] = round(n / (best * 1e-3) / 1e9, 2)
        out[label] = rates
        del table
    print(json.dumps({"metric": "random 8-byte operations per second (G/s), 2^28 per launch, 4 in flight per thread",
                      "threads": 1 << 20, "random_ops": out}))


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=3)
    ap.add_argument("--warmup", type=int, default=1)
    ap.add_argument("--only", default="")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-larger-budget", action="store_true",
                    help="leave out the strips search at max_states 2^28 (profiles of the headline search alone)")
    ap.add_argument("--copy-calibration", action="store_true",
                    help="run only a 1 GiB device copy (the reference kernel for scaling PMC byte counters)")
    ap.add_argument("--random-ops", action="store_true",
                    help="run only the random 8-byte load / CAS / atomic-min / store rates (the state set's ceilings)")
    a = ap.parse_args()
    if a.gpus != 1:
        print(f"bench.py: this build runs on one GPU only (asked for {a.gpus}); the env pool shards by env range and the "
              f"BrFS by state-hash owner, but no multi-GPU path is built", file=sys.stderr)
        sys.exit(2)
    import torch

    if not torch.cuda.is_available():
        print("bench.py: no HIP device", file=sys.stderr)
        sys.exit(1)
    torch.cuda.set_device(0)
    if a.copy_calibration:
        copy_calibration(max(1, a.steps))
        return
    if a.random_ops:
        random_ops(max(1, a.steps))
        return
    only = set(x for x in a.only.split(",") if x)
    cpu = not a.no_cpu
    steps, warmup = max(1, a.steps), max(0, a.warmup)
    head = bench_strips(steps, warmup, cpu, not a.no_larger_budget) if (not only or "strips" in only) else None
    wl = {}
    # each env workload over its stated horizon (gridworld 256, transport 512, transport_xl 128 steps) from reset
    from mymyr_amd import workloads

    for name, w, wu in (("gridworld", workloads.GRIDWORLD, 16), ("transport", workloads.TRANSPORT, 4),
                        ("transport_xl", workloads.TRANSPORT_XL, 1)):
        if not only or name in only:
            wl[name] = bench_env(name, w.steps, wu, cpu)
    if not only or "dedup" in only:
        wl["dedup"] = bench_dedup(steps, min(warmup, 1), cpu)
    line = {
        "metric": METRIC,
        "value": head["value"] if head else None,
        "unit": head["unit"] if head else "expanded states/s",
        "n_gpus": 1, "steps": steps, "warmup": warmup,
        "ms_per_step": head["ms_per_step"] if head else None,
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None, "dtype": "u64", "data": "synthetic",
        "config": {"workload": "strips: random ground STRIPS (512 fluents, 4096 actions, seed 0), BrFS from the initial "
                               "state, max_depth 12, max_states 2^26, witness pruning on, dense atoms",
                   "parallelism": "single GPU"},
        "roofline": head["roofline"] if head else None,
        "cpu_baseline": head.get("cpu_baseline") if head else None,
        "detail": head["detail"] if head else None,
        "workloads": wl,
    }
    print(json.dumps(line))


if __name__ == "__main__":
    main()
