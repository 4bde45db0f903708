"""The five benchmark workloads of the state-expansion path, by name, with their sizes:

  gridworld    one agent on a 32x32 grid (20% blocked), env pool of 1024 envs x 256 steps, reward -1 per step
  strips       random ground STRIPS (512 fluents, 4096 actions), BrFS from the initial state, depth 12,
               dense atoms; the frontier explodes, so the BrFS stops at max_states (the reference's own rule)
  transport    typed transport (64 locations, 16 trucks, 128 packages), env pool of 65536 envs x 512 steps
  dedup        2^26 rows of 1024 bits, ~30% exact duplicates, inserted in 2^20-row batches at load 0.5
  transport_xl transport with 128 locations, 32 trucks, 512 packages, env pool of 262144 envs x 128 steps, with the
               per-env true-atom index tensor (int32, -1 padded) and schema masks emitted every step
"""

from __future__ import annotations

import os
from dataclasses import dataclass, field

from . import gen

SEED = 0


@dataclass(frozen=True)
class EnvWorkload:
    name: str
    num_envs: int
    steps: int
    env: dict = field(default_factory=dict)  # DeviceEnvPool / HostEnv keyword arguments
    atoms: str = "auto"
    encode: bool = False  # emit the true-atom index tensor and schema masks per step

    def text(self) -> str:
        return TASKS[self.name]()


@dataclass(frozen=True)
class BrfsWorkload:
    name: str
    max_depth: int
    max_states: int
    atoms: str = "dense"

    def text(self) -> str:
        return TASKS[self.name]()


TASKS = {
    "gridworld": lambda: gen.gridworld(32, 32, 0.2, seed=SEED),
    "strips": lambda: gen.random_strips(512, 4096, seed=SEED),
    "transport": lambda: gen.transport(64, 16, 128, goals=32, seed=SEED),
    "transport_xl": lambda: gen.transport(128, 32, 512, goals=32, seed=SEED),
}

# task tables: several instances of one domain (different sizes, so different row widths), stepped in one batch with a
# per-row instance
TABLES = {
    "gridworld_table": [lambda: gen.gridworld(6, 6, 0.2, seed=1), lambda: gen.gridworld(12, 10, 0.2, seed=2),
                        lambda: gen.gridworld(16, 16, 0.15, seed=3)],
    "transport_table": [lambda: gen.transport(8, 2, 4, goals=3, seed=1), lambda: gen.transport(24, 6, 40, goals=6, seed=2),
                        lambda: gen.transport(6, 2, 3, goals=2, seed=3)],
    # more instances than one launch per instance serves: grids of 4x4 to 13x13 cells (rows of 1 to 3 words)
    "gridworld_many": [(lambda w: (lambda: gen.gridworld(w, w - i % 3, 0.15, seed=10 + i)))(4 + (i * 7) % 10) for i in range(20)],
}
# a suite of two domains: gridworld and transport instances interleaved (global ids in this order)
TABLES["mixed_suite"] = [TABLES["gridworld_table"][0], TABLES["transport_table"][0], TABLES["gridworld_table"][1],
                         TABLES["transport_table"][2], TABLES["gridworld_table"][2]]

GRIDWORLD = EnvWorkload("gridworld", 1024, 256, {"seed": SEED, "step_reward": -1.0, "goal_reward": 0.0})
TRANSPORT = EnvWorkload("transport", 65536, 512, {"seed": SEED})
TRANSPORT_XL = EnvWorkload("transport_xl", 262144, 128, {"seed": SEED}, encode=True)
STRIPS = BrfsWorkload("strips", 12, 1 << 26)
DEDUP_ROWS = 1 << 26
DEDUP_BATCH = 1 << 20
DEDUP_WORDS = 16
DEDUP_DUP = 0.3


def _write_once(path: str, text) -> str:
    if not os.path.exists(path):
        os.makedirs(os.path.dirname(path), exist_ok=True)
        with open(path + ".tmp", "w") as f:
            f.write(text())
        os.replace(path + ".tmp", path)
    return path


def task_file(name: str, directory: str) -> str:
    """Writes the workload's task text to directory/name.txt (once) and returns the path."""
    return _write_once(os.path.join(directory, f"{name}.txt"), TASKS[name])


def table_files(name: str, directory: str) -> list[str]:
    """Writes the instances of task table `name` to directory/name_<i>.txt (once) and returns the paths."""
    return [_write_once(os.path.join(directory, f"{name}_{i}.txt"), t) for i, t in enumerate(TABLES[name])]
