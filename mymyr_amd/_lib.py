"""ctypes binding of libmymyr_amd.so (the C ABI declared in include/mymyr_amd.h).

The library is built in-tree (``make -C mymyr_amd``); importing this module without it raises ImportError, so no
caller can silently run without the HIP path.
"""

from __future__ import annotations

import ctypes
import os
from ctypes import POINTER, Structure, c_char_p, c_double, c_int, c_int32, c_int64, c_size_t, c_uint8, c_uint32, c_uint64, c_void_p

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmymyr_amd.so")
ABI_VERSION = 20  # MYA_ABI_VERSION of include/mymyr_amd.h


class MyaError(RuntimeError):
    """A failed mymyr_amd call; the message is the library's mya_last_error()."""


class TaskInfo(Structure):
    _fields_ = [
        ("words", c_uint32),
        ("fluent_slots", c_uint32),
        ("atom_mode", c_uint32),
        ("num_schemas", c_uint32),
        ("label_width", c_uint32),
        ("num_objects", c_uint32),
        ("max_arity", c_uint32),
        ("goal_unsat", c_uint32),
        ("dense_fluent", c_uint64),
        ("reachable_fluent", c_uint64),
        ("view_words", c_uint32),
        ("reserved", c_uint32),
    ]


class EnvConfig(Structure):
    _fields_ = [
        ("seed", c_uint64),
        ("max_steps", c_uint32),
        ("step_reward", ctypes.c_float),
        ("goal_reward", ctypes.c_float),
        ("dead_end_reward", ctypes.c_float),
        ("dead_end", c_int32),
        ("dead_end_terminal", c_int32),
        ("autoreset", c_int32),
        ("canonical_order", c_int32),
        ("witness_pruning", c_int32),
        ("reserved", c_int32),
    ]


class EnvBatch(Structure):
    _fields_ = [
        ("states", c_void_p),
        ("rows", c_uint64),
        ("words", c_uint32),
        ("reserved", c_uint32),
        ("steps", c_void_p),
        ("draws", c_void_p),
        ("at_goal", c_void_p),
        ("first_env", c_uint64),
        ("counts", c_void_p),
        ("goal_pos", c_void_p),
        ("goal_neg", c_void_p),
        ("task_ids", c_void_p),
        ("seeds", c_void_p),
        ("env_ids", c_void_p),
        ("reset_counts", c_void_p),
        ("sampling_seeds", c_void_p),
        ("visited", c_void_p),
        ("visited_count", c_void_p),
        ("visited_status", c_void_p),
        ("visited_capacity", c_uint32),
        ("visited_status_per_row", c_int32),
    ]


class StepOutputs(Structure):
    _fields_ = [
        ("reward", c_void_p),
        ("terminated", c_void_p),
        ("truncated", c_void_p),
        ("count", c_void_p),
        ("final_states", c_void_p),
        ("schema", c_void_p),
        ("binding", c_void_p),
        ("label_width", c_uint32),
        ("final_words", c_uint32),
        ("invalid", c_void_p),
        ("goal", c_void_p),
        ("atoms", c_void_p),
        ("masks", c_void_p),
        ("max_atoms", c_uint32),
        ("reserved", c_uint32),
        ("revisited", c_void_p),
    ]


# BrfsOptions::layers' scorer: (user, rows [n, words], n, words, scores [n])
LAYER_SCORER = ctypes.CFUNCTYPE(None, c_void_p, POINTER(c_uint64), c_uint64, c_uint32, POINTER(c_double))
GOAL_TEST = ctypes.CFUNCTYPE(ctypes.c_int32, c_void_p, POINTER(c_uint64), c_uint64, c_uint32, POINTER(ctypes.c_uint8))


class BrfsOptions(Structure):
    _fields_ = [
        ("max_depth", c_uint32),
        ("witness_pruning", c_int32),
        ("max_states", c_uint64),
        ("max_expanded", c_uint64),
        ("stop_at_goal", c_int32),
        ("fingerprint", c_int32),
        ("chunk", c_uint64),
        ("memory_states", c_uint64),
        ("timings", c_int32),
        ("reserved", c_int32),
        ("start", c_void_p),
        ("blocked", c_void_p),
        ("blocked_count", c_uint64),
        ("words", c_uint32),
        ("timed", c_int32),
        ("max_seconds", c_double),
        ("cancel", c_void_p),
        ("goal_kind", c_int32),
        ("goal_count", c_uint32),
        ("goal_offsets", c_void_p),
        ("goal_literals", c_void_p),
        ("observer", c_void_p),
        ("progress_interval", c_uint64),
        ("layer_kind", c_int32),
        ("prefer_fewer_satisfied_goals", c_int32),
        ("layer_seed", c_uint64),
        ("max_next_layer_states", c_uint32),
        ("beam_width", c_uint32),
        ("randomize_ties", c_int32),
        ("beam_novelty", c_int32),
        ("layer_scorer", LAYER_SCORER),
        ("layer_scorer_user", c_void_p),
        ("goal_test", GOAL_TEST),
        ("goal_test_user", c_void_p),
    ]


GOAL_LITERAL_INTS = 9  # MYA_GOAL_LITERAL_INTS


class SearchStatistics(Structure):
    _fields_ = [("expanded", c_uint64), ("generated", c_uint64), ("states", c_uint64), ("pruned", c_uint64),
                ("seconds", c_double), ("memory_bytes", c_uint64)]


ON_START = ctypes.CFUNCTYPE(None, c_void_p, ctypes.POINTER(c_uint64), c_uint32)
ON_PASS = ctypes.CFUNCTYPE(None, c_void_p, c_uint32, ctypes.POINTER(SearchStatistics))
ON_PROGRESS = ctypes.CFUNCTYPE(c_int32, c_void_p, ctypes.POINTER(SearchStatistics))
ON_SOLUTION = ctypes.CFUNCTYPE(None, c_void_p, ctypes.POINTER(c_int32), ctypes.POINTER(c_int32), c_uint32, c_uint32, c_double)
ON_END = ctypes.CFUNCTYPE(None, c_void_p, c_int32, ctypes.POINTER(SearchStatistics))
ON_EXPAND = ctypes.CFUNCTYPE(None, c_void_p, c_uint64, ctypes.POINTER(c_uint64), c_uint32)
ON_GENERATE = ctypes.CFUNCTYPE(None, c_void_p, c_uint64, c_int32, ctypes.POINTER(c_int32), c_uint32, c_uint64, ctypes.POINTER(c_uint64),
                               c_uint32, c_int32)
ON_PRUNE = ctypes.CFUNCTYPE(None, c_void_p, c_uint64, c_int32, ctypes.POINTER(c_int32), c_uint32, ctypes.POINTER(c_uint64), c_uint32)


class SearchObserver(Structure):
    _fields_ = [("user", c_void_p), ("on_start", ON_START), ("on_pass", ON_PASS), ("on_progress", ON_PROGRESS),
                ("on_solution", ON_SOLUTION), ("on_end", ON_END), ("on_expand", ON_EXPAND), ("on_generate", ON_GENERATE),
                ("on_prune", ON_PRUNE)]


class BrfsResult(Structure):
    _fields_ = [
        ("status", c_int32),
        ("solved", c_int32),
        ("exhausted", c_int32),
        ("layers", c_uint32),
        ("states", c_uint64),
        ("expanded", c_uint64),
        ("generated", c_uint64),
        ("goal_states", c_uint64),
        ("fingerprint", c_uint64),
        ("first_goal", c_int64),
        ("search_s", c_double),
        ("device_s", c_double),
        ("kernel_ms", c_double * 8),
        ("kernel_bytes", c_uint64 * 8),
        ("kernel_launches", c_uint64 * 8),
        ("pruned", c_uint64),
        ("memory_bytes", c_uint64),
        ("words", c_uint32),
        ("fluent_slots", c_uint32),
        ("threads_used", c_uint32),
        ("reserved2", c_uint32),
        ("store", ctypes.c_char * 16),
        ("message", ctypes.c_char * 256),
    ]


class BrfsPlan(Structure):
    _fields_ = [
        ("schema", c_void_p),
        ("binding", c_void_p),
        ("cap", c_uint32),
        ("label_width", c_uint32),
        ("goal_state", c_void_p),
        ("goal_cap", c_uint32),
        ("length", c_uint32),
        ("goal_words", c_uint32),
        ("reserved", c_uint32),
        ("cost", c_double),
    ]


class MemoryUsage(Structure):
    _fields_ = [
        ("reserved", c_uint64),
        ("used", c_uint64),
        ("reserved_high", c_uint64),
        ("used_high", c_uint64),
        ("allocations", c_uint64),
        ("driver_allocations", c_uint64),
    ]


def memory_usage() -> dict:
    """The library's device memory figures (mya_memory_usage_get): reserved / used bytes, their high-water marks, and
    the blocks handed out and taken from the driver so far."""
    u = MemoryUsage()
    check(lib.mya_memory_usage_get(ctypes.byref(u)))
    return {k: int(getattr(u, k)) for k, _ in MemoryUsage._fields_}


class ExpandOptions(Structure):
    _fields_ = [
        ("canonical_order", c_int32),
        ("witness_pruning", c_int32),
        ("validate", c_int32),
        ("drop_noops", c_int32),
    ]


class Expansion(Structure):
    _fields_ = [
        ("capacity", c_uint64),
        ("words", c_uint32),
        ("label_width", c_uint32),
        ("succ", c_void_p),
        ("parent", c_void_p),
        ("schema", c_void_p),
        ("binding", c_void_p),
        ("goal", c_void_p),
        ("offsets", c_void_p),
        ("succ_hash", c_void_p),
        ("noop", c_void_p),
        ("index", c_void_p),
        ("generated", c_uint64),
        ("total", c_uint64),
        ("words_needed", c_uint32),
        ("reserved", c_uint32),
    ]


class PaddedExpansion(Structure):
    _fields_ = [
        ("k", c_uint32),
        ("words", c_uint32),
        ("label_width", c_uint32),
        ("reserved", c_uint32),
        ("index", c_void_p),
        ("mask", c_void_p),
        ("count", c_void_p),
        ("succ", c_void_p),
        ("schema", c_void_p),
        ("binding", c_void_p),
        ("goal", c_void_p),
        ("succ_hash", c_void_p),
        ("noop", c_void_p),
        ("canonical", c_void_p),
        ("overflow", c_int32),
        ("reserved2", c_int32),
    ]


def current_stream() -> int:
    """torch's current HIP stream on the current device as a raw hipStream_t: torch.cuda.current_stream().cuda_stream
    without building the Stream object (a few microseconds per call, which a per-step call would pay every step)."""
    import torch

    raw = getattr(torch._C, "_cuda_getCurrentRawStream", None)
    if raw is None:
        return torch.cuda.current_stream().cuda_stream
    return raw(torch._C._cuda_getDevice())


def _load() -> ctypes.CDLL:
    # torch-ROCm ships its own libamdhip64.so.7. Loaded first, the library would bind the system's copy and the
    # process would hold two HIP runtimes (torch's then finds no device); with torch imported first, the library
    # binds to the runtime already loaded under that soname, and both share one runtime.
    try:
        import torch  # noqa: F401
    except ImportError:
        pass
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"mymyr_amd: {LIB_PATH} is not built (run `make -C mymyr_amd` or __graft_entry__.build())")
    lib = ctypes.CDLL(LIB_PATH)
    lib.mya_abi_version.restype = c_int
    if lib.mya_abi_version() != ABI_VERSION:
        raise ImportError(f"mymyr_amd: {LIB_PATH} has ABI version {lib.mya_abi_version()}, this binding expects {ABI_VERSION} "
                          f"(rebuild with `make -C mymyr_amd`)")
    sigs = {
        "mya_last_error": (c_char_p, []),
        "mya_abi_version": (c_int, []),
        "mya_memory_usage_get": (c_int, [POINTER(MemoryUsage)]),
        "mya_task_load_text": (c_int, [c_char_p, c_size_t, c_int, POINTER(c_void_p)]),
        "mya_task_load_file": (c_int, [c_char_p, c_int, POINTER(c_void_p)]),
        "mya_task_free": (None, [c_void_p]),
        "mya_task_info_get": (c_int, [c_void_p, POINTER(TaskInfo)]),
        "mya_task_slots": (c_int, [c_void_p, c_void_p, c_void_p]),
        "mya_task_initial": (c_int, [c_void_p, c_void_p, c_uint32]),
        "mya_hash_rows": (c_int, [c_void_p, c_uint64, c_uint32, c_void_p, c_void_p]),
        "mya_hash_words": (c_uint64, [c_void_p, c_uint32, c_uint64]),
        "mya_hash_state": (c_uint64, [c_void_p, c_uint32]),
        "mya_philox": (None, [c_uint64, c_uint64, c_uint64, c_uint32, c_void_p]),
        "mya_successor_index": (c_uint32, [c_uint64, c_uint64, c_uint64, c_uint32]),
        "mya_instance_draw": (c_int32, [c_uint64, c_uint64, c_uint32, c_uint32, c_void_p, c_void_p, c_uint32]),
        "mya_hashset_create": (c_int, [c_uint64, c_uint32, c_double, c_uint64, POINTER(c_void_p)]),
        "mya_hashset_free": (None, [c_void_p]),
        "mya_hashset_insert": (c_int, [c_void_p, c_void_p, c_uint64, c_void_p, c_void_p, POINTER(c_uint64), c_void_p]),
        "mya_hashset_size": (c_int, [c_void_p, POINTER(c_uint64)]),
        "mya_hashset_rows": (c_int, [c_void_p, POINTER(c_void_p)]),
        "mya_hashset_clear": (c_int, [c_void_p, c_void_p]),
        "mya_dedup_rows": (c_int, [c_uint64, c_uint64, c_uint32, c_uint64, c_double, c_void_p, c_void_p]),
        "mya_random_ops": (c_int, [c_void_p, c_uint64, c_uint64, c_int, c_uint64, c_void_p, c_void_p]),
        "mya_buffer_create": (c_int, [c_uint64, POINTER(c_void_p)]),
        "mya_buffer_data": (c_void_p, [c_void_p]),
        "mya_buffer_bytes": (c_uint64, [c_void_p]),
        "mya_buffer_release": (None, [c_void_p]),
        "mya_buffer_export": (c_int, [c_void_p, c_uint64, c_uint8, c_uint8, c_int32, c_void_p, c_void_p, c_uint64, c_void_p,
                                      c_int64, c_int, POINTER(c_void_p)]),
        "mya_hashset_export_rows": (c_int, [c_void_p, c_uint64, c_int64, c_int, POINTER(c_void_p)]),
        "mya_dlpack_capsule_destructor": (None, [c_void_p]),
    }
    optional = {
        "mya_env_create": (c_int, [c_void_p, POINTER(EnvConfig), POINTER(c_void_p)]),
        "mya_env_create_table": (c_int, [c_void_p, c_uint32, POINTER(EnvConfig), POINTER(c_void_p)]),
        "mya_env_create_suite": (c_int, [c_void_p, c_uint32, POINTER(EnvConfig), POINTER(c_void_p)]),
        "mya_env_free": (None, [c_void_p]),
        "mya_env_reset": (c_int, [c_void_p, POINTER(EnvBatch), c_void_p, c_void_p, c_int, c_int, c_void_p]),
        "mya_env_set_sampling": (c_int, [c_void_p, c_uint32, c_void_p, c_void_p, c_uint32]),
        "mya_env_set_seed": (c_int, [c_void_p, c_uint64, c_void_p]),
        "mya_env_clear_visited": (c_int, [c_void_p, POINTER(EnvBatch), c_void_p, c_void_p]),
        "mya_env_reserve": (c_int, [c_void_p, c_uint64]),
        "mya_env_random_actions": (c_int, [c_void_p, POINTER(EnvBatch), c_void_p, c_uint32, c_void_p, c_void_p]),
        "mya_env_goal": (c_int, [c_void_p, POINTER(EnvBatch), c_void_p, c_void_p]),
        "mya_env_step": (c_int, [c_void_p, POINTER(EnvBatch), POINTER(StepOutputs), c_void_p, c_void_p, c_void_p]),
        "mya_env_step_labels": (c_int, [c_void_p, POINTER(EnvBatch), POINTER(StepOutputs), c_void_p, c_void_p, c_uint32, c_void_p,
                                        c_void_p]),
        "mya_env_check": (c_int, [c_void_p]),
        "mya_env_refresh": (c_int, [c_void_p, POINTER(EnvBatch), c_void_p, c_void_p]),
        "mya_env_initial_count": (c_int, [c_void_p, c_uint32, POINTER(c_uint32), POINTER(c_uint8)]),
        "mya_brfs": (c_int, [c_void_p, POINTER(BrfsOptions), POINTER(BrfsResult), c_void_p, c_uint32, POINTER(BrfsPlan)]),
        "mya_encode_atoms": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, c_void_p, c_uint32, c_void_p]),
        "mya_schema_masks": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, c_void_p, c_void_p]),
        "mya_expand": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, POINTER(ExpandOptions), POINTER(Expansion), c_void_p]),
        "mya_expand_noalloc": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, POINTER(ExpandOptions), POINTER(Expansion), c_void_p]),
        "mya_env_expand": (c_int, [c_void_p, c_void_p, c_void_p, c_uint64, c_uint32, POINTER(ExpandOptions), POINTER(Expansion),
                                   c_void_p]),
        "mya_visited_mask": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, c_void_p, c_void_p, c_void_p, c_uint64, c_uint64, c_void_p,
                                     c_void_p]),
        "mya_label_actions": (c_int, [c_void_p, c_void_p, c_void_p, c_uint32, c_uint64, c_void_p, c_void_p, c_uint32, c_void_p, c_void_p]),
        "mya_pad": (c_int, [POINTER(Expansion), c_uint64, POINTER(PaddedExpansion), c_void_p]),
        "mya_successors": (c_int, [c_void_p, c_void_p, c_uint64, c_uint32, c_int32, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    }
    for name, (res, args) in list(sigs.items()) + list(optional.items()):
        fn = getattr(lib, name, None)
        if fn is None:
            if name in sigs:
                raise ImportError(f"mymyr_amd: {LIB_PATH} lacks {name}")
            continue
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int) -> None:
    if rc != 0:
        raise MyaError(lib.mya_last_error().decode())
