"""Task loading: the reference's ``Task.from_text_file`` / ``Task.create`` entry points over the C ABI
(reference: include/mymyr/task/task.hpp:166-167, python/mymyr task construction).
"""

from __future__ import annotations

import ctypes

import numpy as np

from . import _lib
from ._lib import check, lib

ATOMS = {"auto": 0, "reachable": 1, "dense": 2, "lazy": 3}
MODES = {0: "reachable", 1: "dense", 2: "lazy"}


class Task:
    """A compiled planning task (host tables plus the device image, uploaded on first device use).

    With ``atoms="lazy"`` the slots start with the initial state's atoms and grow as device searches and expansions
    meet new ones (in ascending canonical id per device launch), so ``words``, ``fluent_slots`` and the slot records
    are read anew on each access."""

    def __init__(self, handle: int, source: str):
        self._h = ctypes.c_void_p(handle)
        self.source = source
        info = self._info()
        self.atom_mode = MODES[info.atom_mode]
        self.num_schemas = info.num_schemas
        self.label_width = info.label_width
        self.num_objects = info.num_objects
        self.max_arity = info.max_arity
        self.dense_fluent = info.dense_fluent
        self.reachable_fluent = info.reachable_fluent
        self.view_words = info.view_words

    def _info(self) -> "_lib.TaskInfo":
        info = _lib.TaskInfo()
        check(lib.mya_task_info_get(self._h, ctypes.byref(info)))
        return info

    @property
    def words(self) -> int:
        """State words (lazy slots: the current width)."""
        return self._info().words

    @property
    def fluent_slots(self) -> int:
        """Assigned atom slots."""
        return self._info().fluent_slots

    @property
    def goal_unsatisfiable(self) -> bool:
        """No state is a goal under the current slots."""
        return bool(self._info().goal_unsat)

    @property
    def frozen(self) -> bool:
        """Whether the slot table is fixed (every mode but lazy)."""
        return self.atom_mode != "lazy"

    @classmethod
    def from_text(cls, text: str, atoms: str = "auto") -> "Task":
        h = ctypes.c_void_p()
        data = text.encode()
        check(lib.mya_task_load_text(data, len(data), ATOMS[atoms], ctypes.byref(h)))
        return cls(h.value, "<text>")

    @classmethod
    def from_text_file(cls, path: str, atoms: str = "auto") -> "Task":
        h = ctypes.c_void_p()
        check(lib.mya_task_load_file(str(path).encode(), ATOMS[atoms], ctypes.byref(h)))
        return cls(h.value, str(path))

    @property
    def handle(self) -> ctypes.c_void_p:
        return self._h

    def slot_records(self) -> tuple[np.ndarray, np.ndarray]:
        """(records [slots, 1 + max(1, max_arity)] uint32: predicate then arguments, canonical ids [slots] uint64)."""
        stride = 1 + max(1, self.max_arity)
        n = self.fluent_slots
        rec = np.zeros((n, stride), dtype=np.uint32)
        cid = np.zeros(n, dtype=np.uint64)
        check(lib.mya_task_slots(self._h, rec.ctypes.data, cid.ctypes.data))
        return rec, cid

    def initial_state(self, words: int | None = None) -> np.ndarray:
        w = self.words if words is None else words
        row = np.zeros(w, dtype=np.uint64)
        check(lib.mya_task_initial(self._h, row.ctypes.data, w))
        return row

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value and lib is not None:  # at interpreter exit the module's globals may be gone
            lib.mya_task_free(h)
            self._h = ctypes.c_void_p()
