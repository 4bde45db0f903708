"""Device operations on torch tensors (torch-ROCm supplies device memory and the current stream):

  hash_rows(states)        the public state hash of each row (reference: mymyr.cuda hash_rows,
                           python/src/cuda_bindings.cpp:1289-1320)
  StateSet                 the device dedup set (reference: include/mymyr/cuda/state_set.hpp); StateSet.rows()
                           exports the stored rows over DLPack
"""

from __future__ import annotations

import ctypes

import torch

from . import _lib
from ._lib import check, lib


def _stream() -> int:
    return _lib.current_stream()


def _require(t: torch.Tensor, name: str, dtype=None, ndim=None) -> None:
    if not t.is_cuda:
        raise ValueError(f"mymyr_amd: {name} must be a device tensor")
    if not t.is_contiguous():
        raise ValueError(f"mymyr_amd: {name} must be contiguous")
    if dtype is not None and t.dtype != dtype:
        raise ValueError(f"mymyr_amd: {name} must be {dtype}, got {t.dtype}")
    if ndim is not None and t.dim() != ndim:
        raise ValueError(f"mymyr_amd: {name} must have {ndim} dimensions")


def _u64(t: torch.Tensor) -> torch.Tensor:
    """uint64 rows are carried as int64 tensors (same bits)."""
    return t.view(torch.int64) if t.dtype == torch.uint64 else t


def hash_rows(states: torch.Tensor) -> torch.Tensor:
    """[rows, words] uint64/int64 device tensor -> [rows] int64 (the u64 hash bits)."""
    s = _u64(states)
    _require(s, "states", torch.int64, 2)
    out = torch.empty(s.shape[0], dtype=torch.int64, device=s.device)
    check(lib.mya_hash_rows(s.data_ptr(), s.shape[0], s.shape[1], out.data_ptr(), _stream()))
    return out


def dedup_rows(start: int, count: int, words: int = 16, seed: int = 0, dup: float = 0.3, device="cuda") -> torch.Tensor:
    """Rows [start, start + count) of the seeded dedup stream, generated on the device ([count, words] int64)."""
    out = torch.empty((count, words), dtype=torch.int64, device=device)
    check(lib.mya_dedup_rows(start, count, words, seed, dup, out.data_ptr(), _stream()))
    return out


class StateSet:
    """Device-resident open-addressing state set (rows of `words` u64 words)."""

    def __init__(self, max_states: int, words: int, max_load: float = 0.5, batch: int = 1 << 20):
        h = ctypes.c_void_p()
        check(lib.mya_hashset_create(max_states, words, max_load, batch, ctypes.byref(h)))
        self._h = h
        self.words = words

    def insert(self, rows: torch.Tensor, want_ids: bool = True, count: bool = True) -> tuple[int | None, torch.Tensor | None, torch.Tensor]:
        """Inserts rows; returns (new states, ids [n] int64 or None, is_new [n] uint8). With count=False the insert is
        asynchronous on torch's current stream and the first item is None (len() synchronizes and reports overflow)."""
        r = _u64(rows)
        _require(r, "rows", torch.int64, 2)
        if r.shape[1] != self.words:
            raise ValueError(f"mymyr_amd: rows of {r.shape[1]} words; the set holds {self.words}")
        n = r.shape[0]
        ids = torch.empty(n, dtype=torch.int64, device=r.device) if want_ids else None
        is_new = torch.empty(n, dtype=torch.uint8, device=r.device)
        cnt = ctypes.c_uint64()
        check(lib.mya_hashset_insert(self._h, r.data_ptr(), n, None if ids is None else ids.data_ptr(), is_new.data_ptr(),
                                     ctypes.byref(cnt) if count else None, _stream()))
        return (cnt.value if count else None), ids, is_new

    def __len__(self) -> int:
        s = ctypes.c_uint64()
        check(lib.mya_hashset_size(self._h, ctypes.byref(s)))
        return s.value

    def clear(self) -> None:
        check(lib.mya_hashset_clear(self._h, _stream()))

    def rows(self, read_only: bool = False):
        """The stored rows [len, words] (uint64) as a DLPack-exportable device array, without a copy:
        ``torch.from_dlpack(s.rows())``. Waits for the last insert. The export holds the set's memory until the consumer
        drops it; a later clear() makes its contents undefined."""
        from .dlpack import DeviceArray
        flags = 1 if read_only else 0
        n = len(self)

        def export(consumer: int, versioned: int, out: ctypes.c_void_p) -> int:
            return lib.mya_hashset_export_rows(self._h, flags, consumer, versioned, ctypes.byref(out))

        return DeviceArray(export, torch.cuda.current_device(), (n, self.words), "uint64", owner=self)

    def __del__(self):
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib.mya_hashset_free(h)
            self._h = ctypes.c_void_p()
