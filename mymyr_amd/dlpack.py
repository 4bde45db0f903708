"""DLPack export of library-owned device arrays.

Python side of the reference's DLArray export (python/src/arrays.cpp:100-235, python/mymyr/_interop.py:14-27):
``DeviceBuffer`` is device memory owned by libmymyr_amd (reference-counted), ``DeviceArray`` a typed view of it or of
a state set's rows that any DLPack consumer takes without a copy (``torch.from_dlpack(a)``). The capsules carry
managed tensors built by the C ABI (``mya_buffer_export`` / ``mya_hashset_export_rows``) with device type kDLROCM;
their destructor is the library's own, so dropping an unconsumed capsule needs no Python callback.

Protocol details as the reference's ``__dlpack__``: ``stream`` None means the default stream, -1 no synchronization,
any other int a hipStream_t of the consumer (1 and 2, CUDA's legacy and per-thread default streams, do not exist on
ROCm and are refused); ``max_version`` (1, x) or later selects the versioned capsule; ``dl_device`` must be the
array's own device; ``copy=True`` is refused (copy in the consumer).
"""

from __future__ import annotations

import ctypes
from typing import Callable

from ._lib import check, lib

DL_ROCM = 10

# dtype name -> (DLPack type code, bits): int 0, uint 1, float 2, bool 6
DTYPES = {
    "int8": (0, 8), "int16": (0, 16), "int32": (0, 32), "int64": (0, 64),
    "uint8": (1, 8), "uint16": (1, 16), "uint32": (1, 32), "uint64": (1, 64),
    "float16": (2, 16), "float32": (2, 32), "float64": (2, 64),
    "bool": (6, 8),
}

FLAG_READ_ONLY = 1

_NAME_LEGACY = b"dltensor"
_NAME_VERSIONED = b"dltensor_versioned"

_capsule_new = ctypes.pythonapi.PyCapsule_New
_capsule_new.restype = ctypes.py_object
_capsule_new.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]
_DESTRUCTOR = ctypes.cast(lib.mya_dlpack_capsule_destructor, ctypes.c_void_p).value


def _torch_stream() -> int:
    import torch
    return torch.cuda.current_stream().cuda_stream


def _consumer_stream(stream) -> int:
    if stream is None:
        return 0
    if not isinstance(stream, int):
        raise TypeError("mymyr_amd: __dlpack__: stream must be an int or None")
    if stream in (1, 2):
        raise BufferError("mymyr_amd: __dlpack__: streams 1 and 2 are CUDA's default streams; on ROCm pass 0 or a "
                          "hipStream_t")
    if stream < -1:
        raise BufferError("mymyr_amd: __dlpack__: invalid stream")
    return stream


class DeviceArray:
    """A typed device array that exports itself over DLPack (``__dlpack__`` / ``__dlpack_device__``)."""

    def __init__(self, export: Callable[[int, int, ctypes.c_void_p], int], device: int, shape: tuple, dtype: str,
                 owner=None):
        self._export = export
        self._device = device
        self.shape = tuple(shape)
        self.dtype = dtype
        self._owner = owner  # keeps the Python handle of the buffer or set alive while the view exists

    def __dlpack_device__(self) -> tuple[int, int]:
        return (DL_ROCM, self._device)

    def __dlpack__(self, *, stream=None, max_version=None, dl_device=None, copy=None):
        consumer = _consumer_stream(stream)
        if dl_device is not None and tuple(dl_device) != self.__dlpack_device__():
            raise BufferError("mymyr_amd: __dlpack__: only the array's own device is supported")
        if copy:
            raise BufferError("mymyr_amd: __dlpack__: copy=True is not supported for device arrays (copy in the consumer)")
        versioned = max_version is not None and len(max_version) >= 1 and max_version[0] >= 1
        out = ctypes.c_void_p()
        check(self._export(consumer, int(versioned), out))
        return _capsule_new(out, _NAME_VERSIONED if versioned else _NAME_LEGACY, _DESTRUCTOR)


class DeviceBuffer:
    """Device memory owned by the library on the current device (contents start undefined)."""

    def __init__(self, nbytes: int):
        h = ctypes.c_void_p()
        check(lib.mya_buffer_create(int(nbytes), ctypes.byref(h)))
        self._h = h
        import torch
        self.device = torch.cuda.current_device()

    @property
    def ptr(self) -> int:
        return lib.mya_buffer_data(self._h) or 0

    @property
    def nbytes(self) -> int:
        return lib.mya_buffer_bytes(self._h)

    def array(self, dtype: str, shape, strides=None, offset: int = 0, read_only: bool = False,
              producer_stream: int | None = None) -> DeviceArray:
        """A view of the buffer: `shape` and element `strides` (None: row-major) from byte `offset`. Work queued on
        producer_stream (default: torch's current stream at export time) precedes the consumer's later work."""
        if dtype not in DTYPES:
            raise ValueError(f"mymyr_amd: unsupported dtype {dtype!r}")
        code, bits = DTYPES[dtype]
        shape = tuple(int(x) for x in shape)
        nd = len(shape)
        shape_c = (ctypes.c_int64 * max(1, nd))(*shape)
        strides_c = None if strides is None else (ctypes.c_int64 * max(1, nd))(*[int(x) for x in strides])
        flags = FLAG_READ_ONLY if read_only else 0

        def export(consumer: int, versioned: int, out: ctypes.c_void_p) -> int:
            producer = _torch_stream() if producer_stream is None else producer_stream
            return lib.mya_buffer_export(self._h, offset, code, bits, nd, shape_c, strides_c, flags, producer, consumer,
                                         versioned, ctypes.byref(out))

        return DeviceArray(export, self.device, shape, dtype, owner=self)

    def release(self) -> None:
        """Drops this handle's reference (exported tensors keep the memory until their deleters run)."""
        h = getattr(self, "_h", None)
        if h is not None and h.value:
            lib.mya_buffer_release(h)
            self._h = ctypes.c_void_p()

    def __del__(self):
        self.release()
