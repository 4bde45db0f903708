"""DLPack export (the reference's DLArray export, python/src/arrays.cpp:100-235, and its tests
tests/python/test_interop.py): the exported structs have DLPack's layout (checked against the dlpack.h that torch
ships), the capsule destructor follows the DLPack Python protocol, argument errors are refused on the host, and on
the device torch takes library buffers and state-set rows without a copy."""

import ctypes
import gc
import os
import shutil
import subprocess

import numpy as np
import pytest

from mymyr_amd._lib import MyaError, lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _torch_include():
    try:
        import torch
    except ImportError:
        return None
    d = os.path.join(os.path.dirname(torch.__file__), "include")
    return d if os.path.exists(os.path.join(d, "ATen", "dlpack.h")) else None


def test_struct_layout_matches_dlpack_header(tmp_path):
    inc = _torch_include()
    if inc is None or shutil.which("gcc") is None:
        pytest.skip("no dlpack.h or gcc")
    pairs = [("mya_dl_device", "DLDevice", ["device_type", "device_id"]),
             ("mya_dl_dtype", "DLDataType", ["code", "bits", "lanes"]),
             ("mya_dl_tensor", "DLTensor", ["data", "device", "ndim", "dtype", "shape", "strides", "byte_offset"]),
             ("mya_dl_managed", "DLManagedTensor", ["dl_tensor", "manager_ctx", "deleter"]),
             ("mya_dl_version", "DLPackVersion", ["major", "minor"]),
             ("mya_dl_managed_versioned", "DLManagedTensorVersioned",
              ["version", "manager_ctx", "deleter", "flags", "dl_tensor"])]
    lines = ['#include "mymyr_amd.h"', "#include <ATen/dlpack.h>", "#include <stddef.h>"]
    for ours, theirs, fields in pairs:
        lines.append(f'_Static_assert(sizeof({ours}) == sizeof({theirs}), "{ours}");')
        for f in fields:
            lines.append(f'_Static_assert(offsetof({ours}, {f}) == offsetof({theirs}, {f}), "{ours}.{f}");')
    lines += ['_Static_assert(MYA_DL_ROCM == kDLROCM, "rocm");', '_Static_assert(MYA_DL_INT == kDLInt, "int");',
              '_Static_assert(MYA_DL_UINT == kDLUInt, "uint");', '_Static_assert(MYA_DL_FLOAT == kDLFloat, "float");',
              '_Static_assert(MYA_DL_BOOL == kDLBool, "bool");',
              '_Static_assert(MYA_DL_FLAG_READ_ONLY == DLPACK_FLAG_BITMASK_READ_ONLY, "ro");',
              '_Static_assert(MYA_DL_MAJOR == DLPACK_MAJOR_VERSION, "major");']
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines) + "\n")
    r = subprocess.run(["gcc", "-fsyntax-only", "-std=c11", "-I", os.path.join(ROOT, "include"), "-I", inc, str(src)],
                       capture_output=True, text=True)
    assert r.returncode == 0, r.stderr


class _Tensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("device_type", ctypes.c_int32), ("device_id", ctypes.c_int32),
                ("ndim", ctypes.c_int32), ("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16),
                ("shape", ctypes.c_void_p), ("strides", ctypes.c_void_p), ("byte_offset", ctypes.c_uint64)]


_DELETER = ctypes.CFUNCTYPE(None, ctypes.c_void_p)


class _ManagedV(ctypes.Structure):
    _fields_ = [("major", ctypes.c_uint32), ("minor", ctypes.c_uint32), ("ctx", ctypes.c_void_p), ("deleter", _DELETER),
                ("flags", ctypes.c_uint64), ("t", _Tensor)]


class _Managed(ctypes.Structure):
    _fields_ = [("t", _Tensor), ("ctx", ctypes.c_void_p), ("deleter", _DELETER)]


def test_capsule_destructor_follows_the_protocol():
    from mymyr_amd import dlpack

    new = ctypes.pythonapi.PyCapsule_New
    new.restype = ctypes.py_object
    new.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]
    set_name = ctypes.pythonapi.PyCapsule_SetName
    set_name.restype = ctypes.c_int
    set_name.argtypes = [ctypes.py_object, ctypes.c_char_p]
    called = []
    deleter = _DELETER(lambda p: called.append(p))
    names = [b"dltensor_versioned", b"dltensor", b"used_dltensor_versioned"]
    mv, ml = _ManagedV(), _Managed()
    mv.deleter = deleter
    ml.deleter = deleter
    # an unconsumed capsule of either kind calls its tensor's deleter when it dies
    cap = new(ctypes.addressof(mv), names[0], dlpack._DESTRUCTOR)
    del cap
    gc.collect()
    assert called == [ctypes.addressof(mv)]
    cap = new(ctypes.addressof(ml), names[1], dlpack._DESTRUCTOR)
    del cap
    gc.collect()
    assert called == [ctypes.addressof(mv), ctypes.addressof(ml)]
    # a consumer renames the capsule when it takes the tensor: then the destructor leaves it alone
    cap = new(ctypes.addressof(mv), names[0], dlpack._DESTRUCTOR)
    assert set_name(cap, names[2]) == 0
    del cap
    gc.collect()
    assert len(called) == 2


def test_export_argument_errors_on_host():
    out = ctypes.c_void_p()
    shape = (ctypes.c_int64 * 1)(4)
    assert lib.mya_buffer_export(None, 0, 1, 8, 1, shape, None, 0, None, -1, 1, ctypes.byref(out)) != 0
    assert "null argument" in lib.mya_last_error().decode()
    assert lib.mya_hashset_export_rows(None, 0, -1, 1, ctypes.byref(out)) != 0
    assert lib.mya_buffer_data(None) is None and lib.mya_buffer_bytes(None) == 0
    lib.mya_buffer_release(None)


# ---------------------------------------------------------------------------------------------------------- device


@pytest.mark.gpu
def test_buffer_round_trip_through_torch():
    import torch
    from mymyr_amd.dlpack import DeviceBuffer

    b = DeviceBuffer(4096)
    a = torch.from_dlpack(b.array("int32", (16, 64)))  # versioned capsule
    assert a.device.type == "cuda" and a.data_ptr() == b.ptr and a.shape == (16, 64) and a.dtype == torch.int32
    a.copy_(torch.arange(1024, dtype=torch.int32, device="cuda").view(16, 64))
    # a strided view from a byte offset: rows 2, 4, .. of columns 8..15
    v = torch.from_dlpack(b.array("int32", (7, 8), strides=(128, 1), offset=(2 * 64 + 8) * 4))
    assert torch.equal(v, a[2::2, 8:16][:7])
    # the legacy capsule, as older consumers take it
    cap = b.array("uint8", (4096,)).__dlpack__(stream=torch.cuda.current_stream().cuda_stream)
    u = torch.utils.dlpack.from_dlpack(cap)
    assert u.data_ptr() == b.ptr and int(u[4]) == 1  # int32 1 little-endian
    # the exports keep the memory after the creator's handle is dropped
    b.release()
    del b
    gc.collect()
    torch.cuda.synchronize()
    assert int(a[15, 63]) == 1023 and torch.equal(v[0], torch.arange(136, 144, dtype=torch.int32, device="cuda"))


@pytest.mark.gpu
def test_buffer_export_refuses_views_past_the_end():
    from mymyr_amd.dlpack import DeviceBuffer

    b = DeviceBuffer(1024)
    with pytest.raises(MyaError, match="past the buffer"):
        b.array("int64", (129,)).__dlpack__()
    with pytest.raises(MyaError, match="past the buffer"):
        b.array("int32", (2, 200), strides=(200, 1), offset=4).__dlpack__()
    with pytest.raises(MyaError, match="multiple of the element size"):
        b.array("int64", (4,), offset=4).__dlpack__()
    with pytest.raises(MyaError, match="negative stride"):
        b.array("int32", (2, 2), strides=(-2, 1)).__dlpack__()
    with pytest.raises(BufferError):
        b.array("int32", (4,)).__dlpack__(stream=1)
    with pytest.raises(BufferError):
        b.array("int32", (4,)).__dlpack__(copy=True)
    # an empty view is fine anywhere inside the buffer
    import torch
    assert torch.from_dlpack(b.array("int64", (0, 5))).shape == (0, 5)


@pytest.mark.gpu
def test_stream_handoff_orders_producer_before_consumer():
    import torch
    from mymyr_amd.dlpack import DeviceBuffer

    n = 1 << 24
    b = DeviceBuffer(n * 4)
    side = torch.cuda.Stream()
    t = torch.from_dlpack(b.array("int32", (n,), producer_stream=0))
    t.zero_()
    torch.cuda.synchronize()
    with torch.cuda.stream(side):
        # work queued on the side stream, exported to a consumer on the default stream
        src = torch.arange(n, dtype=torch.int32, device="cuda")
        t.copy_(src * 2 + 1)
        arr = b.array("int32", (n,), producer_stream=side.cuda_stream)
    cap = arr.__dlpack__(stream=torch.cuda.default_stream().cuda_stream)
    got = torch.utils.dlpack.from_dlpack(cap)
    s = got[-1].item()  # read on the default stream
    assert s == 2 * (n - 1) + 1


@pytest.mark.gpu
def test_state_set_rows_export():
    import torch
    from mymyr_amd import gen, hip

    rows = gen.dedup_rows(0, 5000, 16, seed=11)
    s = hip.StateSet(10000, 16, 0.5, batch=2048)
    n, ids, is_new = s.insert(torch.from_numpy(rows.view(np.int64)).cuda())
    got = torch.from_dlpack(s.rows())
    assert got.shape == (n, 16)
    g = got.cpu().numpy().view(np.uint64)
    first = is_new.cpu().numpy().astype(bool)
    assert np.array_equal(g, rows[first])  # new states in id order = first occurrences in row order
    # the rows outlive the set's handle
    del s
    gc.collect()
    assert np.array_equal(got.cpu().numpy().view(np.uint64), g)
