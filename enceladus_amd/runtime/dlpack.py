"""DLPack export of `Tensor` as kDLROCM (reference: runtime/tensor.py:159-194 exports
kDLMetal through `_C/bindings.mm:273-338`).

The capsule holds a `DLManagedTensor` (or, for consumers that ask for DLPack >= 1.0, a
`DLManagedTensorVersioned`) whose `data` is the HBM device pointer. The structures follow
dlpack.h v1.0 and are built with ctypes; the deleter is a C callback that drops this
module's reference to the exporting tensor, which keeps the memory alive until the consumer
is done with it. A capsule that is never consumed is released by its destructor.
"""

from __future__ import annotations

import ctypes
import threading

import numpy as np

K_DL_ROCM = 10

# dtype name -> (DLDataTypeCode, bits): kDLInt 0, kDLUInt 1, kDLFloat 2, kDLBfloat 4, kDLBool 6
DLPACK_DTYPES = {
    "i1": (6, 8), "i8": (0, 8), "u8": (1, 8), "i16": (0, 16), "u16": (1, 16),
    "i32": (0, 32), "u32": (1, 32), "i64": (0, 64), "u64": (1, 64),
    "fp16": (2, 16), "bf16": (4, 16), "fp32": (2, 32), "fp64": (2, 64),
}


class DLDevice(ctypes.Structure):
    _fields_ = [("device_type", ctypes.c_int32), ("device_id", ctypes.c_int32)]


class DLDataType(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16)]


class DLTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("device", DLDevice), ("ndim", ctypes.c_int32),
                ("dtype", DLDataType), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("strides", ctypes.POINTER(ctypes.c_int64)), ("byte_offset", ctypes.c_uint64)]


class DLManagedTensor(ctypes.Structure):
    pass


_DELETER = ctypes.CFUNCTYPE(None, ctypes.c_void_p)
DLManagedTensor._fields_ = [("dl_tensor", DLTensor), ("manager_ctx", ctypes.c_void_p),
                            ("deleter", _DELETER)]


class DLPackVersion(ctypes.Structure):
    _fields_ = [("major", ctypes.c_uint32), ("minor", ctypes.c_uint32)]


class DLManagedTensorVersioned(ctypes.Structure):
    _fields_ = [("version", DLPackVersion), ("manager_ctx", ctypes.c_void_p),
                ("deleter", _DELETER), ("flags", ctypes.c_uint64), ("dl_tensor", DLTensor)]


# exports alive in consumers: id -> (owner tensor, managed struct, shape/strides arrays)
_LIVE: dict[int, tuple] = {}
_LOCK = threading.Lock()


def _release(addr: int) -> None:
    with _LOCK:
        _LIVE.pop(addr, None)


@_DELETER
def _deleter(addr):
    _release(addr)


# The destructor receives the capsule while it is being deallocated: it is handled as a raw
# pointer (a py_object conversion would take a new reference to a dying object).
_CAPSULE_DESTRUCTOR = ctypes.CFUNCTYPE(None, ctypes.c_void_p)
_PyCapsule_New = ctypes.pythonapi.PyCapsule_New
_PyCapsule_New.restype = ctypes.py_object
_PyCapsule_New.argtypes = [ctypes.c_void_p, ctypes.c_char_p, _CAPSULE_DESTRUCTOR]
_PyCapsule_IsValid = ctypes.pythonapi.PyCapsule_IsValid
_PyCapsule_IsValid.restype = ctypes.c_int
_PyCapsule_IsValid.argtypes = [ctypes.c_void_p, ctypes.c_char_p]
_PyCapsule_GetPointer = ctypes.pythonapi.PyCapsule_GetPointer
_PyCapsule_GetPointer.restype = ctypes.c_void_p
_PyCapsule_GetPointer.argtypes = [ctypes.c_void_p, ctypes.c_char_p]


@_CAPSULE_DESTRUCTOR
def _capsule_destructor(cap):
    # a consumer renames the capsule ("used_dltensor...") when it takes ownership; an
    # unconsumed capsule still owns its tensor
    for name in (b"dltensor", b"dltensor_versioned"):
        if _PyCapsule_IsValid(cap, name):
            _release(_PyCapsule_GetPointer(cap, name))


def export(owner, ptr: int, shape, strides, dtype_name: str, device_id: int = 0,
           versioned: bool = False):
    """A DLPack capsule over `ptr` (device memory of GPU `device_id`) that keeps `owner`
    alive until the consumer calls the deleter."""
    code, bits = DLPACK_DTYPES[dtype_name]
    nd = len(shape)
    shp = (ctypes.c_int64 * max(nd, 1))(*shape)
    std = (ctypes.c_int64 * max(nd, 1))(*strides)
    t = DLTensor(ctypes.c_void_p(ptr), DLDevice(K_DL_ROCM, device_id), nd,
                 DLDataType(code, bits, 1), ctypes.cast(shp, ctypes.POINTER(ctypes.c_int64)),
                 ctypes.cast(std, ctypes.POINTER(ctypes.c_int64)), 0)
    if versioned:
        m = DLManagedTensorVersioned(DLPackVersion(1, 0), None, _deleter, 0, t)
        name = b"dltensor_versioned"
    else:
        m = DLManagedTensor(t, None, _deleter)
        name = b"dltensor"
    addr = ctypes.addressof(m)
    with _LOCK:
        _LIVE[addr] = (owner, m, shp, std)
    return _PyCapsule_New(addr, name, _capsule_destructor)


def live_exports() -> int:
    """Number of exported capsules whose consumer has not released them yet."""
    with _LOCK:
        return len(_LIVE)


def dtype_code(np_dtype: np.dtype) -> tuple[int, int]:
    from enceladus_amd.language import core
    return DLPACK_DTYPES[core.dtype_from_numpy(np_dtype).name]
