"""Borrow raw device (or host) memory as a torch tensor through a DLPack capsule.

Replaces the reference's CuPy UnownedMemory + DLPack route
(elastic_kv/backing.py:443-458) with a capsule built directly from ctypes:
the DLManagedTensor lives in Python, its deleter drops the entry that keeps
the owner alive, and torch.from_dlpack consumes the capsule without copying.
"""

import ctypes as ct
import threading

import torch

# DLPack device types (dlpack.h): host memory and ROCm device memory.
KDL_CPU = 1
KDL_ROCM = 10

_KDL_UINT = 1


class _DLDevice(ct.Structure):
    _fields_ = [("device_type", ct.c_int32), ("device_id", ct.c_int32)]


class _DLDataType(ct.Structure):
    _fields_ = [("code", ct.c_uint8), ("bits", ct.c_uint8), ("lanes", ct.c_uint16)]


class _DLTensor(ct.Structure):
    _fields_ = [
        ("data", ct.c_void_p),
        ("device", _DLDevice),
        ("ndim", ct.c_int32),
        ("dtype", _DLDataType),
        ("shape", ct.POINTER(ct.c_int64)),
        ("strides", ct.POINTER(ct.c_int64)),
        ("byte_offset", ct.c_uint64),
    ]


class _DLManagedTensor(ct.Structure):
    pass


_DELETER = ct.CFUNCTYPE(None, ct.POINTER(_DLManagedTensor))
_DLManagedTensor._fields_ = [
    ("dl_tensor", _DLTensor),
    ("manager_ctx", ct.c_void_p),
    ("deleter", _DELETER),
]

_capsule_new = ct.pythonapi.PyCapsule_New
_capsule_new.restype = ct.py_object
_capsule_new.argtypes = [ct.c_void_p, ct.c_char_p, ct.c_void_p]

# address of a live DLManagedTensor -> (struct, shape array, owner)
_live = {}
_lock = threading.Lock()


# The deleter can run during interpreter shutdown, after this module's
# globals are cleared: everything it uses is bound as a default argument.
@_DELETER
def _release(managed, _cast=ct.cast, _void_p=ct.c_void_p, _lock=_lock, _live=_live):
    key = _cast(managed, _void_p).value
    with _lock:
        _live.pop(key, None)


def live_borrows():
    """Number of borrowed views whose consumer has not released them yet."""
    with _lock:
        return len(_live)


def borrow_bytes(address, nbytes, device_type, device_id, owner):
    """Return a uint8 tensor of `nbytes` at `address` that keeps `owner` alive."""
    if nbytes < 0:
        raise ValueError("byte count must be nonnegative")
    shape = (ct.c_int64 * 1)(nbytes)
    managed = _DLManagedTensor()
    managed.dl_tensor.data = address
    managed.dl_tensor.device = _DLDevice(device_type, device_id)
    managed.dl_tensor.ndim = 1
    managed.dl_tensor.dtype = _DLDataType(_KDL_UINT, 8, 1)
    managed.dl_tensor.shape = shape
    managed.dl_tensor.strides = None
    managed.dl_tensor.byte_offset = 0
    managed.manager_ctx = None
    managed.deleter = _release
    key = ct.addressof(managed)
    with _lock:
        _live[key] = (managed, shape, owner)
    try:
        capsule = _capsule_new(key, b"dltensor", None)
        return torch.from_dlpack(capsule)
    except BaseException:
        with _lock:
            _live.pop(key, None)
        raise
