"""Array carriers accepted by the kernel wrappers.

The kernels work on memory described by an address, a shape, a dtype, strides and a device.  A
torch tensor is one carrier of that description.  The wrappers accept any object that exports it
through one of the two common protocols, without a copy:

* DLPack (``__dlpack__`` / ``__dlpack_device__``): CuPy, JAX, NumPy (host memory), TensorFlow,
  torch and others;
* the CUDA array interface (``__cuda_array_interface__``, v2/v3), which array libraries also export
  for HIP device memory: ``data`` = (address, read-only), ``shape``, ``typestr`` and ``strides``.
  Such memory belongs to the current device, as the protocol defines.

``DeviceArray`` describes raw memory the caller owns -- a ``hipMalloc`` result, a pointer from
another runtime -- with no array library at all.

Every such argument becomes a torch view of the same memory.  Results written through ``out=``
therefore land in the caller's buffer.  Results the wrappers allocate are torch tensors, which
export ``__dlpack__`` so the caller's library can take them without a copy.  The caller orders its
own work before the call: the kernels run on torch's current stream and do not wait on the
producer's stream.
"""
from __future__ import annotations

import ctypes
import functools
import threading

import numpy as np
import torch

# DLPack constants (dlpack.h): device types and dtype codes.
_KDL_CPU, _KDL_ROCM = 1, 10
_KDL_INT, _KDL_UINT, _KDL_FLOAT, _KDL_BOOL = 0, 1, 2, 6


class _DLDevice(ctypes.Structure):
    _fields_ = [("device_type", ctypes.c_int32), ("device_id", ctypes.c_int32)]


class _DLDataType(ctypes.Structure):
    _fields_ = [("code", ctypes.c_uint8), ("bits", ctypes.c_uint8), ("lanes", ctypes.c_uint16)]


class _DLTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("device", _DLDevice), ("ndim", ctypes.c_int32),
                ("dtype", _DLDataType), ("shape", ctypes.POINTER(ctypes.c_int64)),
                ("strides", ctypes.POINTER(ctypes.c_int64)), ("byte_offset", ctypes.c_uint64)]


class _DLManagedTensor(ctypes.Structure):
    pass


_DELETER = ctypes.CFUNCTYPE(None, ctypes.POINTER(_DLManagedTensor))
_DLManagedTensor._fields_ = [("dl_tensor", _DLTensor), ("manager_ctx", ctypes.c_void_p), ("deleter", _DELETER)]

# Exported tensors stay referenced here (with the owner of their memory) until the consumer calls
# the deleter.  A capsule that no consumer takes keeps its entry: capsules are only made inside
# as_tensor, which consumes them at once.
_live: dict[int, tuple] = {}
_live_lock = threading.Lock()


@_DELETER
def _release(managed) -> None:
    with _live_lock:
        _live.pop(ctypes.addressof(managed.contents), None)


_capsule_new = ctypes.pythonapi.PyCapsule_New
_capsule_new.restype = ctypes.py_object
_capsule_new.argtypes = [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_void_p]


def _dl_dtype(dtype: np.dtype) -> _DLDataType:
    kind = {"i": _KDL_INT, "u": _KDL_UINT, "f": _KDL_FLOAT, "b": _KDL_BOOL}.get(dtype.kind)
    if kind is None:
        raise TypeError(f"unsupported dtype {dtype}")
    return _DLDataType(kind, dtype.itemsize * 8, 1)


class DeviceArray:
    """Raw memory as an array: address, shape, dtype, strides (in elements) and device.

    ``device`` is a GPU ordinal or ``"cpu"`` for host memory.  ``owner`` is kept alive as long
    as any view of the memory exists.  The object exports DLPack, so ``torch.from_dlpack`` (and
    every wrapper here) takes it without a copy.
    """

    def __init__(self, ptr: int, shape, dtype, device=0, strides=None, owner=None):
        self.ptr = int(ptr)
        self.shape = tuple(int(s) for s in shape)
        self.dtype = np.dtype(dtype)
        self.strides = None if strides is None else tuple(int(s) for s in strides)
        if self.strides is not None and len(self.strides) != len(self.shape):
            raise ValueError("strides must have one entry per dimension")
        self.device = device
        self.owner = owner

    @classmethod
    def from_cuda_array_interface(cls, obj) -> "DeviceArray":
        cai = obj.__cuda_array_interface__
        dtype = np.dtype(cai["typestr"])
        strides = cai.get("strides")
        if strides is not None:
            if any(s % dtype.itemsize for s in strides):
                raise ValueError("__cuda_array_interface__ strides are not whole elements")
            strides = [s // dtype.itemsize for s in strides]
        return cls(cai["data"][0], cai["shape"], dtype, torch.cuda.current_device(), strides, owner=obj)

    def __dlpack_device__(self):
        return (_KDL_CPU, 0) if self.device == "cpu" else (_KDL_ROCM, int(self.device))

    def __dlpack__(self, stream=None, **_):
        n = len(self.shape)
        shape = (ctypes.c_int64 * max(n, 1))(*self.shape)
        strides = None if self.strides is None else (ctypes.c_int64 * max(n, 1))(*self.strides)
        managed = _DLManagedTensor()
        dev_type, dev_id = self.__dlpack_device__()
        managed.dl_tensor = _DLTensor(self.ptr, _DLDevice(dev_type, dev_id), n, _dl_dtype(self.dtype),
                                      ctypes.cast(shape, ctypes.POINTER(ctypes.c_int64)),
                                      None if strides is None else ctypes.cast(strides, ctypes.POINTER(ctypes.c_int64)),
                                      0)
        managed.manager_ctx = None
        managed.deleter = _release
        with _live_lock:
            _live[ctypes.addressof(managed)] = (managed, shape, strides, self.owner, self)
        return _capsule_new(ctypes.addressof(managed), b"dltensor", None)


def as_tensor(x):
    """``x`` as a torch tensor over the same memory when it is an array carrier; otherwise ``x``."""
    if x is None or isinstance(x, (torch.Tensor, bool, int, float, str, bytes, tuple, list, dict, torch.device)):
        return x
    if hasattr(x, "__dlpack__") and hasattr(x, "__dlpack_device__"):
        return torch.from_dlpack(x)
    if hasattr(x, "__cuda_array_interface__"):
        return torch.from_dlpack(DeviceArray.from_cuda_array_interface(x))
    return x


def accepts_carriers(fn):
    """Wrap a kernel entry so that every array argument may be any carrier ``as_tensor`` takes."""
    @functools.wraps(fn)
    def wrapper(*args, **kwargs):
        return fn(*(as_tensor(a) for a in args), **{k: as_tensor(v) for k, v in kwargs.items()})
    return wrapper
