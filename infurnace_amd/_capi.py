"""ctypes binding of libinfurnace_hip.so (the C ABI in include/infurnace_amd.h).

The library is loaded from the package directory only (built in-tree by
``infurnace_amd.build``).  There is no fallback: when the library is missing
or does not export every declared entry point, ``lib()`` raises
``NativeLibraryError`` and every operation that needs it fails loudly.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "libinfurnace_hip.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
ABI_VERSION = 1

IFN_OK = 0
IFN_ERR_INVALID_ARGUMENT = -1
IFN_ERR_UNSUPPORTED = -2
IFN_ERR_ALIGNMENT = -3
IFN_ERR_WORKSPACE = -4
IFN_ERR_HIP = -5

_p = ctypes.c_void_p
_i32 = ctypes.c_int32
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); the declarations of include/infurnace_amd.h
SIGNATURES: dict[str, tuple] = {
    "ifn_status_string": (ctypes.c_char_p, [ctypes.c_int]),
    "ifn_abi_version": (ctypes.c_int, []),
    "ifn_store_kv": (ctypes.c_int, [_p, _i64, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _p]),
    "ifn_store_kv_layers": (ctypes.c_int, [_p, _i32, _i64, _p, _p, _p, _p, _i32, _i32, _i32, _i32, _p]),
    "ifn_paged_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "ifn_paged_decode": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _p, _i32, _i32, _i32, _i32,
                                        _i32, _i32, _f32, _p, _sz, _p]),
    "ifn_paged_decode_append": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _p, _p, _p, _p, _i32, _i32, _i32,
                                               _i32, _i32, _i32, _f32, _p, _sz, _p]),
    "ifn_paged_decode_plan_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _i32]),
    "ifn_paged_decode_plan": (ctypes.c_int, [_p, _sz, _p, _i32, _p, _p, _p, _i64, _i32, _i32, _i32, _i32, _i32,
                                             _i32, _p]),
    "ifn_paged_decode_planned": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _p, _i32, _i32, _i32, _i32, _i32,
                                                _i32, _f32, _p, _sz, _p, _sz, _p]),
    "ifn_paged_decode_append_planned": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _p, _p, _p, _p, _i32, _i32,
                                                       _i32, _i32, _i32, _i32, _f32, _p, _sz, _p, _sz, _p]),
    # the first layer's decode of a step, writing the step's plan (same arguments as the planned calls)
    "ifn_paged_decode_planning": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _p, _i32, _i32, _i32, _i32, _i32,
                                                 _i32, _f32, _p, _sz, _p, _sz, _p]),
    "ifn_paged_decode_append_planning": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _p, _p, _p, _p, _i32, _i32,
                                                        _i32, _i32, _i32, _i32, _f32, _p, _sz, _p, _sz, _p]),
    "ifn_paged_decode_noalloc_max_bytes": (_sz, []),
    "ifn_paged_decode_noalloc": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _p, _i32, _i32, _i32, _i32,
                                                _i32, _i32, _f32, _p]),
    "ifn_paged_decode_shared_prefix_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "ifn_paged_decode_shared_prefix": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _i32, _p, _p, _i32, _i32,
                                                      _i32, _i32, _i32, _i32, _f32, _p, _sz, _p]),
    "ifn_paged_decode_shared_prefix_planned": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _p, _i32, _p, _p, _i32,
                                                              _i32, _i32, _i32, _i32, _i32, _f32, _p, _sz, _p, _sz,
                                                              _p]),
    # plan, bytes, block_tables, max_pages, seq_lens, active, shared_pages, num_pages, batch, hq, hkv, d, bs, msl,
    # stream
    "ifn_paged_decode_shared_prefix_plan": (ctypes.c_int, [_p, _sz, _p, _i32, _p, _p, _i32, _i64, _i32, _i32, _i32,
                                                           _i32, _i32, _i32, _p]),
    "ifn_paged_prefill_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "ifn_paged_prefill": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _i32, _i32, _i32, _i32, _i32,
                                         _i32, _f32, _p, _sz, _p]),
    "ifn_paged_prefill_append": (ctypes.c_int, [_p, _p, _p, _i64, _p, _i32, _i32, _i32, _p, _p, _i32, _i32, _i32,
                                                _i32, _f32, _p, _sz, _p]),
    "ifn_qk_norm_rope_append": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _p, _i64,
                                               _i32, _i32, _i32, _i32, _i32, _f32, _p]),
    "ifn_paged_decode_prep_append": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _i64, _p, _i32,
                                                    _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32, _f32, _p,
                                                    _sz, _p, _sz, _p]),
    "ifn_paged_decode_prep_append_planning": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _p, _p, _i64, _p,
                                                             _i32, _p, _p, _i32, _i32, _i32, _i32, _i32, _i32, _f32,
                                                             _f32, _p, _sz, _p, _sz, _p]),
    # out, q, k, v, q_norm_weight, k_norm_weight, rope_table, max_positions, pool, num_pages, block_table,
    # max_pages, query_start, T, hq, hkv, head_dim, block_size, eps, scale, workspace, bytes, stream
    "ifn_paged_prefill_prep_append": (ctypes.c_int, [_p, _p, _p, _p, _p, _p, _p, _i32, _p, _i64, _p, _i32, _i32,
                                                     _i32, _i32, _i32, _i32, _i32, _f32, _f32, _p, _sz, _p]),
    "ifn_zero_pages": (ctypes.c_int, [_p, _i32, _i64, _p, _i32, _i32, _i32, _i32, _p]),
    "ifn_copy_pages": (ctypes.c_int, [_p, _i32, _i64, _p, _p, _i32, _i32, _i32, _i32, _p]),
}


class NativeLibraryError(RuntimeError):
    """libinfurnace_hip.so is missing, stale or incomplete."""


class KernelLaunchError(RuntimeError):
    """A C entry point returned a non-zero status."""

    def __init__(self, name: str, status: int):
        self.status = status
        super().__init__(f"{name} failed: {status_string(status)} ({status})")


_lib: ctypes.CDLL | None = None
_lock = threading.Lock()


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryError(
                    f"{LIB_PATH} not found: build it with `python -m infurnace_amd.build` "
                    "(there is no CPU fallback)")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                try:
                    fn = getattr(L, name)
                except AttributeError as e:
                    raise NativeLibraryError(f"{LIB_PATH} does not export {name}; rebuild it") from e
                fn.restype = res
                fn.argtypes = args
            if L.ifn_abi_version() != ABI_VERSION:
                raise NativeLibraryError(f"{LIB_PATH} ABI {L.ifn_abi_version()} != {ABI_VERSION}; rebuild it")
            _lib = L
    return _lib


def status_string(status: int) -> str:
    return lib().ifn_status_string(status).decode()


def check(name: str, status: int) -> None:
    if status != IFN_OK:
        raise KernelLaunchError(name, status)


def call(name: str, *args) -> None:
    """Invoke a status-returning entry point and raise on failure."""
    check(name, getattr(lib(), name)(*args))
