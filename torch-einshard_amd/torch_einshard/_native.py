"""ctypes binding of libeinshard_hip.so (C ABI declared in include/einshard_hip.h).

The library is loaded after ``torch`` so that it binds to the HIP runtime torch
already mapped (both carry the soname ``libamdhip64.so.7``).  There is no
fallback: if the library is missing or a call fails, a Python exception says
so.
"""

import ctypes
import os
import threading

import torch

__all__ = [
    "EsAxis",
    "GatherDesc",
    "BcastDesc",
    "ReduceDesc",
    "ContractDesc",
    "lib",
    "library_path",
    "call",
    "MAX_AXES",
    "DTYPE_CODES",
    "BOUNDARY_CODES",
    "NativeError",
]

MAX_AXES = 8
ABI_VERSION = 1

ES_OK = 0
ES_ERR_INVALID = -1
ES_ERR_UNSUPPORTED = -2
ES_ERR_LAUNCH = -3
ES_ERR_WORKSPACE = -4

DTYPE_CODES = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2}
BOUNDARY_CODES = {"constant": 0, "replicate": 1, "periodic": 2}

_c_i64_axes = ctypes.c_int64 * MAX_AXES
_c_i32_axes = ctypes.c_int32 * MAX_AXES


class EsAxis(ctypes.Structure):
    _fields_ = [("size", ctypes.c_int64), ("a", ctypes.c_int64), ("b", ctypes.c_int64), ("c", ctypes.c_int64)]


_axes_array = EsAxis * MAX_AXES


class GatherDesc(ctypes.Structure):
    _fields_ = [
        ("elem_size", ctypes.c_int32),
        ("boundary", ctypes.c_int32),
        ("fill_bits", ctypes.c_uint64),
        ("out_rank", ctypes.c_int32),
        ("in_rank", ctypes.c_int32),
        ("out_size", _c_i64_axes),
        ("in_size", _c_i64_axes),
        ("in_stride", _c_i64_axes),
        ("offset", _c_i64_axes),
        ("pos", _c_i32_axes),
        ("win", _c_i32_axes),
    ]


class BcastDesc(ctypes.Structure):
    _fields_ = [("dtype", ctypes.c_int32), ("rank", ctypes.c_int32), ("axes", _axes_array)]


class ReduceDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("has_y", ctypes.c_int32),
        ("n_keep", ctypes.c_int32),
        ("n_red", ctypes.c_int32),
        ("keep", _axes_array),
        ("red", _axes_array),
    ]


class ContractDesc(ctypes.Structure):
    _fields_ = [
        ("dtype", ctypes.c_int32),
        ("n_batch", ctypes.c_int32),
        ("n_m", ctypes.c_int32),
        ("n_n", ctypes.c_int32),
        ("n_k", ctypes.c_int32),
        ("batch", _axes_array),
        ("m", _axes_array),
        ("n", _axes_array),
        ("k", _axes_array),
    ]


class NativeError(RuntimeError):
    """A libeinshard_hip entry point returned an error status."""

    def __init__(self, entry, status, message):
        self.entry = entry
        self.status = status
        super().__init__(f"{entry} failed (status {status}): {message}")


_PACKAGE_DIR = os.path.dirname(os.path.abspath(__file__))
_lib = None
_lock = threading.Lock()


def library_path():
    return os.environ.get("EINSHARD_HIP_LIB") or os.path.join(_PACKAGE_DIR, "_lib", "libeinshard_hip.so")


_SIGNATURES = {
    "es_gather": (ctypes.c_int, [ctypes.POINTER(GatherDesc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]),
    "es_bcast": (
        ctypes.c_int,
        [ctypes.POINTER(BcastDesc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p],
    ),
    "es_reduce_workspace_bytes": (ctypes.c_int64, [ctypes.POINTER(ReduceDesc)]),
    "es_reduce": (
        ctypes.c_int,
        [
            ctypes.POINTER(ReduceDesc),
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_int64,
            ctypes.c_void_p,
        ],
    ),
    "es_contract": (
        ctypes.c_int,
        [ctypes.POINTER(ContractDesc), ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p],
    ),
    "es_contract_bias": (
        ctypes.c_int,
        [
            ctypes.POINTER(ContractDesc),
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
            ctypes.c_void_p,
        ],
    ),
    "es_abi_version": (ctypes.c_int, []),
    "es_version": (ctypes.c_char_p, []),
    "es_last_error": (ctypes.c_char_p, []),
    "es_last_kernel": (ctypes.c_char_p, []),
}


def lib():
    """Load (once) and return the ctypes handle of libeinshard_hip.so."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise RuntimeError(
                f"libeinshard_hip.so not found at {path}: build it first "
                "(python -m torch_einshard._build, or __graft_entry__.build())"
            )
        handle = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        for name, (restype, argtypes) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = restype
            fn.argtypes = argtypes
        if handle.es_abi_version() != ABI_VERSION:
            raise RuntimeError(
                f"libeinshard_hip ABI version {handle.es_abi_version()} does not match the binding ({ABI_VERSION})"
            )
        _lib = handle
        return _lib


def last_kernel():
    return lib().es_last_kernel().decode()


def call(entry, *args):
    """Call an entry point; raise on a negative status."""
    handle = lib()
    status = getattr(handle, entry)(*args)
    if status < 0:
        raise NativeError(entry, status, handle.es_last_error().decode())
    return status


def stream_of(tensor):
    return ctypes.c_void_p(torch.cuda.current_stream(tensor.device).cuda_stream)
