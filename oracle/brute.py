"""ctypes wrappers of oracle/brute.c — TEST INFRASTRUCTURE ONLY.

``brute_einsum(equation, *tensors)`` evaluates a torch.einsum equation in fp64
by exhaustive loops (ellipsis, diagonals and size-1 broadcasting expanded
here into plain labels and strides).  ``brute_window`` evaluates the closed
form of einwindow / einhalo byte by byte.
"""

import ctypes
import os
import subprocess

import numpy as np
import torch

__all__ = ["brute_einsum", "brute_window", "library"]

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libes_brute.so")
_MAX = 16
_lib = None

_DTYPE = {torch.float32: 0, torch.bfloat16: 1, torch.float16: 2, torch.float64: 3}


def library():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        _lib = ctypes.CDLL(_LIB_PATH)
        _lib.brute_einsum.restype = ctypes.c_int
        _lib.brute_window.restype = ctypes.c_int
    return _lib


def _i64(values, n=_MAX):
    arr = (ctypes.c_int64 * n)()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr


def _i32(values, n=_MAX):
    arr = (ctypes.c_int * n)()
    for i, v in enumerate(values):
        arr[i] = int(v)
    return arr


def brute_einsum(equation, *tensors):
    """fp64 result (a float64 CPU tensor) of ``torch.einsum(equation, *tensors)``."""
    tensors = [t.detach().cpu().contiguous() for t in tensors]
    lhs, rhs = equation.replace(" ", "").split("->")
    specs = lhs.split(",")
    ell_rank = max(
        (t.dim() - len(spec.replace("...", "")) if "..." in spec else 0) for spec, t in zip(specs, tensors)
    )
    ell_labels = [f"#{i}" for i in range(ell_rank)]

    def expand(spec, ndim):
        if "..." not in spec:
            return list(spec)
        head, tail = spec.split("...")
        k = ndim - len(head) - len(tail)
        return list(head) + ell_labels[ell_rank - k:] + list(tail)

    dims = [expand(spec, t.dim()) for spec, t in zip(specs, tensors)]
    out = expand(rhs, len(rhs.replace("...", "")) + ell_rank)
    order = []
    for d in dims:
        for label in d:
            if label not in order:
                order.append(label)
    size = {}
    for d, t in zip(dims, tensors):
        for label, n in zip(d, t.shape):
            if n != 1:
                size[label] = n
            else:
                size.setdefault(label, 1)
    index = {label: i for i, label in enumerate(order)}
    labels_in = (ctypes.c_int * (2 * _MAX))()
    strides_in = (ctypes.c_int64 * (2 * _MAX))()
    ranks = (ctypes.c_int * 2)()
    data = (ctypes.c_void_p * 2)()
    dtypes = (ctypes.c_int * 2)()
    for t_i, (d, t) in enumerate(zip(dims, tensors)):
        ranks[t_i] = t.dim()
        data[t_i] = t.data_ptr()
        dtypes[t_i] = _DTYPE[t.dtype]
        for j, (label, n, s) in enumerate(zip(d, t.shape, t.stride())):
            labels_in[t_i * _MAX + j] = index[label]
            strides_in[t_i * _MAX + j] = 0 if (n == 1 and size[label] != 1) else s
    out_shape = [size[label] for label in out]
    result = torch.zeros(out_shape, dtype=torch.float64)
    rc = library().brute_einsum(
        len(order),
        _i64([size[label] for label in order]),
        len(tensors),
        ranks,
        labels_in,
        strides_in,
        data,
        dtypes,
        len(out),
        _i32([index[label] for label in out]),
        ctypes.c_void_p(result.data_ptr()),
    )
    if rc != 0:
        raise ValueError(f"brute_einsum: bad arguments for {equation!r}")
    return result


def brute_window(x, out_shape, pos, win, left, *, boundary="constant", fill=0):
    """Closed-form window/halo: see oracle/brute.c.  Returns a CPU tensor."""
    x = x.detach().cpu()
    out = torch.empty(out_shape, dtype=x.dtype)
    fill_t = torch.empty((1,), dtype=x.dtype).fill_(fill)
    code = {"constant": 0, "replicate": 1, "periodic": 2}[boundary]
    rc = library().brute_window(
        x.element_size(),
        x.dim(),
        _i64(x.shape),
        _i64(x.stride()),
        len(out_shape),
        _i64(out_shape),
        _i32(pos),
        _i32(win),
        _i64(left),
        code,
        ctypes.c_void_p(fill_t.data_ptr()),
        ctypes.c_void_p(x.data_ptr()),
        ctypes.c_void_p(out.data_ptr()),
    )
    if rc != 0:
        raise ValueError("brute_window: bad arguments")
    return out


def numpy_einsum_f64(equation, *tensors):
    """Second independent reference: numpy's einsum in float64."""
    arrays = [t.detach().cpu().to(torch.float64).numpy() for t in tensors]
    return torch.from_numpy(np.einsum(equation, *arrays, optimize=False))
