"""Run planned operations on the GPU through libeinshard_hip.

Every function here takes device tensors, allocates the (dense) output with
``torch.empty`` and enqueues exactly one library entry point on the current
stream.  Tensors are passed by data pointer plus element strides; nothing is
copied or made contiguous on the host side.
"""

import ctypes

import torch

from . import _native
from ._native import MAX_AXES, BcastDesc, ContractDesc, GatherDesc, ReduceDesc, call
from .planner import BcastOp, ContractOp, EmptyOp, GatherOp, ReduceOp

__all__ = ["check_device_tensors", "run_op", "run_gather", "dtype_code", "fill_bits"]

_ELEM_SIZES = {1, 2, 4, 8}


def check_device_tensors(xs, *, what="einshard"):
    """All operands must be ROCm device tensors on one device with one dtype."""
    for x in xs:
        if not isinstance(x, torch.Tensor):
            raise TypeError(f"{what}: expected torch.Tensor operands, got {type(x).__name__}")
    devices = {x.device for x in xs}
    if len(devices) != 1:
        raise RuntimeError(f"{what}: operands are on different devices {sorted(map(str, devices))}")
    device = xs[0].device
    if device.type != "cuda":
        raise RuntimeError(
            f"{what}: this build executes on MI355X (ROCm) device tensors only; got a tensor on {device}"
        )
    dtypes = {x.dtype for x in xs}
    if len(dtypes) != 1:
        raise RuntimeError(f"{what}: operands must share one dtype, got {sorted(map(str, dtypes))}")
    return device, xs[0].dtype


def dtype_code(dtype, what):
    try:
        return _native.DTYPE_CODES[dtype]
    except KeyError:
        raise NotImplementedError(
            f"{what}: dtype {dtype} is not supported by the MI355X kernels (float32, bfloat16, float16)"
        ) from None


def fill_bits(value, dtype):
    """Bit pattern of ``value`` converted to ``dtype`` the way ``Tensor.fill_`` converts it."""
    raw = torch.empty((1,), dtype=dtype).fill_(value).view(torch.uint8)
    return int.from_bytes(bytes(raw.tolist()), "little")


def _set_axes(array, axes, what):
    if len(axes) > MAX_AXES:
        raise NotImplementedError(f"{what}: more than {MAX_AXES} independent axes after merging")
    for i, axis in enumerate(axes):
        array[i].size = axis.size
        array[i].a = axis.a
        array[i].b = axis.b
        array[i].c = axis.c
    return len(axes)


def _ptr(tensor):
    return ctypes.c_void_p(tensor.data_ptr())


def run_gather(desc, x, out):
    call("es_gather", ctypes.byref(desc), _ptr(x), _ptr(out), _native.stream_of(out))


def run_op(op, xs, dtype, device):
    """Execute a planner op over operands ``xs`` (one or two tensors)."""
    out = torch.empty(op.out_shape, dtype=dtype, device=device)
    if isinstance(op, EmptyOp) or out.numel() == 0:
        return out
    stream = _native.stream_of(out)

    if isinstance(op, GatherOp):
        desc = GatherDesc()
        elem = xs[0].element_size()
        if elem not in _ELEM_SIZES:
            raise NotImplementedError(f"einshard: element size {elem} is not supported")
        desc.elem_size = elem
        desc.boundary = 0
        desc.fill_bits = 0
        axes = op.axes or []
        if len(axes) > MAX_AXES:
            raise NotImplementedError(f"einshard: more than {MAX_AXES} independent axes after merging")
        if not axes:
            desc.out_rank = 1
            desc.out_size[0] = 1
            desc.in_rank = 0
        else:
            desc.out_rank = len(axes)
            desc.in_rank = len(axes)
            for i, axis in enumerate(axes):
                desc.out_size[i] = axis.size
                desc.in_size[i] = axis.size
                desc.in_stride[i] = axis.a
                desc.offset[i] = 0
                desc.pos[i] = i
                desc.win[i] = -1
        call("es_gather", ctypes.byref(desc), _ptr(xs[0]), _ptr(out), stream)
        return out

    code = dtype_code(dtype, "einshard")

    if isinstance(op, BcastOp):
        desc = BcastDesc()
        desc.dtype = code
        desc.rank = _set_axes(desc.axes, op.axes, "einshard")
        call("es_bcast", ctypes.byref(desc), _ptr(xs[0]), _ptr(xs[1]), _ptr(out), stream)
        return out

    if isinstance(op, ReduceOp):
        desc = ReduceDesc()
        desc.dtype = code
        desc.has_y = 1 if op.has_y else 0
        desc.n_keep = _set_axes(desc.keep, op.keep, "einshard")
        desc.n_red = _set_axes(desc.red, op.red, "einshard")
        need = call("es_reduce_workspace_bytes", ctypes.byref(desc))
        workspace = torch.empty(max(int(need), 1), dtype=torch.uint8, device=device) if need > 0 else None
        y = xs[1] if op.has_y else xs[0]
        call(
            "es_reduce",
            ctypes.byref(desc),
            _ptr(xs[0]),
            _ptr(y),
            _ptr(out),
            _ptr(workspace) if workspace is not None else ctypes.c_void_p(0),
            ctypes.c_int64(int(need) if need > 0 else 0),
            stream,
        )
        return out

    if isinstance(op, ContractOp):
        desc = ContractDesc()
        desc.dtype = code
        desc.n_batch = _set_axes(desc.batch, op.batch, "einshard")
        desc.n_m = _set_axes(desc.m, op.m, "einshard")
        desc.n_n = _set_axes(desc.n, op.n, "einshard")
        desc.n_k = _set_axes(desc.k, op.k, "einshard")
        a, b = (xs[1], xs[0]) if op.swapped else (xs[0], xs[1])
        call("es_contract", ctypes.byref(desc), _ptr(a), _ptr(b), _ptr(out), stream)
        return out

    raise TypeError(f"unknown planned op {type(op).__name__}")
