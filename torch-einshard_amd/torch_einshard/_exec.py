"""Run planned operations on the GPU through libeinshard_hip.

Every function here takes device tensors, allocates the (dense) output with
``torch.empty`` and enqueues one library entry point on the current stream —
preceded, for a large 16-bit contraction whose operand is contiguous along M or
N, by one es_gather that copies that operand K-contiguous into a temporary.
Tensors are passed by data pointer plus element strides; nothing is copied or
made contiguous on the host side.
"""

import ctypes
from dataclasses import replace

import torch

from . import _native
from ._native import MAX_AXES, BcastDesc, ContractDesc, GatherDesc, ReduceDesc, call
from .planner import BcastOp, ContractOp, EmptyOp, GatherOp, ReduceOp, SubAxis, dense_strides

__all__ = ["check_device_tensors", "run_op", "run_gather", "dtype_code", "fill_bits", "Prepared", "prepare_op", "launch"]

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


class Prepared:
    """One planned launch.  The descriptor is built (and the reduction workspace
    size queried) once; a call then only allocates the output and binds data
    pointers, so a repeated expression costs one ctypes call on the host.

    ``repack`` lists operands first copied into a dense temporary by es_gather:
    (operand index, gather descriptor, temporary shape).

    ``split`` (a split-K contraction): (partials, reduce descriptor, its workspace
    bytes).  The contraction writes ``partials`` stacked partial results, which one
    es_reduce sums into the output."""

    __slots__ = ("entry", "desc", "ref", "out_shape", "order", "workspace", "noop", "repack", "split")

    def __init__(self, entry, desc, out_shape, order, workspace=0, noop=False, repack=(), split=None):
        self.entry = entry
        self.desc = desc
        self.ref = ctypes.byref(desc) if desc is not None else None
        self.out_shape = tuple(out_shape)
        self.order = order
        self.workspace = workspace
        self.noop = noop
        self.repack = tuple((index, desc_, ctypes.byref(desc_), shape) for index, desc_, shape in repack)
        self.split = None if split is None else (split[0], split[1], ctypes.byref(split[1]), split[2])


def _raw_stream(device):
    return torch._C._cuda_getCurrentRawStream(device.index if device.index is not None else torch.cuda.current_device())


def launch(prep, xs, device, dtype, bias=None):
    """Allocate the output and enqueue ``prep`` on the current stream of ``device``.

    ``bias`` (a contraction only): a dense vector over the N group added to every
    output row before the one rounding (es_contract_bias)."""
    out = torch.empty(prep.out_shape, dtype=dtype, device=device)
    if prep.noop or out.numel() == 0:
        return out
    handle = _native.lib()
    fn = getattr(handle, prep.entry)
    stream = _raw_stream(device)
    if prep.repack:
        xs = list(xs)
        for index, _, ref, shape in prep.repack:
            tmp = torch.empty(shape, dtype=xs[index].dtype, device=device)
            status = handle.es_gather(ref, xs[index].data_ptr(), tmp.data_ptr(), stream)
            if status < 0:
                raise _native.NativeError("es_gather", status, handle.es_last_error().decode())
            xs[index] = tmp
    ptrs = [xs[i].data_ptr() for i in prep.order]
    if prep.split is not None:
        # split-K: partial results, then their sum (a fixed order: deterministic)
        if bias is not None:
            raise AssertionError("a split-K contraction takes no bias")
        partials, _, rref, need = prep.split
        tmp = torch.empty((partials, out.numel()), dtype=dtype, device=device)
        status = fn(prep.ref, *ptrs, tmp.data_ptr(), stream)
        if status < 0:
            raise _native.NativeError(prep.entry, status, handle.es_last_error().decode())
        ws = torch.empty(need, dtype=torch.uint8, device=device) if need > 0 else None
        status = handle.es_reduce(rref, tmp.data_ptr(), tmp.data_ptr(), out.data_ptr(),
                                  ws.data_ptr() if ws is not None else None, need, stream)
        if status < 0:
            raise _native.NativeError("es_reduce", status, handle.es_last_error().decode())
        return out
    if prep.entry == "es_reduce":
        need = prep.workspace
        ws = torch.empty(need, dtype=torch.uint8, device=device) if need > 0 else None
        status = fn(prep.ref, ptrs[0], ptrs[1], out.data_ptr(), ws.data_ptr() if ws is not None else None, need, stream)
    elif bias is not None:
        if prep.entry != "es_contract":
            raise AssertionError("a bias applies to a contraction only")
        status = handle.es_contract_bias(prep.ref, *ptrs, bias.data_ptr(), out.data_ptr(), stream)
        if status < 0:
            raise _native.NativeError("es_contract_bias", status, handle.es_last_error().decode())
        return out
    else:
        status = fn(prep.ref, *ptrs, out.data_ptr(), stream)
    if status < 0:
        raise _native.NativeError(prep.entry, status, handle.es_last_error().decode())
    return out


def _ptr(tensor):
    return ctypes.c_void_p(tensor.data_ptr())


def run_gather(desc, x, out):
    call("es_gather", ctypes.byref(desc), _ptr(x), _ptr(out), _native.stream_of(out))


# The 256 x 256 contraction kernel for 16-bit types (contract_pipe) reads each operand
# K-contiguous (innermost K sub-axis of unit stride, a whole number of 64-deep K
# tiles) or contiguous along its rows (M for x, N for y: innermost row sub-axis of unit
# stride, 8-element runs, every other stride a multiple of 8), with every byte offset
# below 2^32.  When it would be chosen (enough tiles for every CU) and an operand fits
# neither while its rows are still the unit-stride axis, that operand is first copied
# K-contiguous into a temporary: one es_gather over its bytes buys the faster kernel.
_BIG_TILE = 256
_CU_TILES = 256
_K_TILE_BYTES = 128


def _prod(values):
    out = 1
    for v in values:
        out *= v
    return out


def _max_offset_bytes(op, field, rows, elem_size):
    axes = list(op.batch) + list(rows) + list(op.k)
    return sum((a.size - 1) * abs(getattr(a, field)) for a in axes if a.size > 0) * elem_size


def _rows_contiguous_ok(op, field, rows, elem_size):
    """contract_pipe's test for an operand contiguous along its rows (its other
    conditions, K tiles and 32-bit offsets, are checked by the caller)."""
    vec = 16 // elem_size
    if getattr(rows[-1], field) != 1 or rows[-1].size % vec:
        return False
    others = list(op.batch) + list(rows[:-1]) + list(op.k)
    return all(getattr(a, field) % vec == 0 for a in others)


def _repack_for_k_contiguity(op, order, elem_size):
    if elem_size != 2 or not op.k or not op.m or not op.n:
        return op, ()
    tiles = _prod(a.size for a in op.batch)
    tiles *= -(-_prod(a.size for a in op.m) // _BIG_TILE) * -(-_prod(a.size for a in op.n) // _BIG_TILE)
    if tiles < _CU_TILES:
        return op, ()
    k_tile = _K_TILE_BYTES // elem_size
    off32 = all(_max_offset_bytes(op, f, r, elem_size) + 16 < 1 << 32 for f, r in (("a", op.m), ("b", op.n)))
    repack = []
    for field, rows, index in (("a", op.m, order[0]), ("b", op.n, order[1])):
        k_ok = getattr(op.k[-1], field) == 1 and op.k[-1].size % k_tile == 0
        rows_inner = getattr(rows[-1], field) == 1
        if k_ok or not rows_inner:
            continue
        if off32 and op.k[-1].size % k_tile == 0 and _rows_contiguous_ok(op, field, rows, elem_size):
            continue  # read in place through transposing LDS reads
        axes = list(op.batch) + list(rows) + list(op.k)
        if len(axes) > MAX_AXES:
            continue
        shape = tuple(a.size for a in axes)
        dense = dense_strides(shape)
        desc = GatherDesc()
        desc.elem_size = elem_size
        desc.boundary = 0
        desc.fill_bits = 0
        desc.out_rank = desc.in_rank = len(axes)
        for i, axis in enumerate(axes):
            desc.out_size[i] = desc.in_size[i] = axis.size
            desc.in_stride[i] = getattr(axis, field)
            desc.offset[i] = 0
            desc.pos[i] = i
            desc.win[i] = -1
        repack.append((index, desc, shape))
        nb, nr = len(op.batch), len(rows)

        def restride(group, start, field=field, dense=dense):
            return [replace(axis, **{field: dense[start + i]}) for i, axis in enumerate(group)]

        batch = restride(op.batch, 0)
        new_rows = restride(rows, nb)
        k = restride(op.k, nb + nr)
        op = replace(op, batch=batch, k=k, **({"m": new_rows} if field == "a" else {"n": new_rows}))
    return op, tuple(repack)


# Split-K: a contraction with few output tiles and a long K leaves most CUs idle (a
# weight gradient: out channels x kernel taps, summed over every position of a batch).
# Its outermost K sub-axis is then cut into S parts that run as S more batch entries,
# writing S stacked partial results; one es_reduce (over a leading axis, a fixed order)
# adds them.  Partials are rounded to the output dtype, one rounding more than a
# single pass.
_SPLIT_TILE = 128       # tile edge the count below is taken at
_SPLIT_BELOW = 128      # split when fewer output tiles than this ...
_SPLIT_MIN_K = 8192     # ... and K is at least this long
_SPLIT_TARGET = 256     # aim for this many tiles
_SPLIT_K_PART = 512     # and keep at least this much K in each part


# A 16-bit contraction that contract_pipe can read (both operands K-contiguous or
# contiguous along their rows, 32-bit offsets) but that has fewer than one 256 x 256
# tile per CU runs on 128 x 128 tiles at about half the speed per flop.  It is split
# instead into parts that give the pipelined kernel at least a tile per CU when a
# cycle model says so: per round of tiles, K steps times the cost of one plus a fixed
# prologue and epilogue, and the reduction's bytes.  The constants are measured
# (MI355X, ~2 GHz under MFMA load): a 64-deep K step of a 256 x 256 pipelined tile
# 2,450 cycles, its prologue and epilogue 23,300; a 128 x 128 tile's step 1,750
# cycles (448 us for the 1792 x 4096 x 16384 weight gradient); es_reduce ~2,500 bytes
# per cycle.
_PIPE_STEP = 2450
_PIPE_FIXED = 23300
_T128_STEP = 1750
_T128_FIXED = 6000
_REDUCE_BYTES_PER_CYCLE = 2500
_PIPE_K_PART = 1024     # K per part of a pipelined split: 16 K steps


def _pipe_readable(op, elem_size):
    """The host conditions of contract_pipe for both operands (es_contract.hip: a
    whole number of 64-deep K tiles, each operand K-contiguous or contiguous along its
    rows, at most 4 K sub-axes, every byte offset below 2^32)."""
    k_tile = _K_TILE_BYTES // elem_size
    vec = 16 // elem_size
    if elem_size != 2 or not op.k or len(op.k) > 4 or op.k[-1].size % k_tile:
        return False
    for field, rows in (("a", op.m), ("b", op.n)):
        if _max_offset_bytes(op, field, rows, elem_size) + 16 >= 1 << 32:
            return False
        k_contig = getattr(op.k[-1], field) == 1 and all(
            getattr(a, field) % vec == 0 for a in list(op.batch) + list(rows) + list(op.k[:-1]))
        if not k_contig and not _rows_contiguous_ok(op, field, rows, elem_size):
            return False
    return True


def _rounds(tiles):
    return -(-tiles // _CU_TILES)


def _split_k(op, elem_size=None):
    """(op with a leading split batch axis, partial count) or (op, 1).  ``elem_size``
    2 lets a split target the pipelined kernel."""
    if not op.k or not op.m or not op.n:
        return op, 1
    nb = _prod(a.size for a in op.batch)
    m, n = _prod(a.size for a in op.m), _prod(a.size for a in op.n)
    tiles = nb * -(-m // _SPLIT_TILE) * -(-n // _SPLIT_TILE)
    k_total = _prod(a.size for a in op.k)
    if k_total < _SPLIT_MIN_K:
        return op, 1
    outer = op.k[0]
    divisors = [d for d in range(2, outer.size + 1) if outer.size % d == 0]
    best = 1
    if tiles < _SPLIT_BELOW:
        want = -(-_SPLIT_TARGET // tiles)
        for d in divisors:
            if d <= want and k_total // d >= _SPLIT_K_PART:
                best = d
    inner = 1  # > 1: the outer K sub-axis is cut whole and the next one into `inner` parts
    tiles256 = nb * -(-m // _BIG_TILE) * -(-n // _BIG_TILE)
    if elem_size == 2 and tiles256 < _CU_TILES and _pipe_readable(op, elem_size):
        out_bytes = _prod(op.out_shape) * elem_size
        cost = _rounds(tiles * best) * (k_total // best // 64 * _T128_STEP + _T128_FIXED)
        if best > 1:
            cost += (best + 1) * out_bytes / _REDUCE_BYTES_PER_CYCLE
        # a short outer sub-axis (a batch of 16 positions' rows) also cuts into the next
        cuts = [(d, 1) for d in divisors]
        if len(op.k) > 2:
            second = op.k[1].size
            cuts += [(outer.size * d, d) for d in range(2, second + 1) if second % d == 0]
        for d, d2 in cuts:
            if tiles256 * d < _CU_TILES or k_total // d < _PIPE_K_PART:
                continue
            if len(op.k) == 1 and (outer.size // d) % (_K_TILE_BYTES // elem_size):
                continue  # a cut through the innermost K sub-axis keeps whole K tiles
            c = _rounds(tiles256 * d) * (k_total // d // 64 * _PIPE_STEP + _PIPE_FIXED)
            c += (d + 1) * out_bytes / _REDUCE_BYTES_PER_CYCLE
            if c < cost:
                cost, best, inner = c, d, d2
    if best == 1:
        return op, 1
    out_numel = _prod(op.out_shape)
    out_shape = (best,) + tuple(op.out_shape)
    if inner > 1:
        # part p = i * inner + j: all of outer position i, the j-th run of the next sub-axis
        second = op.k[1]
        rest = second.size // inner
        split = [SubAxis(outer.size, a=outer.a, b=outer.b, c=inner * out_numel, label="split"),
                 SubAxis(inner, a=second.a * rest, b=second.b * rest, c=out_numel, label="split")]
        k = ([SubAxis(rest, a=second.a, b=second.b, label=second.label)] if rest > 1 else []) + list(op.k[2:])
        return replace(op, out_shape=out_shape, batch=split + list(op.batch), k=k), best
    rest = outer.size // best
    split_axis = SubAxis(best, a=outer.a * rest, b=outer.b * rest, c=out_numel, label="split")
    k = ([SubAxis(rest, a=outer.a, b=outer.b, label=outer.label)] if rest > 1 else []) + list(op.k[1:])
    return replace(op, out_shape=out_shape, batch=[split_axis] + list(op.batch), k=k), best


def prepare_op(op, dtype, elem_size, split=True):
    """Build the descriptor of a planner op for operands of ``dtype`` (``split``: a
    contraction with few tiles and a long K may run as split-K)."""
    if isinstance(op, EmptyOp) or any(size == 0 for size in op.out_shape):
        # nothing to compute: an empty output of any dtype, like torch.einsum
        return Prepared(None, None, op.out_shape, (), noop=True)

    if isinstance(op, GatherOp):
        desc = GatherDesc()
        if elem_size not in _ELEM_SIZES:
            raise NotImplementedError(f"einshard: element size {elem_size} is not supported")
        desc.elem_size = elem_size
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
        return Prepared("es_gather", desc, op.out_shape, (0,))

    code = dtype_code(dtype, "einshard")

    if isinstance(op, BcastOp):
        desc = BcastDesc()
        desc.dtype = code
        desc.rank = _set_axes(desc.axes, op.axes, "einshard")
        return Prepared("es_bcast", desc, op.out_shape, (0, 1))

    if isinstance(op, ReduceOp):
        desc = ReduceDesc()
        desc.dtype = code
        desc.has_y = 1 if op.has_y else 0
        desc.n_keep = _set_axes(desc.keep, op.keep, "einshard")
        desc.n_red = _set_axes(desc.red, op.red, "einshard")
        need = int(call("es_reduce_workspace_bytes", ctypes.byref(desc)))
        return Prepared("es_reduce", desc, op.out_shape, (0, 1 if op.has_y else 0), workspace=need)

    if isinstance(op, ContractOp):
        order = (1, 0) if op.swapped else (0, 1)
        op, repack = _repack_for_k_contiguity(op, order, elem_size)
        out_shape = op.out_shape
        parts = 1
        if split:
            op, parts = _split_k(op, elem_size)
        desc = ContractDesc()
        desc.dtype = code
        desc.n_batch = _set_axes(desc.batch, op.batch, "einshard")
        desc.n_m = _set_axes(desc.m, op.m, "einshard")
        desc.n_n = _set_axes(desc.n, op.n, "einshard")
        desc.n_k = _set_axes(desc.k, op.k, "einshard")
        if parts == 1:
            return Prepared("es_contract", desc, out_shape, order, repack=repack)
        numel = _prod(out_shape)
        rdesc = ReduceDesc()
        rdesc.dtype = code
        rdesc.has_y = 0
        rdesc.n_keep = _set_axes(rdesc.keep, [SubAxis(numel, a=1)], "einshard")
        rdesc.n_red = _set_axes(rdesc.red, [SubAxis(parts, a=numel)], "einshard")
        need = int(call("es_reduce_workspace_bytes", ctypes.byref(rdesc)))
        return Prepared("es_contract", desc, out_shape, order, repack=repack, split=(parts, rdesc, need))

    raise TypeError(f"unknown planned op {type(op).__name__}")


def run_op(op, xs, dtype, device):
    """Execute a planner op over operands ``xs`` (one or two tensors)."""
    return launch(prepare_op(op, dtype, xs[0].element_size()), xs, device, dtype)
