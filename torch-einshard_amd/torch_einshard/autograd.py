"""Backward passes of the local einshard / einwindow / einhalo paths.

The reference's outputs are differentiable because ``torch.einsum``, ``F.pad``,
``unfold`` and ``permute`` are (src/torch_einshard/einsum.py:132,
halo.py:27-55, 402-418).  Here the forward runs on the MI355X kernels, so the
gradients are planned onto the same kernels:

* einsum: for operand i with labels D_i, the gradient is the einsum of the
  output gradient (labels E) with the other operand, producing the labels of
  D_i that appear in E or in the other operand — one es_contract / es_reduce /
  es_bcast / es_gather launch.  Labels only operand i carries were summed in the
  forward, so the gradient is constant along them (an expanded view); labels
  operand i broadcast from size 1 are summed away and kept as size 1; repeated
  labels (a diagonal) write the gradient onto the diagonal of a zero tensor.
* window / halo: the adjoint of the gather ``out[o] = x[resolve(o[pos] +
  o[win] + offset)]`` (see halo.py of this package), computed deterministically
  by a gather of the output gradient followed by a sum — no atomics, a fixed
  summation order.
"""

import ctypes

import torch

from . import _native
from ._exec import check_device_tensors, dtype_code, launch, prepare_op
from .planner import ELLIPSIS, lower_einsum

__all__ = ["einsum_labels", "differentiable_einsum", "differentiable_gather", "gather_adjoint", "needs_grad"]


def needs_grad(xs):
    return torch.is_grad_enabled() and any(isinstance(x, torch.Tensor) and x.requires_grad for x in xs)


def einsum_labels(xs, input_labels, output_labels):
    """Evaluate an einsum over explicit label lists on the device kernels (no autograd)."""
    xs = list(xs)
    op = lower_einsum(input_labels, [tuple(x.shape) for x in xs], [tuple(x.stride()) for x in xs], output_labels)
    device, dtype = check_device_tensors(xs)
    return launch(prepare_op(op, dtype, xs[0].element_size()), xs, device, dtype)


def _explicit_labels(input_labels, shapes, output_labels):
    """Replace ``...`` by one label per ellipsis dim, right-aligned like the planner."""
    ranks = []
    for labels, shape in zip(input_labels, shapes):
        named = sum(1 for label in labels if label != ELLIPSIS)
        ranks.append(max(len(shape) - named, 0) if ELLIPSIS in labels else 0)
    total = max(ranks) if ranks else 0

    def expand(labels, rank):
        out = []
        for label in labels:
            if label == ELLIPSIS:
                out.extend(("...", total - rank + j) for j in range(rank))
            else:
                out.append(label)
        return out

    inputs = [expand(labels, rank) for labels, rank in zip(input_labels, ranks)]
    output = expand(output_labels, total)
    return inputs, output


def _operand_grad(gz, out_labels, other, other_labels, labels, shape):
    """Gradient of one operand with dims ``labels`` / ``shape`` (see the module docstring)."""
    size_of = dict(zip(out_labels, gz.shape))
    if other is not None:
        for label, size in zip(other_labels, other.shape):
            if size != 1:
                size_of[label] = size
    unique = []
    own_size = {}
    for label, size in zip(labels, shape):
        if label not in own_size:
            unique.append(label)
            own_size[label] = size
    reachable = set(out_labels) | (set(other_labels) if other is not None else set())
    # labels the einsum produces: reachable and not broadcast from size 1 here
    produced = [
        label for label in unique if label in reachable and not (own_size[label] == 1 and size_of.get(label, 1) != 1)
    ]
    xs = [gz] if other is None else [gz, other]
    in_labels = [list(out_labels)] if other is None else [list(out_labels), list(other_labels)]
    g = einsum_labels(xs, in_labels, produced)
    # insert the dims the einsum did not produce: size 1 (broadcast) or expanded (summed-only)
    full_shape = []
    index = []
    for label in unique:
        if label in produced:
            index.append(label)
            full_shape.append(own_size[label])
        else:
            index.append(None)
            full_shape.append(own_size[label])
    view_shape = [own_size[label] if label is not None else 1 for label in index]
    g = g.reshape(view_shape).expand(full_shape)
    if len(unique) == len(labels):
        return g
    # repeated labels: the gradient lives on the diagonal
    dx = torch.zeros(shape, dtype=g.dtype, device=g.device)
    strides = {}
    for label, stride in zip(labels, dx.stride()):
        strides[label] = strides.get(label, 0) + stride
    diag = dx.as_strided([own_size[label] for label in unique], [strides[label] for label in unique])
    diag.copy_(g)
    return dx


class _EinsumFn(torch.autograd.Function):
    @staticmethod
    def forward(ctx, spec, *xs):
        input_labels, output_labels = spec
        ctx.spec = spec
        ctx.save_for_backward(*xs)
        return einsum_labels(xs, input_labels, output_labels)

    @staticmethod
    def backward(ctx, gz):
        input_labels, output_labels = ctx.spec
        xs = ctx.saved_tensors
        gz = gz.contiguous() if gz.dim() and gz.stride(-1) == 0 else gz
        grads = [None] * len(xs)
        for i, x in enumerate(xs):
            if not ctx.needs_input_grad[i + 1]:
                continue
            other = xs[1 - i] if len(xs) == 2 else None
            other_labels = input_labels[1 - i] if len(xs) == 2 else None
            grads[i] = _operand_grad(gz, output_labels, other, other_labels, input_labels[i], tuple(x.shape))
        return (None, *grads)


def differentiable_einsum(xs, input_labels, output_labels):
    """Einsum over label lists whose result carries a grad_fn when an input requires grad."""
    inputs, output = _explicit_labels(input_labels, [tuple(x.shape) for x in xs], output_labels)
    spec = (tuple(tuple(labels) for labels in inputs), tuple(output))
    return _EinsumFn.apply(spec, *xs)


# ---- window / halo ---------------------------------------------------------------

def _gather_into(src_ptr, dtype, device, out_shape, in_dims, boundary=0, fill_bits=0):
    """One es_gather into a new dense tensor.

    ``in_dims``: per source dim (size, element stride, pos, win, offset) with the
    meaning of es_gather_desc; ``src_ptr`` is the address of source index 0.
    """
    out = torch.empty(out_shape, dtype=dtype, device=device)
    if out.numel() == 0:
        return out
    desc = _native.GatherDesc()
    desc.elem_size = out.element_size()
    desc.boundary = boundary
    desc.fill_bits = fill_bits
    desc.out_rank = len(out_shape)
    for i, size in enumerate(out_shape):
        desc.out_size[i] = size
    desc.in_rank = len(in_dims)
    for j, (size, stride, pos, win, offset) in enumerate(in_dims):
        desc.in_size[j] = size
        desc.in_stride[j] = stride
        desc.pos[j] = pos
        desc.win[j] = win
        desc.offset[j] = offset
    _native.call("es_gather", ctypes.byref(desc), src_ptr, out.data_ptr(), _native.stream_of(out))
    return out


def _sum_dims(x, keep_dims, red_dims):
    """Sum of ``x`` over ``red_dims`` (one es_reduce); the result is dense over ``keep_dims``."""
    out = torch.empty([x.shape[d] for d in keep_dims], dtype=x.dtype, device=x.device)
    if out.numel() == 0:
        return out
    desc = _native.ReduceDesc()
    desc.dtype = dtype_code(x.dtype, "einwindow backward")
    desc.has_y = 0
    desc.n_keep = len(keep_dims)
    for i, d in enumerate(keep_dims):
        desc.keep[i].size, desc.keep[i].a, desc.keep[i].b, desc.keep[i].c = x.shape[d], x.stride(d), 0, 0
    desc.n_red = len(red_dims)
    for i, d in enumerate(red_dims):
        desc.red[i].size, desc.red[i].a, desc.red[i].b, desc.red[i].c = x.shape[d], x.stride(d), 0, 0
    need = int(_native.call("es_reduce_workspace_bytes", ctypes.byref(desc)))
    ws = torch.empty(need, dtype=torch.uint8, device=x.device) if need > 0 else None
    _native.call(
        "es_reduce",
        ctypes.byref(desc),
        x.data_ptr(),
        x.data_ptr(),
        out.data_ptr(),
        ws.data_ptr() if ws is not None else None,
        need,
        _native.stream_of(out),
    )
    return out


def _fold_windows(gz, out_shape, dims):
    """G[.., t_j, ..] = sum_w gz[.., pos_j = t_j - w, .., win_j = w, ..] for every windowed
    input dim j (t_j in [0, P_j + K_j - 1)); other dims pass through.  G has one dim
    per input dim, in input-dim order."""
    rank = len(dims)
    windowed = [j for j, (_, win, _) in enumerate(dims) if win >= 0]
    t_sizes = [out_shape[pos] + (out_shape[win] - 1 if win >= 0 else 0) for pos, win, _ in dims]
    if not windowed:
        # a halo: G is gz read in input-dim order (a strided view, no copy)
        return gz.as_strided(t_sizes, [gz.stride(pos) for pos, _, _ in dims])
    # H[w'_0 .. w'_{k-1}, t_0 .. t_{r-1}] with w' = K - 1 - w: the window axis is read
    # backwards (negative stride from its last element) so that the gz index of
    # pos_j is t_j + w' - (K - 1), a sum of output coordinates.  Window dims lead,
    # so the innermost dim stays the input's innermost (vector gathers).
    nw = len(windowed)
    h_shape = [out_shape[dims[j][1]] for j in windowed] + t_sizes
    w_dim = {j: n for n, j in enumerate(windowed)}
    base = gz.data_ptr()
    src = []
    for d in range(gz.dim()):
        for j, (pos, win, _) in enumerate(dims):
            if d == pos:
                if win >= 0:
                    src.append((gz.shape[d], gz.stride(d), nw + j, w_dim[j], -(out_shape[win] - 1)))
                else:
                    src.append((gz.shape[d], gz.stride(d), nw + j, -1, 0))
                break
            if d == win:
                base += (gz.shape[d] - 1) * gz.stride(d) * gz.element_size()
                src.append((gz.shape[d], -gz.stride(d), w_dim[j], -1, 0))
                break
    h = _gather_into(base, gz.dtype, gz.device, h_shape, src)
    return _sum_dims(h, list(range(nw, nw + rank)), list(range(nw)))


def _edge_sum(v, j):
    """Sum of ``v`` over dim ``j``, kept as a size-1 dim."""
    keep = [d for d in range(v.dim()) if d != j]
    return _sum_dims(v, keep, [j]).unsqueeze(j)


def gather_adjoint(gz, x_shape, out_shape, dims, boundary):
    """Gradient of the window / halo gather with respect to its input.

    ``dims``: per input dim (pos, win, offset) as in es_gather_desc; ``boundary``:
    "constant", "replicate" or "periodic".  The forward reads input index
    resolve(t + offset) for padded coordinate t = o[pos] + o[win]."""
    g = _fold_windows(gz, out_shape, dims)
    rank = len(dims)
    offsets = [offset for _, _, offset in dims]
    x_shape = tuple(x_shape)
    if boundary == "periodic":
        # pad every dim to whole periods aligned so that q = t + a, a = offset mod n,
        # satisfies q = t + offset (mod n); then sum the periods
        pad_sizes, src = [], []
        for j in range(rank):
            n = x_shape[j]
            a = offsets[j] % n
            periods = -(-(g.shape[j] + a) // n)
            pad_sizes.append(periods * n)
            src.append((g.shape[j], g.stride(j), j, -1, -a))
        padded = _gather_into(g.data_ptr(), g.dtype, g.device, pad_sizes, src)
        split = []
        for j in range(rank):
            split.extend([pad_sizes[j] // x_shape[j], x_shape[j]])
        return _sum_dims(padded.view(split), [2 * j + 1 for j in range(rank)], [2 * j for j in range(rank)])
    if boundary == "constant":
        src = [(g.shape[j], g.stride(j), j, -1, -offsets[j]) for j in range(rank)]
        return _gather_into(g.data_ptr(), g.dtype, g.device, x_shape, src)
    # replicate: resolve one dim at a time; positions clamped onto the first / last
    # index add their sum there
    c = g
    for j in range(rank):
        n, t_size, offset = x_shape[j], c.shape[j], offsets[j]
        shape = list(c.shape)
        shape[j] = n
        src = [(c.shape[d], c.stride(d), d, -1, -offset if d == j else 0) for d in range(rank)]
        r = _gather_into(c.data_ptr(), c.dtype, c.device, tuple(shape), src)
        left = min(-offset, t_size)  # t < -offset: input index below 0
        if left > 0:
            r.narrow(j, 0, 1).add_(_edge_sum(c.narrow(j, 0, left), j))
        start = max(n - offset, 0)  # t >= n - offset: input index above n - 1
        if start < t_size:
            r.narrow(j, n - 1, 1).add_(_edge_sum(c.narrow(j, start, t_size - start), j))
        c = r
    return c


class _GatherFn(torch.autograd.Function):
    """The window / halo gather with its adjoint as backward."""

    @staticmethod
    def forward(ctx, geometry, prep, x):
        out_shape, dims, boundary = geometry
        ctx.geometry = geometry
        ctx.x_shape = tuple(x.shape)
        return launch(prep, (x,), x.device, x.dtype)

    @staticmethod
    def backward(ctx, gz):
        out_shape, dims, boundary = ctx.geometry
        return None, None, gather_adjoint(gz, ctx.x_shape, out_shape, dims, boundary)


def differentiable_gather(prep, x, out_shape, dims, boundary):
    """Run a prepared window / halo gather; the result carries a grad_fn when x requires grad."""
    geometry = (tuple(out_shape), tuple(tuple(d) for d in dims), boundary)
    return _GatherFn.apply(geometry, prep, x)
