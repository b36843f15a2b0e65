"""``einconv``: a halo followed by a convolution, run as one implicit GEMM.

The reference (src/torch_einshard/conv.py:65-210) pads the input with its halo
rule, permutes input and weight into ``F.conv{1,2,3}d``'s layouts and calls the
convolution with padding 0.  Here, on the MI355X kernels:

1. one es_gather writes the padded input ``xp`` as (batch axes..., spatial
   axes..., channel): the halo, with the reference's boundary rules, and the
   permutation in one pass (halo.py of this package);
2. one es_gather copies the weight to (out channel, kernel axes..., channel);
3. one es_contract (es_contract_bias with a bias) computes

       out[m..., o] = bias[o] + sum_{k..., c} xp[m_batch..., m_s + d * k..., c] * w[o, k..., c]

   reading ``xp`` in place through an overlapping strided view: the spatial
   axes of M and the kernel axes of K both step through xp's spatial strides
   (K's scaled by the dilation d).  No im2col copy exists; the contraction walks
   K = (kernel..., channel) with additions only.

Backward (same kernels): the bias gradient sums the output gradient; the weight
gradient contracts the output gradient with the same strided view of ``xp``;
the gradient of ``xp`` is the same implicit GEMM of the output gradient, padded
by d * (K - 1) on each side, with the weight flipped along its kernel axes and
its two channel axes exchanged; the two gathers' adjoints carry the gradients
back to ``x`` and ``weight``.

Validation order and messages follow conv.py:86-180.
"""

import torch
from torch.utils.checkpoint import checkpoint as torch_checkpoint

from ._cache import call_key, lookup, remember
from ._exec import check_device_tensors, launch, prepare_op
from .autograd import _gather_into, _sum_dims, differentiable_gather, needs_grad
from .families import cached_expand_axis_families, expand_family_mapping
from .grammar import parse_sharding
from .halo import _check_padding, _normalize_halo, _prepare
from .planner import ContractOp, SubAxis, _merge, dense_strides
from .sharding import EllipsisAxis

__all__ = ["einconv"]


def _axes(spec):
    return spec.axes if hasattr(spec, "axes") else spec


def _axis_names(axes, *, label):
    names = []
    for axis in axes:
        if isinstance(axis, EllipsisAxis):
            raise NotImplementedError(f"einconv does not support ellipsis axes in {label}")
        if not hasattr(axis, "name"):
            raise NotImplementedError(f"einconv does not support factored axes in {label}")
        if axis.name in names:
            raise ValueError(f"Axis {axis.name!r} appears more than once in {label}")
        names.append(axis.name)
    return names


def _per_axis(value, ndim, *, label):
    if isinstance(value, int):
        return (value,) * ndim
    values = tuple(value)
    if len(values) != ndim:
        raise ValueError(f"{label} must have {ndim} values")
    return values


def _default_padding(weight, kernel_dims, dilation):
    """Half the effective kernel (d * (K - 1)) on each side; it must be even."""
    padding = []
    for dim, dil in zip(kernel_dims, dilation):
        reach = dil * (weight.shape[dim] - 1)
        if reach % 2:
            raise ValueError("Default einconv padding requires odd effective kernel sizes")
        padding.append(reach // 2)
    return tuple(padding)


def _checkpoint(function, tensors, mode, use_reentrant):
    if mode in (False, None, "none"):
        return function(*tensors)
    if mode in (True, "full", "conv"):
        return torch_checkpoint(function, *tensors, use_reentrant=use_reentrant)
    raise ValueError("checkpoint must be one of 'full', 'conv', 'none', True, or False")


# ---- the implicit GEMM --------------------------------------------------------------


def _conv_op(xp, wk, dilation, out_order):
    """The contraction of a padded input ``xp`` = (batch..., spatial..., channel) with a
    weight ``wk`` = (out channel, kernel..., channel).  Conv output dims (batch...,
    spatial..., out channel) are written dense in ``out_order`` (a permutation of
    them).  Returns (ContractOp, output shape)."""
    ns = len(dilation)
    nb = xp.dim() - ns - 1
    kernel = wk.shape[1 : 1 + ns]
    conv_shape = list(xp.shape[:nb])
    conv_shape += [xp.shape[nb + j] - dilation[j] * (kernel[j] - 1) for j in range(ns)]
    conv_shape.append(wk.shape[0])
    out_shape = tuple(conv_shape[d] for d in out_order)
    out_strides = dense_strides(out_shape)
    c_stride = {d: out_strides[i] for i, d in enumerate(out_order)}
    o_dim = nb + ns
    m = [SubAxis(conv_shape[d], a=xp.stride(d), c=c_stride[d]) for d in out_order if d != o_dim]
    n = [SubAxis(conv_shape[o_dim], b=wk.stride(0), c=c_stride[o_dim])]
    k = [SubAxis(kernel[j], a=dilation[j] * xp.stride(nb + j), b=wk.stride(1 + j)) for j in range(ns)]
    k.append(SubAxis(xp.shape[-1], a=xp.stride(-1), b=wk.stride(-1)))
    op = ContractOp(out_shape, swapped=False, m=_merge(m, ("a", "c")), n=n, k=_merge(k, ("a", "b")))
    return op, out_shape


def _conv_prepare(xp, wk, dilation, out_order, bias=False):
    """The prepared contraction of one implicit-GEMM convolution (with a bias it never
    runs as split-K: every partial would add it)."""
    op, _ = _conv_op(xp, wk, dilation, out_order)
    return prepare_op(op, xp.dtype, xp.element_size(), split=not bias)


def _conv_launch(prep, xp, wk, bias):
    if bias is not None and bias.stride(0) != 1:
        bias = bias.contiguous()
    return launch(prep, (xp, wk), xp.device, xp.dtype, bias=bias)


def _conv(xp, wk, bias, dilation, out_order):
    """Run one implicit-GEMM convolution (no autograd)."""
    check_device_tensors([xp, wk] + ([] if bias is None else [bias]), what="einconv")
    return _conv_launch(_conv_prepare(xp, wk, dilation, out_order, bias is not None), xp, wk, bias)


def _weight_grad(gz, xp, dilation, out_order, w_shape):
    """dL/dw[o, k..., c] = sum_m gz[m, o] * xp[m + d * k, c]: one contraction with
    M = out channel, N = (kernel..., channel) over the strided view of xp, K = the
    conv output's batch and spatial dims."""
    ns = len(dilation)
    nb = xp.dim() - ns - 1
    o_dim = nb + ns
    pos = {d: i for i, d in enumerate(out_order)}  # conv dim -> gz dim
    w_strides = dense_strides(w_shape)
    m = [SubAxis(w_shape[0], a=gz.stride(pos[o_dim]), c=w_strides[0])]
    n = [SubAxis(w_shape[1 + j], b=dilation[j] * xp.stride(nb + j), c=w_strides[1 + j]) for j in range(ns)]
    n.append(SubAxis(w_shape[-1], b=xp.stride(-1), c=w_strides[-1]))
    k = [SubAxis(gz.shape[pos[d]], a=gz.stride(pos[d]), b=xp.stride(d)) for d in range(o_dim)]
    op = ContractOp(tuple(w_shape), swapped=False, m=m, n=_merge(n, ("b", "c")), k=_merge(k, ("a", "b")))
    device, dtype = check_device_tensors([gz, xp], what="einconv backward")
    return launch(prepare_op(op, dtype, gz.element_size()), (gz, xp), device, dtype)


def _input_grad(gz, wk, dilation, out_order, xp_shape):
    """dL/dxp: gz padded by d * (K - 1) on both sides of every spatial dim, as
    (batch..., spatial..., out channel), convolved with the weight flipped along its
    kernel dims and with its channel dims exchanged, (channel, kernel..., out channel)."""
    ns = len(dilation)
    nb = len(xp_shape) - ns - 1
    o_dim = nb + ns
    kernel = wk.shape[1 : 1 + ns]
    reach = [dilation[j] * (kernel[j] - 1) for j in range(ns)]
    pos = {d: i for i, d in enumerate(out_order)}
    gpad_shape = [gz.shape[pos[d]] for d in range(nb)]
    gpad_shape += [gz.shape[pos[nb + j]] + 2 * reach[j] for j in range(ns)]
    gpad_shape.append(gz.shape[pos[o_dim]])
    src = []
    for i in range(gz.dim()):
        d = out_order[i]
        offset = -reach[d - nb] if nb <= d < o_dim else 0
        src.append((gz.shape[i], gz.stride(i), d, -1, offset))
    gpad = _gather_into(gz.data_ptr(), gz.dtype, gz.device, tuple(gpad_shape), src)
    base = wk.data_ptr()
    src = [(wk.shape[0], wk.stride(0), 1 + ns, -1, 0)]
    for j in range(ns):
        base += (kernel[j] - 1) * wk.stride(1 + j) * wk.element_size()
        src.append((kernel[j], -wk.stride(1 + j), 1 + j, -1, 0))
    src.append((wk.shape[-1], wk.stride(-1), 0, -1, 0))
    wflip_shape = (wk.shape[-1], *kernel, wk.shape[0])
    wflip = _gather_into(base, wk.dtype, wk.device, wflip_shape, src)
    return _conv(gpad, wflip, None, dilation, tuple(range(len(xp_shape))))


class _ConvFn(torch.autograd.Function):
    """The implicit-GEMM convolution with its adjoints as backward."""

    @staticmethod
    def forward(ctx, geometry, xp, wk, bias):
        dilation, out_order = geometry
        ctx.geometry = geometry
        ctx.has_bias = bias is not None
        ctx.save_for_backward(xp, wk)
        return _conv(xp, wk, bias, dilation, out_order)

    @staticmethod
    def backward(ctx, gz):
        dilation, out_order = ctx.geometry
        xp, wk = ctx.saved_tensors
        grad_xp = grad_wk = grad_bias = None
        if ctx.needs_input_grad[1]:
            grad_xp = _input_grad(gz, wk, dilation, out_order, tuple(xp.shape))
        if ctx.needs_input_grad[2]:
            grad_wk = _weight_grad(gz, xp, dilation, out_order, tuple(wk.shape))
        if ctx.has_bias and ctx.needs_input_grad[3]:
            o_pos = out_order.index(xp.dim() - 1)
            grad_bias = _sum_dims(gz, [o_pos], [i for i in range(gz.dim()) if i != o_pos])
        return None, grad_xp, grad_wk, grad_bias


def _gather_run(prep, t, out_shape, dims, boundary):
    """One prepared es_gather (differentiable when ``t`` requires grad)."""
    if needs_grad([t]):
        return differentiable_gather(prep, t, out_shape, dims, boundary)
    return launch(prep, (t,), t.device, t.dtype)


def _replay(plan, x, weight, bias):
    """A cached no-grad call: the two gathers and the contraction, prepared."""
    prep_x, prep_w, prep_c = plan
    xp = launch(prep_x, (x,), x.device, x.dtype)
    wk = launch(prep_w, (weight,), weight.device, weight.dtype)
    return _conv_launch(prep_c, xp, wk, bias)


_MODES = (False, None, "none", True, "full", "conv")


# ---- the public entry ---------------------------------------------------------------


def einconv(
    shard,
    x,
    weight,
    windows,
    *,
    bias=None,
    padding=None,
    stride=1,
    dilation=1,
    groups=1,
    boundary="constant",
    fill=0,
    mesh=None,
    shapes=None,
    families=None,
    checkpoint="full",
    use_reentrant=False,
):
    """Halo ``x`` along the window source axes, then convolve it with ``weight``.

    ``windows`` maps each spatial input axis to its weight kernel axis; the output is
    the input's axes with the channel axis replaced by the weight's output channel
    axis.  Stride 1 and groups=1, like the reference.

    A call with no tensor requiring grad runs without checkpointing (there is
    nothing to recompute) and caches its prepared launches; later calls with the
    same arguments and operand geometry replay them."""
    tensors = (x, weight) if bias is None else (x, weight, bias)
    grad = needs_grad(tensors)
    key = None
    if not grad:
        key = call_key(
            "einconv", tensors, mesh, shapes, shard, windows, padding, stride, dilation, groups, boundary, fill,
            families, checkpoint, use_reentrant,
        )
        plan = lookup(key)
        if plan is not None:
            return _replay(plan, x, weight, bias)
    shard, _ = cached_expand_axis_families(shard, families=families)
    windows = expand_family_mapping(windows, families, label="Window")
    input_spec, weight_spec, output_spec = parse_sharding(shard)
    if weight_spec is None:
        raise ValueError("einconv expects a binary sharding expression")
    if input_spec.partials or weight_spec.partials or output_spec.partials:
        raise ValueError("einconv does not support partial tensor specs")
    if groups != 1:
        raise NotImplementedError("einconv currently supports only groups=1")

    input_axes = _axes(input_spec)
    weight_axes = _axes(weight_spec)
    output_axes = _axes(output_spec)
    input_names = _axis_names(input_axes, label="input")
    weight_names = _axis_names(weight_axes, label="weight")
    output_names = _axis_names(output_axes, label="output")

    spatial = list(windows)
    kernels = list(windows.values())
    if len(spatial) not in (1, 2, 3):
        raise ValueError("einconv supports 1D, 2D, and 3D convolutions")
    if len(set(kernels)) != len(kernels):
        raise ValueError("Window axes must be distinct")
    absent = [name for name in spatial if name not in input_names]
    if absent:
        raise ValueError(f"Window source axis {absent[0]!r} is not present in the input")
    absent = [name for name in kernels if name not in weight_names]
    if absent:
        raise ValueError(f"Window axis {absent[0]!r} is not present in the weight")
    if any(name in input_names or name in output_names for name in kernels):
        raise ValueError("Window axes must be weight-only axes")
    if any(not axis.local() for axis in weight_axes):
        raise ValueError("einconv weight axes must be local")

    output_by_name = {axis.name: axis for axis in output_axes}
    if any(axis.name in output_by_name and output_by_name[axis.name] != axis for axis in input_axes):
        raise ValueError("einconv output must preserve input axis sharding")

    shared = [name for name in input_names if name in weight_names and name not in spatial]
    channels = [name for name in shared if name not in output_names]
    if len(channels) != 1:
        raise ValueError("einconv expects exactly one input channel axis")
    channel = channels[0]
    if not input_axes[input_names.index(channel)].local():
        raise ValueError("einconv input channel axis must be local")

    out_channels = [name for name in weight_names if name in output_names and name not in input_names]
    if len(out_channels) != 1:
        raise ValueError("einconv expects exactly one output channel axis")
    out_channel = out_channels[0]
    if not output_by_name[out_channel].local():
        raise ValueError("einconv output channel axis must be local")

    unexpected = [name for name in weight_names if name not in {out_channel, channel, *kernels}]
    if unexpected:
        raise ValueError(f"Unexpected weight axis {unexpected[0]!r}")
    if set(output_names) != (set(input_names) - {channel}) | {out_channel}:
        raise ValueError("einconv output axes must be input axes with the channel axis replaced by the output channel axis")

    ndim = len(spatial)
    stride = _per_axis(stride, ndim, label="stride")
    dilation = _per_axis(dilation, ndim, label="dilation")
    if any(value != 1 for value in stride):
        raise NotImplementedError("einconv currently supports only stride=1")

    kernel_dims = tuple(weight_names.index(name) for name in kernels)
    if padding is None:
        pads = _default_padding(weight, kernel_dims, dilation)
    else:
        pads = expand_family_mapping(padding, families, label="Padding")
        if isinstance(pads, dict):
            unknown = set(pads) - set(spatial)
            if unknown:
                raise ValueError(f"Padding axis {sorted(unknown)[0]!r} has no matching window")
            absent = [name for name in spatial if name not in pads]
            if absent:
                raise ValueError(f"Missing padding for window source axis {absent[0]!r}")
            pads = tuple(pads[name] for name in spatial)
        else:
            pads = _per_axis(pads, ndim, label="padding")
    for name, value, kernel_dim, dil in zip(spatial, pads, kernel_dims, dilation):
        left, right = _normalize_halo(value)
        expected = dil * (weight.shape[kernel_dim] - 1)
        if left + right != expected:
            raise ValueError(
                f"Padding for axis {name!r} must preserve the spatial length; "
                f"got left + right = {left + right}, expected {expected}"
            )
    halos = dict(zip(spatial, pads))

    batch = [name for name in input_names if name not in spatial and name != channel]
    conv_names = batch + spatial + [out_channel]
    out_order = tuple(conv_names.index(name) for name in output_names)
    geometry = (tuple(dilation), out_order)

    def _check_shapes(x_arg, w_arg, bias_arg):
        # what F.conv{1,2,3}d rejects; the kernels read exactly these extents
        if x_arg.dim() != len(input_axes):
            raise ValueError(f"einconv: spec has {len(input_axes)} axes but the input has {x_arg.dim()} dims")
        if w_arg.dim() != len(weight_axes):
            raise ValueError(f"einconv: spec has {len(weight_axes)} weight axes but the weight has {w_arg.dim()} dims")
        channels = x_arg.shape[input_names.index(channel)]
        if w_arg.shape[weight_names.index(channel)] != channels:
            raise RuntimeError(
                f"einconv: weight of size {list(w_arg.shape)} expects {w_arg.shape[weight_names.index(channel)]} "
                f"channels along {channel!r}, but the input has {channels}"
            )
        outs = w_arg.shape[weight_names.index(out_channel)]
        if bias_arg is not None and tuple(bias_arg.shape) != (outs,):
            raise RuntimeError(f"einconv: bias of shape {list(bias_arg.shape)} does not match {outs} output channels")

    def pad_plan(x_arg):
        # halo + permutation to (batch..., spatial..., channel) in one gather
        _check_padding(x_arg, input_axes, halos, mesh=mesh, boundary=boundary)
        if x_arg.dim() != len(input_axes):
            raise ValueError(f"einconv: spec has {len(input_axes)} axes but the input has {x_arg.dim()} dims")
        canon = batch + spatial + [channel]
        out_shape = [0] * len(canon)
        dims = []
        for dim, name in enumerate(input_names):
            left, right = _normalize_halo(halos[name]) if name in halos else (0, 0)
            out_shape[canon.index(name)] = x_arg.shape[dim] + left + right
            dims.append((canon.index(name), -1, -left))
        prep, _, _ = _prepare(x_arg, tuple(out_shape), dims, boundary=boundary, fill=fill)
        return prep, out_shape, dims

    def weight_plan(w_arg):
        # (out channel, kernel..., channel): both operands K-contiguous
        canon = [out_channel] + kernels + [channel]
        out_shape = [w_arg.shape[weight_names.index(name)] for name in canon]
        dims = [(canon.index(name), -1, 0) for name in weight_names]
        prep, _, _ = _prepare(w_arg, tuple(out_shape), dims, boundary="constant", fill=0)
        return prep, out_shape, dims

    def operands(x_arg, w_arg, bias_arg):
        check_device_tensors([x_arg, w_arg] + ([] if bias_arg is None else [bias_arg]), what="einconv")
        px = pad_plan(x_arg)
        _check_shapes(x_arg, w_arg, bias_arg)
        pw = weight_plan(w_arg)
        xp = _gather_run(px[0], x_arg, px[1], px[2], boundary)
        wk = _gather_run(pw[0], w_arg, pw[1], pw[2], "constant")
        return xp, wk, px[0], pw[0]

    def run_conv(xp, wk, bias_arg=None):
        if needs_grad([xp, wk, bias_arg]):
            return _ConvFn.apply(geometry, xp, wk, bias_arg)
        return _conv(xp, wk, bias_arg, geometry[0], geometry[1])

    def run_full(x_arg, w_arg, *optional_bias):
        bias_arg = optional_bias[0] if optional_bias else None
        xp, wk, _, _ = operands(x_arg, w_arg, bias_arg)
        if checkpoint == "conv":
            tensors = (xp, wk) if bias_arg is None else (xp, wk, bias_arg)
            return _checkpoint(run_conv, tensors, "conv", use_reentrant)
        return run_conv(xp, wk, bias_arg)

    if not grad:
        if checkpoint not in _MODES:
            raise ValueError("checkpoint must be one of 'full', 'conv', 'none', True, or False")
        xp, wk, prep_x, prep_w = operands(x, weight, bias)
        prep_c = _conv_prepare(xp, wk, geometry[0], geometry[1], bias is not None)
        out = _conv_launch(prep_c, xp, wk, bias)
        if key is not None:
            remember(key, (prep_x, prep_w, prep_c))
        return out
    if checkpoint == "conv":
        return run_full(*tensors)
    return _checkpoint(run_full, tensors, checkpoint, use_reentrant)
