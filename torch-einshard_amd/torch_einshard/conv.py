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

With zero padding and no gradient to record, step 1 is skipped: es_contract_halo
reads the unpadded input through the same view, positions outside it as zeros.

Backward (same kernels): the bias gradient sums the output gradient; the weight
gradient contracts the output gradient with the same strided view of ``xp``;
the gradient of ``xp`` is the same implicit GEMM of the output gradient, padded
by d * (K - 1) on each side with zeros (read in place by es_contract_halo where
it applies), with the weight flipped along its kernel axes and its two channel
axes exchanged; the two gathers' adjoints carry the gradients back to ``x`` and
``weight``.

Validation order and messages follow conv.py:86-180.
"""

import torch
from torch.utils.checkpoint import checkpoint as torch_checkpoint

from ._cache import call_key, lookup, remember
from ._exec import check_device_tensors, fill_bits, launch, prepare_halo, prepare_op
from ._native import ES_ERR_UNSUPPORTED, MAX_AXES, HaloDesc, NativeError
from .autograd import _gather_into, _sum_dims, differentiable_gather, needs_grad
from .families import cached_expand_axis_families, expand_family_mapping
from .grammar import parse_sharding
from .halo import _check_padding, _normalize_halo, _prepare
from .planner import ContractOp, SubAxis, _merge, dense_strides
from .sharding import AxisGroup, EllipsisAxis

__all__ = ["einconv"]


class _Roles:
    """What every named axis of an einconv expression is.

    ``inputs`` / ``weights`` / ``outputs`` map each operand's axis names, in order, to
    their Axis; ``spatial`` are the window source axes of the input and ``kernels`` the
    matching weight axes; ``channel`` is the one contracted input axis, ``out_channel``
    the one weight axis that replaces it in the output; ``batch`` the other input
    axes, in input order."""

    __slots__ = ("inputs", "weights", "outputs", "spatial", "kernels", "channel", "out_channel", "batch")


def _conv_specs(shard, windows, groups, families):
    """The three parsed specs and the family-expanded windows, after the reference's
    first checks (conv.py:84-92): two inputs, no partials, groups=1."""
    text, _ = cached_expand_axis_families(shard, families=families)
    windows = expand_family_mapping(windows, families, label="Window")
    specs = parse_sharding(text)
    if specs[1] is None:
        raise ValueError("einconv expects a binary sharding expression")
    if any(spec.partials for spec in specs):
        raise ValueError("einconv does not support partial tensor specs")
    if groups != 1:
        raise NotImplementedError("einconv currently supports only groups=1")
    return specs, windows


def _named_axes(spec, label):
    """{name: Axis} of one operand; einconv takes plain, distinct axes only."""
    named = {}
    for axis in spec.axes:
        if isinstance(axis, EllipsisAxis):
            raise NotImplementedError(f"einconv does not support ellipsis axes in {label}")
        if isinstance(axis, AxisGroup):
            raise NotImplementedError(f"einconv does not support factored axes in {label}")
        if axis.name in named:
            raise ValueError(f"Axis {axis.name!r} appears more than once in {label}")
        named[axis.name] = axis
    return named


def _the_one(names, what):
    if len(names) != 1:
        raise ValueError(f"einconv expects exactly one {what} axis")
    return names[0]


def _conv_roles(input_spec, weight_spec, output_spec, windows):
    """Classify the axes, raising the reference's errors in its order
    (src/torch_einshard/conv.py:86-147)."""
    roles = _Roles()
    roles.inputs = inputs = _named_axes(input_spec, "input")
    roles.weights = weights = _named_axes(weight_spec, "weight")
    roles.outputs = outputs = _named_axes(output_spec, "output")
    roles.spatial, roles.kernels = list(windows), list(windows.values())
    if not 1 <= len(roles.spatial) <= 3:
        raise ValueError("einconv supports 1D, 2D, and 3D convolutions")
    if len(set(roles.kernels)) < len(roles.kernels):
        raise ValueError("Window axes must be distinct")
    for name in roles.spatial:
        if name not in inputs:
            raise ValueError(f"Window source axis {name!r} is not present in the input")
    for name in roles.kernels:
        if name not in weights:
            raise ValueError(f"Window axis {name!r} is not present in the weight")
    if any(name in inputs or name in outputs for name in roles.kernels):
        raise ValueError("Window axes must be weight-only axes")
    if not all(axis.local() for axis in weights.values()):
        raise ValueError("einconv weight axes must be local")
    if any(name in outputs and outputs[name] != axis for name, axis in inputs.items()):
        raise ValueError("einconv output must preserve input axis sharding")
    roles.channel = _the_one(
        [n for n in inputs if n in weights and n not in windows and n not in outputs], "input channel")
    if not inputs[roles.channel].local():
        raise ValueError("einconv input channel axis must be local")
    roles.out_channel = _the_one([n for n in weights if n in outputs and n not in inputs], "output channel")
    if not outputs[roles.out_channel].local():
        raise ValueError("einconv output channel axis must be local")
    known = {roles.channel, roles.out_channel, *roles.kernels}
    for name in weights:
        if name not in known:
            raise ValueError(f"Unexpected weight axis {name!r}")
    if set(outputs) != (set(inputs) - {roles.channel}) | {roles.out_channel}:
        raise ValueError(
            "einconv output axes must be input axes with the channel axis replaced by the output channel axis")
    roles.batch = [n for n in inputs if n not in windows and n != roles.channel]
    return roles


def _per_axis(value, ndim, label):
    """An int for every spatial axis, or one value per spatial axis."""
    values = (value,) * ndim if isinstance(value, int) else tuple(value)
    if len(values) != ndim:
        raise ValueError(f"{label} must have {ndim} values")
    return values


def _conv_halos(padding, families, roles, weight, dilation):
    """{spatial axis: padding} after the reference's checks (conv.py:155-180): the
    default is half the effective kernel d * (K - 1) on each side (which must then be
    even); a mapping must name exactly the window source axes; every axis's left +
    right must equal d * (K - 1), so the output keeps the input's spatial length."""
    kernel_dims = [list(roles.weights).index(k) for k in roles.kernels]

    def reach(i):
        return dilation[i] * (weight.shape[kernel_dims[i]] - 1)

    ndim = len(roles.spatial)
    if padding is None:
        if any(reach(i) % 2 for i in range(ndim)):
            raise ValueError("Default einconv padding requires odd effective kernel sizes")
        values = tuple(reach(i) // 2 for i in range(ndim))
    else:
        given = expand_family_mapping(padding, families, label="Padding")
        if isinstance(given, dict):
            stray = sorted(set(given) - set(roles.spatial))
            if stray:
                raise ValueError(f"Padding axis {stray[0]!r} has no matching window")
            for name in roles.spatial:
                if name not in given:
                    raise ValueError(f"Missing padding for window source axis {name!r}")
            values = tuple(given[name] for name in roles.spatial)
        else:
            values = _per_axis(given, ndim, "padding")
    for i, (name, value) in enumerate(zip(roles.spatial, values)):
        total = sum(_normalize_halo(value))
        if total != reach(i):
            raise ValueError(
                f"Padding for axis {name!r} must preserve the spatial length; "
                f"got left + right = {total}, expected {reach(i)}"
            )
    return dict(zip(roles.spatial, values))


_RUN_DIRECTLY = (False, None, "none")
_RECOMPUTE = (True, "full", "conv")


def _checkpoint(function, tensors, mode, use_reentrant):
    """``function(*tensors)``, under activation checkpointing for the recompute modes."""
    if mode in _RECOMPUTE:
        return torch_checkpoint(function, *tensors, use_reentrant=use_reentrant)
    if mode in _RUN_DIRECTLY:
        return function(*tensors)
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


def _halo_prepare(x, wk, xdims, pads, dilation, out_order):
    """The prepared es_contract_halo of a convolution read straight from the unpadded
    input ``x`` (zero padding), or None when it does not apply.  ``xdims`` are x's dims
    of (batch..., spatial..., channel), ``pads`` the (left, right) zero padding of each
    spatial dim, ``wk`` the weight as (out channel, kernel..., channel).  The
    contraction's M sub-axes are the output positions and its K sub-axes the taps then
    the channel, unmerged: the kernel reads positions and taps from them."""
    ns = len(dilation)
    nb = len(xdims) - ns - 1
    o_dim = nb + ns
    cdim = xdims[-1]
    if x.stride(cdim) != 1 or x.shape[cdim] == 0 or ns not in (1, 2):
        return None
    kernel = wk.shape[1 : 1 + ns]
    conv_shape = [x.shape[xdims[d]] for d in range(nb)]
    conv_shape += [x.shape[xdims[nb + j]] + sum(pads[j]) - dilation[j] * (kernel[j] - 1) for j in range(ns)]
    conv_shape.append(wk.shape[0])
    if min(conv_shape) <= 0 or len(conv_shape) - 1 > MAX_AXES:
        return None
    out_shape = tuple(conv_shape[d] for d in out_order)
    out_strides = dense_strides(out_shape)
    c_stride = {d: out_strides[i] for i, d in enumerate(out_order)}
    m_dims = [d for d in out_order if d != o_dim]
    m = [SubAxis(conv_shape[d], a=x.stride(xdims[d]), c=c_stride[d]) for d in m_dims]
    n = [SubAxis(conv_shape[o_dim], b=wk.stride(0), c=c_stride[o_dim])]
    k = [SubAxis(kernel[j], a=dilation[j] * x.stride(xdims[nb + j]), b=wk.stride(1 + j)) for j in range(ns)]
    k.append(SubAxis(x.shape[cdim], a=1, b=wk.stride(-1)))
    halo = HaloDesc()
    halo.n = ns
    for j in range(ns):
        halo.dim[j].m_axis = m_dims.index(nb + j)
        halo.dim[j].extent = x.shape[xdims[nb + j]]
        halo.dim[j].dilation = dilation[j]
        halo.dim[j].pad = pads[j][0]
    return prepare_halo(ContractOp(out_shape, swapped=False, m=m, n=n, k=k), halo, x.dtype)


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


def _input_grad(gz, wk, dilation, out_order, xp_shape, halo=True):
    """dL/dxp: gz padded by d * (K - 1) on both sides of every spatial dim, as
    (batch..., spatial..., out channel), convolved with the weight flipped along its
    kernel dims and with its channel dims exchanged, (channel, kernel..., out channel).
    The padding is zeros, so es_contract_halo reads gz in place when it can (``halo``);
    otherwise gz is padded by es_gather first."""
    ns = len(dilation)
    nb = len(xp_shape) - ns - 1
    o_dim = nb + ns
    kernel = wk.shape[1 : 1 + ns]
    reach = [dilation[j] * (kernel[j] - 1) for j in range(ns)]
    pos = {d: i for i, d in enumerate(out_order)}
    base = wk.data_ptr()
    src = [(wk.shape[0], wk.stride(0), 1 + ns, -1, 0)]
    for j in range(ns):
        base += (kernel[j] - 1) * wk.stride(1 + j) * wk.element_size()
        src.append((kernel[j], -wk.stride(1 + j), 1 + j, -1, 0))
    src.append((wk.shape[-1], wk.stride(-1), 0, -1, 0))
    wflip_shape = (wk.shape[-1], *kernel, wk.shape[0])
    wflip = _gather_into(base, wk.dtype, wk.device, wflip_shape, src)
    identity = tuple(range(len(xp_shape)))
    if halo and gz.dtype in (torch.bfloat16, torch.float16):
        xdims = [pos[d] for d in range(o_dim + 1)]
        prep = _halo_prepare(gz, wflip, xdims, [(r, r) for r in reach], dilation, identity)
        if prep is not None:
            try:
                return _conv_launch(prep, gz, wflip, None)
            except NativeError as err:
                if err.status != ES_ERR_UNSUPPORTED:  # the library launched nothing: pad instead
                    raise
    gpad_shape = [gz.shape[pos[d]] for d in range(nb)]
    gpad_shape += [gz.shape[pos[nb + j]] + 2 * reach[j] for j in range(ns)]
    gpad_shape.append(gz.shape[pos[o_dim]])
    src = []
    for i in range(gz.dim()):
        d = out_order[i]
        offset = -reach[d - nb] if nb <= d < o_dim else 0
        src.append((gz.shape[i], gz.stride(i), d, -1, offset))
    gpad = _gather_into(gz.data_ptr(), gz.dtype, gz.device, tuple(gpad_shape), src)
    return _conv(gpad, wflip, None, dilation, identity)


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
    """A cached no-grad call: the gathers and the contraction, prepared (no input
    gather when the contraction reads the unpadded input, es_contract_halo)."""
    prep_x, prep_w, prep_c = plan
    xp = x if prep_x is None else launch(prep_x, (x,), x.device, x.dtype)
    wk = launch(prep_w, (weight,), weight.device, weight.dtype)
    return _conv_launch(prep_c, xp, wk, bias)


_MODES = _RUN_DIRECTLY + _RECOMPUTE


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
        # a plan that reads the input in place needs it 16-byte aligned, which the key
        # does not record; a misaligned input takes the uncached path (and pads)
        if plan is not None and (plan[0] is not None or x.data_ptr() % 16 == 0):
            return _replay(plan, x, weight, bias)
    (input_spec, weight_spec, output_spec), windows = _conv_specs(shard, windows, groups, families)

    roles = _conv_roles(input_spec, weight_spec, output_spec, windows)
    ndim = len(roles.spatial)
    stride = _per_axis(stride, ndim, "stride")
    dilation = _per_axis(dilation, ndim, "dilation")
    if any(value != 1 for value in stride):
        raise NotImplementedError("einconv currently supports only stride=1")
    halos = _conv_halos(padding, families, roles, weight, dilation)
    input_axes, weight_axes = list(roles.inputs.values()), list(roles.weights.values())
    input_names, weight_names, output_names = list(roles.inputs), list(roles.weights), list(roles.outputs)
    spatial, kernels, channel, out_channel = roles.spatial, roles.kernels, roles.channel, roles.out_channel

    batch = roles.batch
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
        _check_padding(x_arg, input_axes, halos, mesh=mesh, boundary=boundary, shapes=shapes)
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

    def halo_plan(x_arg, wk):
        # the convolution straight from the unpadded input when it qualifies: zero
        # padding, a 16-bit input with its channel axis contiguous, one or two spatial dims
        if boundary != "constant" or x_arg.dtype not in (torch.bfloat16, torch.float16) or ndim not in (1, 2):
            return None
        if fill_bits(fill, x_arg.dtype) != 0:  # -0.0 pads with other bits than zeros
            return None
        xdims = [input_names.index(name) for name in batch + spatial + [channel]]
        pads = [_normalize_halo(halos[name]) if name in halos else (0, 0) for name in spatial]
        return _halo_prepare(x_arg, wk, xdims, pads, dilation, out_order)

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
        # the checks and gathers of operands(), with the input's gather skipped when the
        # contraction reads the unpadded input
        check_device_tensors([x, weight] + ([] if bias is None else [bias]), what="einconv")
        px = pad_plan(x)
        _check_shapes(x, weight, bias)
        pw = weight_plan(weight)
        wk = _gather_run(pw[0], weight, pw[1], pw[2], "constant")
        prep_c = halo_plan(x, wk)
        if prep_c is not None:
            try:
                out = _conv_launch(prep_c, x, wk, bias)
            except NativeError as err:
                if err.status != ES_ERR_UNSUPPORTED:  # the library launched nothing: pad instead
                    raise
            else:
                if key is not None:
                    remember(key, (None, pw[0], prep_c))
                return out
        xp = _gather_run(px[0], x, px[1], px[2], boundary)
        prep_c = _conv_prepare(xp, wk, geometry[0], geometry[1], bias is not None)
        out = _conv_launch(prep_c, xp, wk, bias)
        if key is not None:
            remember(key, (px[0], pw[0], prep_c))
        return out
    if checkpoint == "conv":
        return run_full(*tensors)
    return _checkpoint(run_full, tensors, checkpoint, use_reentrant)
