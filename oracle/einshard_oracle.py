"""Restatement of the reference's CPU path for the single-device operations.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Everything runs on CPU
tensors with the same library routines the reference calls, so the result is
the reference's result on the same inputs:

  einshard_cpu    reference src/torch_einshard/einsum.py:101-135 — group
                  expansion by reshape (:56-74, factor inference :31-53), one
                  letter per distinct (name, mesh dim) in first-seen order
                  (:20-28), ``torch.einsum`` (:132), output packing by reshape
                  (:77-98).
  einhalo_cpu     reference halo.py:27-55 (per-axis ``F.pad`` / clamped or
                  wrapped ``index_select``) via :307-344.
  einwindow_cpu   reference halo.py:347-418: the halo above, then ``unfold`` per
                  windowed axis in input order, then ``permute(...).contiguous()``.
  einconv_cpu     reference conv.py:153-207: the halo, permutes to (batch,
                  channel, spatial...) and (out, channel, kernel...), then
                  ``F.conv{1,2,3}d`` with padding 0.
  einroll_cpu     reference roll.py:10-45 (local axes): ``torch.roll`` per axis
                  with a nonzero shift, in spec order; ``x`` itself if none.

The expression parser here is deliberately independent of the product's: a
small tokenizer that accepts the expressions the tests use (axes, ``name/mesh``,
``( )`` groups, ``...``, ``// p`` partials and ``[...]`` annotations, which are
skipped).  Families are not handled here; tests pass already-expanded text.
"""

import re
import string

import torch
import torch.nn.functional as F

__all__ = ["parse", "equation", "einshard_cpu", "einhalo_cpu", "einwindow_cpu"]

_TOKEN = re.compile(r"\s*(\.\.\.|->|//|[(),/\[\]=:]|[A-Za-z0-9_]+(?:-[A-Za-z0-9_]+)*)")


def _tokens(text):
    pos = 0
    out = []
    text = text.rstrip()
    while pos < len(text):
        match = _TOKEN.match(text, pos)
        if not match:
            raise ValueError(f"oracle parser: cannot tokenize {text[pos:]!r}")
        out.append(match.group(1))
        pos = match.end()
    return out


def _parse_tensor(tokens, i):
    """Return (items, i); items: ("axis", name, mesh) | ("group", [(name, mesh)]) | ("ellipsis",)."""
    items = []
    while i < len(tokens) and tokens[i] not in (",", "->", "//", "["):
        tok = tokens[i]
        if tok == "...":
            items.append(("ellipsis",))
            i += 1
        elif tok == "(":
            i += 1
            members = []
            while tokens[i] != ")":
                name = tokens[i]
                mesh = ""
                if i + 2 < len(tokens) and tokens[i + 1] == "/":
                    mesh = tokens[i + 2]
                    i += 2
                members.append((name, mesh))
                i += 1
            items.append(("group", members))
            i += 1
        else:
            name = tok
            mesh = ""
            if i + 2 < len(tokens) and tokens[i + 1] == "/":
                mesh = tokens[i + 2]
                i += 2
            items.append(("axis", name, mesh))
            i += 1
    partials = []
    if i < len(tokens) and tokens[i] == "//":
        i += 1
        if tokens[i] == "(":
            i += 1
            while tokens[i] != ")":
                if tokens[i] != ",":
                    partials.append(tokens[i])
                i += 1
            i += 1
        else:
            partials.append(tokens[i])
            i += 1
    if i < len(tokens) and tokens[i] == "[":
        while tokens[i] != "]":
            i += 1
        i += 1
    return (items, partials), i


def parse(expression):
    """``"x, y -> z"`` -> ([x_items, y_items?], z_items) with partials dropped."""
    tokens = _tokens(expression)
    inputs = []
    i = 0
    spec, i = _parse_tensor(tokens, i)
    inputs.append(spec)
    if tokens[i] == ",":
        spec, i = _parse_tensor(tokens, i + 1)
        inputs.append(spec)
    if tokens[i] != "->":
        raise ValueError(f"oracle parser: expected '->' in {expression!r}")
    out, i = _parse_tensor(tokens, i + 1)
    # the reference grammar needs at least one axis per tensor (grammar.py:18)
    if not out[0] or any(not spec[0] for spec in inputs):
        raise ValueError(f"oracle parser: a tensor without axes in {expression!r}")
    return inputs, out


def _flat_keys(items):
    keys = []
    for item in items:
        if item[0] == "ellipsis":
            keys.append("...")
        elif item[0] == "group":
            keys.extend(item[1])
        else:
            keys.append((item[1], item[2]))
    return keys


def equation(expression):
    """The torch.einsum equation the reference builds (einsum.py:107-130)."""
    inputs, out = parse(expression)
    letters = {}
    parts = []
    for items, _ in inputs:
        text = ""
        for key in _flat_keys(items):
            if key == "...":
                text += "..."
                continue
            if key not in letters:
                letters[key] = string.ascii_lowercase[len(letters)]
            text += letters[key]
        parts.append(text)
    text = ""
    for key in _flat_keys(out[0]):
        text += "..." if key == "..." else letters[key]
    return ",".join(parts) + "->" + text


def _expand(x, items, sizes):
    if not any(item[0] == "group" for item in items):
        return x
    fixed = sum(1 for item in items if item[0] != "ellipsis")
    n_ell = x.dim() - fixed
    shape = []
    dim = 0
    for item in items:
        if item[0] == "ellipsis":
            shape.extend(x.shape[dim:dim + n_ell])
            dim += n_ell
        elif item[0] == "group":
            known = [None if sizes is None else sizes.get(name) for name, _ in item[1]]
            product = 1
            for value in known:
                if value is not None:
                    product *= value
            if None in known:
                known[known.index(None)] = x.shape[dim] // product
            shape.extend(known)
            dim += 1
        else:
            shape.append(x.shape[dim])
            dim += 1
    return x.reshape(shape)


def _pack(z, items):
    if not any(item[0] == "group" for item in items):
        return z
    fixed = sum(len(item[1]) if item[0] == "group" else 1 for item in items if item[0] != "ellipsis")
    n_ell = z.dim() - fixed
    shape = []
    dim = 0
    for item in items:
        if item[0] == "ellipsis":
            shape.extend(z.shape[dim:dim + n_ell])
            dim += n_ell
        elif item[0] == "group":
            size = 1
            for _ in item[1]:
                size *= z.shape[dim]
                dim += 1
            shape.append(size)
        else:
            shape.append(z.shape[dim])
            dim += 1
    return z.reshape(shape)


def einshard_cpu(expression, *xs, sizes=None):
    """The reference's local einshard, on CPU tensors."""
    inputs, out = parse(expression)
    xs = [x.cpu() for x in xs]
    operands = [_expand(x, items, sizes) for x, (items, _) in zip(xs, inputs)]
    result = torch.einsum(equation(expression), *operands)
    return _pack(result, out[0])


def _normalize(value):
    return (value, value) if isinstance(value, int) else tuple(value)


def _pad_dim(x, dim, left, right, boundary, fill):
    if left == 0 and right == 0:
        return x
    n = x.shape[dim]
    if boundary == "periodic":
        pieces = []
        if left:
            pieces.append(torch.index_select(x, dim, torch.arange(n - left, n).remainder(n)))
        pieces.append(x)
        if right:
            pieces.append(torch.index_select(x, dim, torch.arange(right).remainder(n)))
        return torch.cat(pieces, dim=dim).contiguous()
    if boundary == "replicate":
        return torch.index_select(x, dim, torch.arange(-left, n + right).clamp(0, n - 1)).contiguous()
    pad = [0, 0] * x.dim()
    pad[2 * (x.dim() - dim - 1)] = left
    pad[2 * (x.dim() - dim - 1) + 1] = right
    return F.pad(x, pad, mode="constant", value=fill)


def _names(items):
    return [item[1] for item in items]


def einhalo_cpu(spec, x, halos, *, boundary="constant", fill=0):
    inputs, _ = parse(f"{spec} -> {spec}")
    names = _names(inputs[0][0])
    z = x.cpu()
    for dim, name in enumerate(names):
        if name in halos:
            left, right = _normalize(halos[name])
            z = _pad_dim(z, dim, left, right, boundary, fill)
    return z


def einwindow_cpu(expression, x, windows, radius, *, boundary="constant", fill=0):
    inputs, out = parse(expression)
    names = _names(inputs[0][0])
    out_names = _names(out[0])
    z = x.cpu()
    for dim, name in enumerate(names):
        if name in windows:
            left, right = _normalize(radius[name])
            z = _pad_dim(z, dim, left, right, boundary, fill)
    current = list(names)
    for name in names:
        if name not in windows:
            continue
        left, right = _normalize(radius[name])
        z = z.unfold(current.index(name), left + right + 1, 1)
        current.append(windows[name])
    return z.permute([current.index(name) for name in out_names]).contiguous()


def einconv_cpu(expression, x, weight, windows, *, bias=None, padding=None, dilation=1, boundary="constant", fill=0):
    """The reference's local einconv (conv.py:153-207) on CPU tensors: pad every
    window source axis by its halo, permute the input to (batch..., channel,
    spatial...) and the weight to (out channel, channel, kernel...), run
    F.conv{1,2,3}d with padding 0, then permute back to the output order.
    ``padding``: None (the reference default: half the effective kernel per side),
    an int / (left, right) per axis, or a dict keyed by the source axis."""
    inputs, out = parse(expression)
    x_names = _names(inputs[0][0])
    w_names = _names(inputs[1][0])
    out_names = _names(out[0])
    spatial = list(windows)
    kernels = [windows[name] for name in spatial]
    ndim = len(spatial)
    dil = (dilation,) * ndim if isinstance(dilation, int) else tuple(dilation)
    channel = [n for n in x_names if n in w_names and n not in spatial and n not in out_names][0]
    out_channel = [n for n in w_names if n in out_names and n not in x_names][0]
    batch = [n for n in x_names if n not in spatial and n != channel]
    if padding is None:
        pads = [(d * (weight.shape[w_names.index(k)] - 1) // 2,) * 2 for k, d in zip(kernels, dil)]
    elif isinstance(padding, dict):
        pads = [_normalize(padding[name]) for name in spatial]
    else:
        values = (padding,) * ndim if isinstance(padding, int) else tuple(padding)
        pads = [_normalize(v) for v in values]
    z = x.cpu()
    for name, (left, right) in zip(spatial, pads):
        z = _pad_dim(z, x_names.index(name), left, right, boundary, fill)
    z = z.permute([x_names.index(n) for n in batch + [channel] + spatial]).contiguous()
    batch_shape = z.shape[: len(batch)]
    z = z.reshape((-1, z.shape[len(batch)], *z.shape[len(batch) + 1 :]))
    w = weight.cpu().permute([w_names.index(n) for n in [out_channel, channel] + kernels]).contiguous()
    conv = {1: F.conv1d, 2: F.conv2d, 3: F.conv3d}[ndim]
    r = conv(z, w, None if bias is None else bias.cpu(), stride=1, padding=0, dilation=dil)
    r = r.reshape((*batch_shape, *r.shape[1:]))
    conv_names = batch + [out_channel] + spatial
    return r.permute([conv_names.index(n) for n in out_names]).contiguous()


def einroll_cpu(spec, x, shifts):
    """The reference's local einroll (roll.py:10-27): one ``torch.roll`` per axis of
    the spec with a nonzero shift, dims numbered by spec position."""
    inputs, _ = parse(f"{spec} -> {spec}")
    z = x
    for dim, name in enumerate(_names(inputs[0][0])):
        shift = shifts.get(name, 0)
        if shift != 0:
            z = torch.roll(z.cpu(), shifts=shift, dims=dim)
    return z
