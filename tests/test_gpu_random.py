"""Seeded random parity sweep of es.einshard against the oracle.

Each case draws an expression (one or two operands, distinct axis names, any
subset of the labels kept in the output), extents, a dtype and operand layouts
(contiguous, permuted, sliced) from a fixed seed, so a failure names its seed and
replays exactly.  Results are compared with the oracle's torch.einsum on the CPU:
bit-exact for pure copies, and for arithmetic within the dtype's tolerance of the
fp32 result computed from the same rounded inputs.  Two families of extents are
drawn: small ones (every kernel's edge handling) and ones large enough for the
fast contraction kernels (whole 64-deep K tiles, hundreds of output tiles)."""

import random

import pytest
import torch

import torch_einshard as es
from oracle.einshard_oracle import einshard_cpu

from conftest import TOL, assert_bitexact, assert_rel

pytestmark = pytest.mark.gpu

NAMES = "abcdefgh"
DTYPES = [torch.float32, torch.bfloat16, torch.float16]


def _layout(rng, shape):
    """A CPU tensor of ``shape`` that is contiguous, a permuted view or a sliced view."""
    kind = rng.choice(["contiguous", "permuted", "sliced"])
    gen = torch.Generator().manual_seed(rng.randrange(1 << 30))
    if kind == "permuted" and len(shape) > 1:
        order = list(range(len(shape)))
        rng.shuffle(order)
        base = torch.randn([shape[i] for i in order], generator=gen)
        inverse = [order.index(i) for i in range(len(shape))]
        return base.permute(inverse)
    if kind == "sliced" and len(shape) > 0:
        d = rng.randrange(len(shape))
        big = list(shape)
        big[d] = shape[d] * 2
        return torch.randn(big, generator=gen).narrow(d, 0, shape[d]) if rng.random() < 0.5 else torch.randn(
            big, generator=gen
        )[(slice(None),) * d + (slice(None, None, 2),)]
    return torch.randn(shape, generator=gen)


def _prod(values):
    out = 1
    for v in values:
        out *= v
    return out


def _case(seed, large):
    rng = random.Random(seed)
    if large:
        return _contraction_case(rng)
    n_labels = rng.randint(2, 5)
    labels = list(NAMES[:n_labels])
    binary = rng.random() < 0.7
    x_labels = rng.sample(labels, rng.randint(1, min(4, n_labels)))
    if binary:
        y_labels = rng.sample(labels, rng.randint(1, min(4, n_labels)))
        present = sorted(set(x_labels) | set(y_labels), key=labels.index)
    else:
        y_labels = None
        present = list(x_labels)
    out = [name for name in present if rng.random() < 0.6] or [rng.choice(present)]
    rng.shuffle(out)
    sizes = {name: rng.randint(1, 9) for name in labels}
    return _build(rng, x_labels, y_labels, out, sizes)


def _contraction_case(rng):
    """batch / M-only / N-only / contracted labels with extents for the tiled kernels:
    M and N of a few hundred to a few thousand, K from 64 up, at most 2^31
    multiply-adds; axis orders shuffled in both operands and the output."""
    groups = {"b": rng.randint(0, 1), "m": rng.randint(1, 2), "n": rng.randint(1, 2), "k": rng.randint(1, 3)}
    names = iter(NAMES)
    labels = {g: [next(names) for _ in range(c)] for g, c in groups.items()}
    choices = [2, 3, 4, 8, 16, 32, 64, 96, 128, 256, 512, 1024]
    for _ in range(1000):
        sizes = {n: rng.choice(choices) for g in labels for n in labels[g]}
        tot = {g: _prod(sizes[n] for n in labels[g]) for g in labels}
        if (
            tot["b"] <= 4
            and 256 <= tot["m"] <= 8192
            and 128 <= tot["n"] <= 4096
            and 64 <= tot["k"] <= 4096
            and tot["b"] * tot["m"] * tot["n"] * tot["k"] <= 2**31
        ):
            break
    x_labels = labels["b"] + labels["m"] + labels["k"]
    y_labels = labels["b"] + labels["n"] + labels["k"]
    out = labels["b"] + labels["m"] + labels["n"]
    for group in (x_labels, y_labels, out):
        rng.shuffle(group)
    return _build(rng, x_labels, y_labels, out, sizes)


def _build(rng, x_labels, y_labels, out, sizes):
    binary = y_labels is not None
    expr = " ".join(x_labels)
    if binary:
        expr += ", " + " ".join(y_labels)
    expr += " -> " + " ".join(out)
    dtype = rng.choice(DTYPES)
    xs = [_layout(rng, [sizes[n] for n in x_labels])]
    if binary:
        xs.append(_layout(rng, [sizes[n] for n in y_labels]))
    xs = [x.to(dtype) for x in xs]
    present = set(x_labels) | set(y_labels or [])
    copy_only = not binary and present == set(out)
    return expr, xs, dtype, copy_only


def _check(gpu, seed, large):
    expr, xs, dtype, copy_only = _case(seed, large)
    print(f"seed {seed}: {expr} {[tuple(x.shape) for x in xs]} {dtype}", flush=True)
    got = es.einshard(expr, *[x.to(gpu) for x in xs])
    if copy_only:
        assert_bitexact(got, einshard_cpu(expr, *xs))
    else:
        want = einshard_cpu(expr, *[x.float() for x in xs])
        assert got.dtype == dtype, (expr, got.dtype)
        assert_rel(got, want.to(dtype), TOL[dtype])


@pytest.mark.parametrize("seed", range(400))
def test_random_small(gpu, seed):
    _check(gpu, seed, large=False)


@pytest.mark.parametrize("seed", range(1000, 1080))
def test_random_large(gpu, seed):
    _check(gpu, seed, large=True)


# ---- windows, halos, rolls, convolutions --------------------------------------------------

BOUNDARIES = ["constant", "replicate", "periodic"]


def _window_case(seed):
    from oracle.einshard_oracle import einwindow_cpu

    rng = random.Random(seed)
    rank = rng.randint(1, 4)
    names = list(NAMES[:rank])
    shape = [rng.randint(1, 12) for _ in names]
    windowed = rng.sample(names, rng.randint(1, min(2, rank)))
    windows = {n: "w" + n for n in windowed}
    radius = {n: (rng.randint(0, 3), rng.randint(0, 3)) for n in windowed}
    out = names + [windows[n] for n in windowed]
    rng.shuffle(out)
    boundary = rng.choice(BOUNDARIES)
    dtype = rng.choice([torch.float32, torch.bfloat16, torch.int32, torch.float64, torch.uint8])
    x = (_layout(rng, shape) * 20).to(dtype)
    expr = " ".join(names) + " -> " + " ".join(out)
    return expr, x, windows, radius, boundary, einwindow_cpu


@pytest.mark.parametrize("seed", range(2000, 2150))
def test_random_window(gpu, seed):
    expr, x, windows, radius, boundary, oracle = _window_case(seed)
    print(f"seed {seed}: {expr} {tuple(x.shape)} {windows} {radius} {boundary} {x.dtype}", flush=True)
    fill = 3 if x.dtype == torch.uint8 else -3  # F.pad rejects a fill the dtype cannot hold
    got = es.einwindow(expr, x.to(gpu), windows, radius, boundary=boundary, fill=fill)
    assert_bitexact(got, oracle(expr, x, windows, radius, boundary=boundary, fill=fill))


@pytest.mark.parametrize("seed", range(3000, 3100))
def test_random_halo_and_roll(gpu, seed):
    from oracle.einshard_oracle import einhalo_cpu, einroll_cpu

    rng = random.Random(seed)
    rank = rng.randint(1, 5)
    names = list(NAMES[:rank])
    x = _layout(rng, [rng.randint(1, 10) for _ in names]).to(rng.choice([torch.float32, torch.bfloat16, torch.int64]))
    spec = " ".join(names)
    halos = {n: (rng.randint(0, 4), rng.randint(0, 4)) for n in rng.sample(names, rng.randint(1, rank))}
    boundary = rng.choice(BOUNDARIES)
    print(f"seed {seed}: {spec} {tuple(x.shape)} halos {halos} {boundary} {x.dtype}", flush=True)
    got = es.einhalo(spec, x.to(gpu), halos, boundary=boundary, fill=7)
    assert_bitexact(got, einhalo_cpu(spec, x, halos, boundary=boundary, fill=7))
    shifts = {n: rng.randint(-25, 25) for n in rng.sample(names, rng.randint(1, rank))}
    got = es.einroll(spec, x.to(gpu), shifts)
    assert_bitexact(got, einroll_cpu(spec, x, shifts))


@pytest.mark.parametrize("seed", range(4000, 4060))
def test_random_conv(gpu, seed):
    from oracle.einshard_oracle import einconv_cpu

    rng = random.Random(seed)
    nd = rng.randint(1, 3)
    spatial = ["h", "w", "d"][:nd]
    kernels = ["k" + s for s in spatial]
    batch = ["b"] if rng.random() < 0.8 else []
    x_names = batch + spatial + ["c"]
    rng.shuffle(x_names)
    w_names = ["o", "c"] + kernels
    rng.shuffle(w_names)
    out = [n if n != "c" else "o" for n in x_names]
    rng.shuffle(out)
    size = {"b": rng.randint(1, 3), "c": rng.choice([1, 3, 8, 64]), "o": rng.choice([2, 5, 16, 64])}
    for s, k in zip(spatial, kernels):
        size[s] = rng.randint(3, 12 if nd > 1 else 40)
        size[k] = rng.randint(1, 4)
    dilation = tuple(rng.randint(1, 2) for _ in spatial)
    padding = {}
    for s, k, d in zip(spatial, kernels, dilation):
        reach = d * (size[k] - 1)
        left = rng.randint(0, reach)
        padding[s] = (left, reach - left)
    boundary = rng.choice(BOUNDARIES)
    dtype = rng.choice([torch.float32, torch.bfloat16])
    x = _layout(rng, [size[n] for n in x_names]).to(dtype)
    w = (_layout(rng, [size[n] for n in w_names]) * 0.3).to(dtype)
    bias = _layout(rng, [size["o"]]).to(dtype) if rng.random() < 0.5 else None
    expr = f"{' '.join(x_names)}, {' '.join(w_names)} -> {' '.join(out)}"
    windows = dict(zip(spatial, kernels))
    print(f"seed {seed}: {expr} x{tuple(x.shape)} w{tuple(w.shape)} pad {padding} dil {dilation} {boundary} {dtype}",
          flush=True)
    got = es.einconv(expr, x.to(gpu), w.to(gpu), windows, bias=None if bias is None else bias.to(gpu),
                     padding=padding, dilation=dilation, boundary=boundary, fill=0.5, checkpoint=False)
    want = einconv_cpu(expr, x.float(), w.float(), windows, bias=None if bias is None else bias.float(),
                       padding=padding, dilation=dilation, boundary=boundary, fill=0.5)
    assert_rel(got, want.to(dtype), TOL[dtype])
