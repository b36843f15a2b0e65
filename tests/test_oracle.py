"""Pinning the CPU oracle before trusting it.

Every oracle function is checked against something that fixes its answer
independently: the reference's own inline known answers
(tests/golden/known_answers.json), closed forms from the reference's tests,
and brute force (oracle/brute.c: exhaustive fp64 einsum, closed-form window)
plus numpy's einsum.  Planted mistakes show that these checks catch a
transposed operand, a dropped term and an off-by-one window."""

import json
import os

import pytest
import torch
import torch.nn.functional as F

from oracle import PINNING
from oracle.brute import brute_einsum, brute_window, numpy_einsum_f64
from oracle.einshard_oracle import einhalo_cpu, einshard_cpu, einwindow_cpu, equation
from oracle.einshard_oracle import parse as oracle_parse

from conftest import randn

KNOWN = json.load(open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")))


def canonical(eq):
    """Rename letters in first-seen order so equivalent equations compare equal."""
    mapping = {}
    out = []
    for ch in eq:
        if ch.isalpha():
            mapping.setdefault(ch, chr(ord("a") + len(mapping)))
            out.append(mapping[ch])
        else:
            out.append(ch)
    return "".join(out)


def test_every_oracle_function_is_pinned():
    for name, status in PINNING.items():
        assert status.startswith("pinned"), name


@pytest.mark.parametrize("expression, handwritten", KNOWN["equations"]["pairs"])
def test_equation_matches_reference_tests(expression, handwritten):
    assert canonical(equation(expression)) == canonical(handwritten)


def test_equation_keys_letters_by_name_and_mesh_dim():
    # "c" and "c/tp" are different axes in the reference's letter table
    assert canonical(equation("a c, c/tp b -> a b")) == canonical("ab,cd->ad")


BRUTE_CASES = [
    ("a b, b c -> a c", [(5, 4), (4, 6)]),
    ("a b k c, b c l d -> k l d a", [(3, 2, 4, 3), (2, 3, 2, 5)]),
    ("b n c, h c -> b n h", [(2, 3, 4), (5, 4)]),
    ("p b n h -> b n h", [(3, 2, 3, 4)]),
    ("b n h -> b h", [(2, 5, 3)]),
    ("b n h, h -> b n h", [(2, 3, 4), (4,)]),
    ("i, j -> i j", [(3,), (4,)]),
    ("i i -> i", [(5, 5)]),
    ("i i j, j -> i", [(4, 4, 3), (3,)]),
    ("... c, c o -> ... o", [(2, 3, 4), (4, 5)]),
    ("... c -> c", [(2, 3, 4)]),
    ("b ... c -> ... b c", [(2, 3, 4, 5)]),
    ("a b, c -> a c", [(3, 4), (5,)]),
]


@pytest.mark.parametrize("expression, shapes", BRUTE_CASES)
def test_einshard_cpu_matches_brute_force_f64(expression, shapes):
    xs = [randn(*s, seed=100 + i).to(torch.float64) for i, s in enumerate(shapes)]
    got = einshard_cpu(expression, *xs)
    eq = equation(expression)
    want = brute_einsum(eq, *xs)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    lhs, rhs = eq.split("->")
    if "..." in rhs or "..." not in lhs:
        # numpy rejects an ellipsis the output drops; torch sums it (brute force covers that)
        torch.testing.assert_close(numpy_einsum_f64(eq, *xs), want, rtol=1e-12, atol=1e-12)


@pytest.mark.parametrize("dtype, tol", [(torch.float32, 1e-5), (torch.bfloat16, 2e-2)])
def test_einshard_cpu_low_precision_within_budget(dtype, tol):
    x = randn(16, 64, seed=1, dtype=dtype)
    y = randn(64, 24, seed=2, dtype=dtype)
    got = einshard_cpu("a b, b c -> a c", x, y).to(torch.float64)
    want = brute_einsum("ab,bc->ac", x, y)
    scale = max(want.abs().max().item(), want.pow(2).mean().sqrt().item())
    assert (got - want).abs().max().item() / scale <= tol


def test_closed_forms_from_reference_tests():
    # reference tests/test_einsum.py:154-246
    x = randn(2, 3, 12, 5)
    torch.testing.assert_close(einshard_cpu("... (h p) c -> ... h p c", x, sizes={"p": 4}), x.reshape(2, 3, 3, 4, 5))
    x = randn(2, 12, 5)
    torch.testing.assert_close(einshard_cpu("b (h p) c -> b h p c", x, sizes={"p": 4}), x.reshape(2, 3, 4, 5))
    torch.testing.assert_close(
        einshard_cpu("b (h p) c -> b c h p", x, sizes={"h": 3}), x.reshape(2, 3, 4, 5).permute(0, 3, 1, 2)
    )
    x = randn(2, 3, 4, 5)
    torch.testing.assert_close(einshard_cpu("b h p c -> b (h p) c", x), x.reshape(2, 12, 5))
    x = randn(2, 3, 8, 10, 5)
    expected = x.reshape(2, 3, 2, 4, 2, 5, 5).permute(0, 2, 4, 1, 3, 5, 6).reshape(8, 3, 4, 5, 5)
    got = einshard_cpu("b t (h wh) (w ww) c -> (b h w) t wh ww c", x, sizes={"wh": 4, "ww": 5})
    torch.testing.assert_close(got, expected)


def test_halo_known_answers():
    data = KNOWN["halo_arange5_left2_right1"]
    x = torch.tensor(data["input"], dtype=torch.float32)
    assert einhalo_cpu("h", x, {"h": (2, 1)}, fill=-1).tolist() == data["constant_fill_-1"]
    assert einhalo_cpu("h", x, {"h": (2, 1)}, boundary="periodic").tolist() == data["periodic"]
    assert einhalo_cpu("h", x, {"h": (2, 1)}, boundary="replicate").tolist() == data["replicate"]


def test_window_known_answers():
    data = KNOWN["window_h_kh_radius1_fill_-1"]
    x = torch.tensor(data["input"], dtype=torch.float32)
    assert einwindow_cpu("h -> h kh", x, {"h": "kh"}, {"h": 1}, fill=-1).tolist() == data["expected"]
    shape = KNOWN["window_family_shape"]
    z = einwindow_cpu("h w -> h w kh kw", torch.zeros(shape["input_shape"]), {"h": "kh", "w": "kw"}, {"h": 1, "w": 0})
    assert list(z.shape) == shape["expected_shape"]


def test_window_then_contraction_is_conv2d():
    # reference tests/test_halo.py:123-136
    x = torch.arange(12, dtype=torch.float32).reshape(1, 3, 4, 1)
    weight = torch.ones(1, 3, 3, 1)
    patches = einwindow_cpu("b h w c -> b h w kh kw c", x, {"h": "kh", "w": "kw"}, {"h": 1, "w": 1})
    z = einshard_cpu("b h w kh kw c, o kh kw c -> b h w o", patches, weight)
    expected = F.conv2d(x.permute(0, 3, 1, 2), weight.permute(0, 3, 1, 2), padding=1).permute(0, 2, 3, 1)
    torch.testing.assert_close(z, expected)


def _window_dims(names, out_names, windows, radius):
    pos, win, left = [], [], []
    for name in names:
        pos.append(out_names.index(name))
        if name in windows:
            r = radius[name]
            r = (r, r) if isinstance(r, int) else r
            win.append(out_names.index(windows[name]))
            left.append(r[0])
        else:
            win.append(-1)
            left.append(0)
    return pos, win, left


@pytest.mark.parametrize("boundary", ["constant", "replicate", "periodic"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.int16, torch.float64])
def test_window_matches_brute_force_bitwise(boundary, dtype):
    x = (randn(2, 7, 6, 3, seed=9) * 100).to(dtype)
    windows = {"h": "kh", "w": "kw"}
    radius = {"h": (2, 1), "w": 3}
    expr = "b h w c -> b h kh w kw c"
    got = einwindow_cpu(expr, x, windows, radius, boundary=boundary, fill=-7)
    out_names = ["b", "h", "kh", "w", "kw", "c"]
    pos, win, left = _window_dims(["b", "h", "w", "c"], out_names, windows, radius)
    want = brute_window(x, list(got.shape), pos, win, left, boundary=boundary, fill=-7)
    assert torch.equal(got.view(torch.uint8) if dtype == torch.bool else got, want)


@pytest.mark.parametrize("boundary", ["constant", "replicate", "periodic"])
def test_halo_matches_brute_force(boundary):
    x = randn(5, 4, seed=2)
    got = einhalo_cpu("a b", x, {"a": (3, 6), "b": 1}, boundary=boundary, fill=2.5)
    want = brute_window(x, list(got.shape), [0, 1], [-1, -1], [3, 1], boundary=boundary, fill=2.5)
    assert torch.equal(got, want)


# ---- planted mistakes: the checks above must notice these ---------------------------


def test_planted_transposed_operand_is_caught():
    x = randn(6, 6, seed=1).to(torch.float64)
    y = randn(6, 6, seed=2).to(torch.float64)
    good = einshard_cpu("a b, b c -> a c", x, y)
    wrong = brute_einsum("ab,cb->ac", x, y)  # operand transposed
    assert not torch.allclose(good, wrong, rtol=1e-5, atol=1e-6)


def test_planted_dropped_term_is_caught():
    x = randn(4, 5, seed=3).to(torch.float64)
    y = randn(5, 3, seed=4).to(torch.float64)
    dropped = x.clone()
    dropped[:, -1] = 0  # one k term missing
    assert not torch.allclose(einshard_cpu("a b, b c -> a c", dropped, y), brute_einsum("ab,bc->ac", x, y))


def test_planted_window_offset_is_caught():
    x = randn(2, 9, 3, seed=5)
    got = einwindow_cpu("b h c -> b h kh c", x, {"h": "kh"}, {"h": 1})
    off_by_one = brute_window(x, list(got.shape), [0, 1, 3], [-1, 2, -1], [0, 0, 0])
    assert not torch.equal(got, off_by_one)


def test_oracle_parser_rejects_a_tensor_without_axes():
    # reference tests/test_grammar.py:142 and :199 expect "a b ->" to fail
    with pytest.raises(ValueError):
        oracle_parse("a b ->")


# ---- einconv: an fp64 direct sum, independent of F.conv ------------------------------


def _source_index(i, n, boundary):
    if 0 <= i < n:
        return i
    if boundary == "replicate":
        return min(max(i, 0), n - 1)
    if boundary == "periodic":
        return i % n
    return None  # constant: the fill value


def _conv_direct_f64(x, w, bias, names, windows, pads, dilation, boundary, fill):
    """out[...] = bias[o] + sum over (kernel..., channel) of w * x at s + d * k - left,
    by explicit loops over every output element (tiny shapes only)."""
    import itertools

    x_names, w_names, out_names = names
    spatial = list(windows)
    channel = [n for n in x_names if n in w_names and n not in spatial and n not in out_names][0]
    out_ch = [n for n in w_names if n in out_names and n not in x_names][0]
    size = {n: x.shape[i] for i, n in enumerate(x_names)}
    size.update({n: w.shape[i] for i, n in enumerate(w_names)})
    xd, wd = x.to(torch.float64), w.to(torch.float64)
    out = torch.zeros([size[n] for n in out_names], dtype=torch.float64)
    kernels = [windows[s] for s in spatial]
    for oc in itertools.product(*[range(size[n]) for n in out_names]):
        at = dict(zip(out_names, oc))
        total = 0.0 if bias is None else float(bias[at[out_ch]])
        for kc in itertools.product(*[range(size[k]) for k in kernels], range(size[channel])):
            k_at = dict(zip(kernels + [channel], kc))
            xi = []
            for n in x_names:
                if n in windows:
                    j = spatial.index(n)
                    i = _source_index(at[n] + dilation[j] * k_at[windows[n]] - pads[j][0], size[n], boundary)
                    if i is None:
                        break
                    xi.append(i)
                else:
                    xi.append(k_at[n] if n == channel else at[n])
            xv = float(fill) if len(xi) < len(x_names) else float(xd[tuple(xi)])
            wi = tuple(at[n] if n == out_ch else k_at[n] for n in w_names)
            total += float(wd[wi]) * xv
        out[oc] = total
    return out


CONV_DIRECT_CASES = [
    # expression, x shape, w shape, windows, padding (per source axis), dilation
    ("b h c, o c k -> b h o", (2, 7, 3), (4, 3, 3), {"h": "k"}, [(1, 1)], (1,)),
    ("b h c, o c k -> b o h", (2, 9, 2), (3, 2, 3), {"h": "k"}, [(3, 1)], (2,)),
    ("b h w c, o c kh kw -> b h w o", (1, 4, 5, 3), (2, 3, 2, 3), {"h": "kh", "w": "kw"}, [(1, 0), (0, 2)], (1, 1)),
    ("c h b w, kw o kh c -> o w b h", (2, 5, 2, 4), (3, 2, 3, 2), {"h": "kh", "w": "kw"}, [(2, 2), (1, 1)], (2, 1)),
    ("b d h w c, o c kd kh kw -> b d h w o", (1, 3, 4, 3, 2), (2, 2, 3, 1, 3), {"d": "kd", "h": "kh", "w": "kw"},
     [(1, 1), (0, 0), (2, 0)], (1, 1, 1)),
]


@pytest.mark.parametrize("boundary", ["constant", "replicate", "periodic"])
@pytest.mark.parametrize("expr, xs, ws, windows, pads, dilation", CONV_DIRECT_CASES)
def test_einconv_cpu_matches_direct_sum_f64(expr, xs, ws, windows, pads, dilation, boundary):
    from oracle.einshard_oracle import einconv_cpu

    x = randn(*xs, seed=41).to(torch.float64)
    w = randn(*ws, seed=42).to(torch.float64)
    (x_spec, w_spec), out_spec = oracle_parse(expr)
    names = [[item[1] for item in spec[0]] for spec in (x_spec, w_spec, out_spec)]
    out_ch_size = ws[names[1].index([n for n in names[1] if n in names[2] and n not in names[0]][0])]
    bias = randn(out_ch_size, seed=43).to(torch.float64)
    padding = {s: p for s, p in zip(windows, pads)}
    got = einconv_cpu(expr, x, w, windows, bias=bias, padding=padding, dilation=dilation, boundary=boundary, fill=-1.5)
    want = _conv_direct_f64(x, w, bias, names, windows, pads, dilation, boundary, -1.5)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_einconv_cpu_is_conv2d_with_padding_one():
    # reference tests/test_conv.py:11-24: the default padding of a 3 x 3 kernel
    from oracle.einshard_oracle import einconv_cpu

    x = randn(2, 5, 6, 3, seed=333)
    w = randn(4, 3, 3, 3, seed=334)
    bias = randn(4, seed=335)
    got = einconv_cpu("b h w c, o c kh kw -> b h w o", x, w, {"h": "kh", "w": "kw"}, bias=bias)
    want = F.conv2d(x.permute(0, 3, 1, 2), w, bias, padding=1).permute(0, 2, 3, 1)
    torch.testing.assert_close(got, want)


def test_planted_flipped_kernel_is_caught():
    # a true convolution (flipped kernel) instead of the cross-correlation F.conv computes
    x = randn(1, 6, 2, seed=7).to(torch.float64)
    w = randn(2, 2, 3, seed=8).to(torch.float64)
    names = [["b", "h", "c"], ["o", "c", "k"], ["b", "h", "o"]]
    good = _conv_direct_f64(x, w, None, names, {"h": "k"}, [(1, 1)], (1,), "constant", 0)
    flipped = _conv_direct_f64(x, w.flip(-1), None, names, {"h": "k"}, [(1, 1)], (1,), "constant", 0)
    assert not torch.allclose(good, flipped)
    from oracle.einshard_oracle import einconv_cpu

    torch.testing.assert_close(einconv_cpu("b h c, o c k -> b h o", x, w, {"h": "k"}), good)


# ---- einroll: the modular index map ------------------------------------------------------


def _roll_index_map(x, shifts_by_dim):
    """out[i...] = x[(i_d - s_d) mod n_d ...] by explicit index arithmetic."""
    out = torch.empty_like(x)
    flat = x.reshape(-1)
    strides = [1] * x.dim()
    for d in range(x.dim() - 2, -1, -1):
        strides[d] = strides[d + 1] * x.shape[d + 1]
    for linear in range(x.numel()):
        rem, src = linear, 0
        for d in range(x.dim()):
            i = rem // strides[d]
            rem -= i * strides[d]
            src += ((i - shifts_by_dim.get(d, 0)) % x.shape[d]) * strides[d]
        out.view(-1)[linear] = flat[src]
    return out


@pytest.mark.parametrize(
    "spec, shape, shifts, by_dim",
    [
        ("a b", (5, 4), {"a": 2}, {0: 2}),
        ("a b", (5, 4), {"a": -7, "b": 3}, {0: -7, 1: 3}),
        ("b h w c", (2, 4, 6, 3), {"h": 3, "w": -5}, {1: 3, 2: -5}),
        ("t x", (3, 5), {"x": 10, "t": 1}, {0: 1, 1: 10}),
        ("t x", (3, 5), {"z": 2}, {}),
    ],
)
def test_einroll_cpu_matches_index_map(spec, shape, shifts, by_dim):
    from oracle.einshard_oracle import einroll_cpu

    x = torch.arange(int(torch.tensor(shape).prod())).reshape(shape)
    assert torch.equal(einroll_cpu(spec, x, shifts), _roll_index_map(x, by_dim))


def test_einroll_cpu_reference_family_case():
    # reference tests/test_distributed_roll.py:10-20, families already expanded
    from oracle.einshard_oracle import einroll_cpu

    x = randn(2, 3, 4, 5, 6, 7, seed=5)
    got = einroll_cpu("b t h w d c", x, {"h": 1, "w": -2, "d": 3})
    assert torch.equal(got, _roll_index_map(x, {2: 1, 3: -2, 4: 3}))


def test_planted_roll_direction_is_caught():
    from oracle.einshard_oracle import einroll_cpu

    x = torch.arange(12).reshape(3, 4)
    assert not torch.equal(einroll_cpu("a b", x, {"b": 1}), _roll_index_map(x, {1: -1}))
