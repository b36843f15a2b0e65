"""Gradients of es.einshard / es.einwindow / es.einhalo on the GPU against the
oracle's CPU path (torch.einsum, F.pad + unfold + permute: the reference's own
differentiable calls).  Tolerances: fp32 1e-5 and bf16 2e-2 relative with a
scale floor; the window adjoint sums at most a few terms per element."""

import pytest
import torch

import torch_einshard as es
from oracle.einshard_oracle import einhalo_cpu, einshard_cpu, einwindow_cpu

from conftest import TOL, assert_rel, randn

pytestmark = pytest.mark.gpu


def _grads(fn, xs, gz):
    xs = [x.detach().clone().requires_grad_(True) for x in xs]
    out = fn(*xs)
    grads = torch.autograd.grad(out, xs, gz.to(out.device, out.dtype))
    return out.detach(), grads


EINSUM_CASES = [
    ("b n c, h c -> b n h", [(2, 24, 64), (40, 64)], None),
    ("a b k c, b c l d -> k l d a", [(4, 3, 5, 8), (3, 8, 6, 2)], None),
    ("b n h -> b h", [(3, 20, 16)], None),
    ("b n h, h -> b n h", [(3, 20, 16), (16,)], None),
    ("i i -> i", [(12, 12)], None),
    ("b (h p) c -> b h p c", [(2, 12, 5)], {"p": 4}),
    ("... i j, ... j k -> ... i k", [(3, 4, 6), (3, 6, 5)], None),
    ("a b, a b -> a", [(7, 9), (7, 9)], None),
]


@pytest.mark.parametrize("expr, shapes, sizes", EINSUM_CASES)
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_einshard_gradients(gpu, expr, shapes, sizes, dtype):
    xs = [randn(*shape, seed=10 + i, dtype=dtype) for i, shape in enumerate(shapes)]
    shape = einshard_cpu(expr, *xs, sizes=sizes).shape
    gz = randn(max(shape.numel(), 1), seed=99, dtype=dtype).reshape(shape)
    want, want_grads = _grads(lambda *t: einshard_cpu(expr, *t, sizes=sizes), xs, gz)
    got, got_grads = _grads(lambda *t: es.einshard(expr, *t, sizes=sizes), [x.to(gpu) for x in xs], gz)
    assert got.requires_grad is False  # detached copy; the live output carried a grad_fn
    assert_rel(got, want, TOL[dtype])
    for g, w in zip(got_grads, want_grads):
        assert g.shape == w.shape
        assert_rel(g, w, TOL[dtype])


def test_output_has_grad_fn_only_when_needed(gpu):
    x = torch.randn(8, 16, device=gpu)
    w = torch.randn(4, 16, device=gpu)
    assert es.einshard("n c, h c -> n h", x, w).grad_fn is None
    assert es.einshard("n c, h c -> n h", x.requires_grad_(), w).grad_fn is not None
    with torch.no_grad():
        assert es.einshard("n c, h c -> n h", x, w).grad_fn is None


WINDOW_CASES = [
    ("b h w c -> b h w kh kw c", {"h": "kh", "w": "kw"}, {"h": 1, "w": 1}, (2, 9, 7, 8)),
    ("b h w c -> b kh kw h w c", {"h": "kh", "w": "kw"}, {"h": (0, 2), "w": (3, 1)}, (2, 6, 9, 4)),
    ("t c -> t k c", {"t": "k"}, {"t": (4, 0)}, (11, 6)),
]


@pytest.mark.parametrize("expr, windows, radius, shape", WINDOW_CASES)
@pytest.mark.parametrize("boundary", ["constant", "replicate", "periodic"])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_einwindow_gradients(gpu, expr, windows, radius, shape, boundary, dtype):
    x = randn(*shape, seed=31, dtype=dtype)
    fwd_cpu = lambda t: einwindow_cpu(expr, t, windows, radius, boundary=boundary, fill=0.5)
    fwd_gpu = lambda t: es.einwindow(expr, t, windows, radius, boundary=boundary, fill=0.5)
    gz = randn(*fwd_cpu(x).shape, seed=32, dtype=dtype)
    want, (want_g,) = _grads(fwd_cpu, [x], gz)
    got, (got_g,) = _grads(fwd_gpu, [x.to(gpu)], gz)
    assert torch.equal(got.cpu(), want)
    assert_rel(got_g, want_g, TOL[dtype])


@pytest.mark.parametrize("boundary", ["constant", "replicate", "periodic"])
@pytest.mark.parametrize("halos", [{"a": (3, 9), "c": 2}, {"a": (7, 1)}])
def test_einhalo_gradients(gpu, boundary, halos):
    # {"a": (7, 1)} on an axis of 5: the periodic halo wraps more than once
    x = randn(5, 9, 12, seed=33)
    fwd_cpu = lambda t: einhalo_cpu("a b c", t, halos, boundary=boundary, fill=1.5)
    fwd_gpu = lambda t: es.einhalo("a b c", t, halos, boundary=boundary, fill=1.5)
    gz = randn(*fwd_cpu(x).shape, seed=34)
    want, (want_g,) = _grads(fwd_cpu, [x], gz)
    got, (got_g,) = _grads(fwd_gpu, [x.to(gpu)], gz)
    assert torch.equal(got.cpu(), want)
    assert_rel(got_g, want_g, TOL[torch.float32])


def test_halo_gradient_on_a_one_rank_mesh(gpu):
    # reference tests/test_halo.py:139-158 at world size 1: every element is read once
    class OneRank:
        mesh_dim_names = ("dp",)

        def __getitem__(self, name):
            class Dim:
                def size(self):
                    return 1

            return Dim()

    x = torch.arange(14, dtype=torch.float32, device=gpu).reshape(7, 2).requires_grad_(True)
    z = es.einhalo("a/dp b", x, {"a": 1}, mesh=OneRank(), fill=-1)
    z.sum().backward()
    assert torch.equal(x.grad.cpu(), torch.ones(7, 2))
