"""Gradient assembly of the einsum backward (host logic): the device launch inside
``einsum_labels`` is replaced by torch.einsum on CPU tensors, and every gradient is
compared with torch's own autograd through the same equation in float64."""

import pytest
import torch

from torch_einshard import autograd
from torch_einshard.planner import ELLIPSIS


def _cpu_einsum_labels(xs, input_labels, output_labels):
    letters = {}

    def text(labels):
        out = ""
        for label in labels:
            if label == ELLIPSIS:
                out += "..."
                continue
            if label not in letters:
                letters[label] = "abcdefghijklmnopqrstuvwxyz"[len(letters)]
            out += letters[label]
        return out

    ins = [text(labels) for labels in input_labels]
    return torch.einsum(",".join(ins) + "->" + text(output_labels), *[x.detach() for x in xs])


CASES = [
    ("ab,bc->ac", [(3, 4), (4, 5)]),
    ("bij,bjk->bik", [(2, 3, 4), (2, 4, 5)]),
    ("abc->b", [(3, 4, 5)]),
    ("abc->cba", [(3, 4, 5)]),
    ("ab,b->ab", [(3, 4), (4,)]),
    ("i,j->ij", [(3,), (4,)]),
    ("ii->i", [(4, 4)]),
    ("iij,jk->ik", [(3, 3, 4), (4, 2)]),
    ("abc,cd->ad", [(2, 3, 4), (4, 5)]),
    ("ab,ab->", [(3, 4), (3, 4)]),
    ("ab,cb->ac", [(1, 4), (5, 4)]),
]


@pytest.mark.parametrize("equation, shapes", CASES)
def test_gradients_match_torch(monkeypatch, equation, shapes):
    monkeypatch.setattr(autograd, "einsum_labels", _cpu_einsum_labels)
    lhs, rhs = equation.split("->")
    input_labels = [list(part) for part in lhs.split(",")]
    g = torch.Generator().manual_seed(5)
    xs = [torch.randn(*shape, generator=g, dtype=torch.float64, requires_grad=True) for shape in shapes]
    got = autograd.differentiable_einsum(xs, input_labels, list(rhs))
    gz = torch.randn(got.shape, generator=g, dtype=torch.float64)
    grads = torch.autograd.grad(got, xs, gz)
    ref_xs = [x.detach().clone().requires_grad_(True) for x in xs]
    want = torch.einsum(equation, *ref_xs)
    assert torch.allclose(got.detach(), want.detach())
    want_grads = torch.autograd.grad(want, ref_xs, gz)
    for a, b in zip(grads, want_grads):
        assert a.shape == b.shape
        assert torch.allclose(a, b)


def test_ellipsis_broadcast_gradient_is_summed(monkeypatch):
    monkeypatch.setattr(autograd, "einsum_labels", _cpu_einsum_labels)
    g = torch.Generator().manual_seed(6)
    x = torch.randn(1, 3, 4, generator=g, dtype=torch.float64, requires_grad=True)
    y = torch.randn(5, 4, 2, generator=g, dtype=torch.float64, requires_grad=True)
    got = autograd.differentiable_einsum([x, y], [[ELLIPSIS, "i", "j"], [ELLIPSIS, "j", "k"]], [ELLIPSIS, "i", "k"])
    gz = torch.randn(got.shape, generator=g, dtype=torch.float64)
    gx, gy = torch.autograd.grad(got, [x, y], gz)
    xr, yr = x.detach().clone().requires_grad_(True), y.detach().clone().requires_grad_(True)
    want = torch.einsum("...ij,...jk->...ik", xr, yr)
    wx, wy = torch.autograd.grad(want, [xr, yr], gz)
    assert torch.allclose(gx, wx) and gx.shape == x.shape
    assert torch.allclose(gy, wy)


def test_planted_mistake_is_caught(monkeypatch):
    # a gradient that forgets the diagonal scatter would not match torch
    monkeypatch.setattr(autograd, "einsum_labels", _cpu_einsum_labels)
    x = torch.randn(4, 4, dtype=torch.float64, requires_grad=True)
    got = autograd.differentiable_einsum([x], [["i", "i"]], ["i"])
    (gx,) = torch.autograd.grad(got.sum(), [x])
    assert torch.equal(gx, torch.eye(4, dtype=torch.float64))
    assert not torch.equal(gx, torch.ones(4, 4, dtype=torch.float64))
