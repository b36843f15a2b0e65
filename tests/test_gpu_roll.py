"""GPU parity of es.einroll: the reference's local test
(tests/test_distributed_roll.py:10-20) and its one-rank distributed cases on
device, then bit-exact sweeps against the oracle (``torch.roll`` per axis on the
CPU, the reference's own call) and gradients (the opposite roll)."""

import warnings

import pytest
import torch

import torch_einshard as es
from oracle.einshard_oracle import einroll_cpu
from torch_einshard import _native

from conftest import assert_bitexact, randn

pytestmark = pytest.mark.gpu


class _OneRank:
    mesh_dim_names = ("dp", "sp")

    def __getitem__(self, name):
        class Dim:
            def size(self):
                return 1

        return Dim()


def test_local_roll_axis_family(gpu):
    # reference tests/test_distributed_roll.py:10-20
    x = randn(2, 3, 4, 5, 6, 7, seed=1)
    z = es.einroll("b t *spatial c", x.to(gpu), {"spatial": (1, -2, 3)}, families={"spatial": ("h", "w", "d")})
    assert_bitexact(z, torch.roll(x, shifts=(1, -2, 3), dims=(2, 3, 4)))
    assert _native.last_kernel().startswith("gather")


CASES = [
    ("a b", (7, 5), {"a": 2}),
    ("a b", (7, 5), {"a": -9, "b": 3}),
    ("b h w c", (3, 10, 12, 8), {"h": 3, "w": -5}),
    ("b h w c", (3, 10, 12, 8), {"c": 1}),
    ("t x", (4, 6), {"x": 6}),  # a whole turn: a copy with the same values
    ("t x", (4, 6), {"x": 1000003, "t": -1000001}),
    ("a b c d e", (2, 3, 4, 5, 6), {"a": 1, "b": 1, "c": 1, "d": 1, "e": 1}),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float64, torch.int64, torch.uint8, torch.int16])
@pytest.mark.parametrize("spec, shape, shifts", CASES)
def test_roll_is_bitexact(gpu, spec, shape, shifts, dtype):
    x = (randn(*shape, seed=7) * 50).to(dtype)
    got = es.einroll(spec, x.to(gpu), shifts)
    assert_bitexact(got, einroll_cpu(spec, x, shifts))


def test_whole_turn_is_a_copy_not_an_alias(gpu):
    x = randn(4, 6, seed=8).to(gpu)
    got = es.einroll("t x", x, {"x": 6})
    assert got is not x and got.data_ptr() != x.data_ptr()
    assert_bitexact(got, x)


def test_strided_input(gpu):
    base = randn(8, 12, 10, seed=9).to(gpu)
    x = base.permute(2, 0, 1)[:, ::2]
    got = es.einroll("a b c", x, {"a": 4, "c": -3})
    assert_bitexact(got, einroll_cpu("a b c", x.cpu(), {"a": 4, "c": -3}))


def test_empty_axis(gpu):
    x = torch.empty(0, 5, device=gpu)
    assert tuple(es.einroll("a b", x, {"a": 2, "b": 1}).shape) == (0, 5)


def test_repeated_calls_replay_with_fresh_data(gpu):
    for seed in range(3):
        x = randn(6, 9, seed=20 + seed)
        assert_bitexact(es.einroll("a b", x.to(gpu), {"a": -2, "b": 4}), einroll_cpu("a b", x, {"a": -2, "b": 4}))


def test_one_rank_mesh_with_shapes(gpu):
    # reference tests/test_distributed_roll.py:30-47 at world size 1
    full = randn(3, 5, seed=30)
    x = full.to(gpu).requires_grad_(True)
    with warnings.catch_warnings():
        warnings.simplefilter("error")
        z = es.einroll("a/dp b", x, {"a": 2}, mesh=_OneRank(), shapes=[3])
    assert_bitexact(z.detach(), torch.roll(full, shifts=2, dims=0))
    (z**2).sum().backward()
    assert_bitexact(x.grad, 2 * full)


def test_one_rank_mesh_without_shapes_warns(gpu):
    # reference tests/test_distributed_roll.py:106-121 at world size 1
    full = randn(6, 5, seed=31)
    with pytest.warns(RuntimeWarning, match="gather/roll/split fallback"):
        z = es.einroll("a/dp b", full.to(gpu), {"a": 2}, mesh=_OneRank())
    assert_bitexact(z, torch.roll(full, shifts=2, dims=0))


def test_two_sharded_axes_on_one_rank_mesh(gpu):
    # reference tests/test_distributed_roll.py:124-146 at world size 1, uneven sizes
    full = randn(13, 17, seed=32)
    x = full.to(gpu).requires_grad_(True)
    z = es.einroll("a/sp b/dp", x, {"a": 5, "b": -4}, mesh=_OneRank(), shapes={"sp": [13], "dp": [17]})
    assert_bitexact(z.detach(), torch.roll(full, shifts=(5, -4), dims=(0, 1)))
    z.sum().backward()
    assert_bitexact(x.grad, torch.ones_like(full))


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_gradient_is_the_opposite_roll(gpu, dtype):
    x = randn(4, 9, 7, seed=40, dtype=dtype)
    gz = randn(4, 9, 7, seed=41, dtype=dtype)
    xg = x.to(gpu).requires_grad_(True)
    z = es.einroll("a b c", xg, {"b": 4, "c": -10})
    assert z.grad_fn is not None
    (gx,) = torch.autograd.grad(z, [xg], gz.to(gpu))
    xr = x.clone().requires_grad_(True)
    (rx,) = torch.autograd.grad(einroll_cpu("a b c", xr, {"b": 4, "c": -10}), [xr], gz)
    assert_bitexact(gx, rx)


def test_gradient_through_an_expanded_output_gradient(gpu):
    x = randn(5, 6, seed=42).to(gpu).requires_grad_(True)
    es.einroll("a b", x, {"a": 3}).sum().backward()
    assert_bitexact(x.grad, torch.ones(5, 6))


def test_benchmark_shape(gpu):
    # reference benchmarks/bench_local.py:212-229 at the "large" size
    x = randn(4, 128, 128, 128, seed=50)
    got = es.einroll("b h w c", x.to(gpu), {"h": 3, "w": -5})
    assert_bitexact(got, torch.roll(x, shifts=(3, -5), dims=(1, 2)))
