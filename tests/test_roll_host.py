"""es.einroll's host logic without a GPU: the reference's errors and warning
(src/torch_einshard/roll.py:10-45, tests/test_distributed_roll.py:23-27) are raised
before any device work; an unshifted call returns ``x`` itself, as the reference's
loop does; a shifted call on CPU tensors fails loudly (no CPU fallback)."""

import pytest
import torch

import torch_einshard as es


class _Mesh:
    """A mesh stand-in whose every group has ``ranks`` ranks."""

    mesh_dim_names = ("dp", "sp")

    def __init__(self, ranks):
        self.ranks = ranks

    def __getitem__(self, name):
        ranks = self.ranks

        class Dim:
            def size(self):
                return ranks

        return Dim()


def test_einroll_is_exported():
    assert "einroll" in es.__all__


def test_distributed_einroll_requires_mesh():
    # reference tests/test_distributed_roll.py:23-27
    with pytest.raises(ValueError, match="Distributed einroll operations require mesh"):
        es.einroll("a/dp b", torch.randn(4, 3), {"a": 1})


@pytest.mark.parametrize("shifts", [{}, {"a": 0}, {"z": 5}, {"a": 0, "b": 0}])
def test_no_shift_returns_the_input_itself(shifts):
    x = torch.randn(4, 3)
    assert es.einroll("a b", x, shifts) is x
    assert es.einroll("a b", x, shifts) is x  # the cached identity


def test_sharded_axis_without_shift_needs_no_mesh():
    x = torch.randn(4, 3)
    assert es.einroll("a/dp b", x, {"b": 0}) is x


def test_cpu_tensors_are_rejected_without_fallback():
    with pytest.raises(RuntimeError, match="MI355X"):
        es.einroll("a b", torch.randn(4, 3), {"a": 1})


def test_multi_rank_group_is_not_supported():
    with pytest.raises(NotImplementedError, match="slice exchange"):
        es.einroll("a/dp b", torch.randn(4, 3), {"a": 1}, mesh=_Mesh(2))


@pytest.mark.parametrize(
    "shapes, message",
    [
        ({"sp": [4]}, "Missing split shapes for mesh dimension 'dp'"),
        ({"dp": {"z": [4]}}, "Missing split shapes for axis 'a' on mesh dimension 'dp'"),
        ([2, 2], "passed shapes of size 2 not equal to 1"),
    ],
)
def test_split_shapes_are_checked(shapes, message):
    with pytest.raises(ValueError, match=message):
        es.einroll("a/dp b", torch.randn(4, 3), {"a": 1}, mesh=_Mesh(1), shapes=shapes)


def test_missing_shapes_warn_about_the_fallback():
    with pytest.warns(RuntimeWarning, match="gather/roll/split fallback"):
        with pytest.raises(RuntimeError, match="MI355X"):
            es.einroll("a/dp b", torch.randn(4, 3), {"a": 1}, mesh=_Mesh(1))


def test_spec_longer_than_tensor_is_an_index_error():
    # torch.roll(z, dims=2) on a 2-D tensor
    with pytest.raises(IndexError, match="Dimension out of range"):
        es.einroll("a b c", torch.randn(4, 3), {"c": 1})


def test_axis_families_expand_shift_tuples():
    with pytest.raises(RuntimeError, match="MI355X"):
        es.einroll("b *spatial", torch.randn(2, 3, 4), {"spatial": (1, -2)}, families={"spatial": ("h", "w")})
