"""Split shapes on sharded halo and window axes, checked on the host before any
device work (einconv checks its operands' device first; its split-shape check runs in
tests/test_gpu_sharded.py) (reference src/torch_einshard/halo.py:267-285 and
helpers.py:312-351): the group count, the local extent against this rank's split
shape, and the reference's split-shape helpers."""

import pytest
import torch

import torch_einshard as es


@pytest.mark.parametrize(
    "size, chunks, want",
    [(13, 4, [4, 4, 4, 1]), (12, 4, [3, 3, 3, 3]), (9, 4, [2, 2, 2, 3]), (4, 1, [4]), (0, 3, [0, 0, 0])],
)
def test_compute_split_shapes(size, chunks, want):
    # 9 over 4: ceil gives 3, 3, 3 and an empty last shard, so floor is used: 2, 2, 2, 3
    got = es.helpers.compute_split_shapes(size, chunks)
    assert got == want and sum(got) == size


def test_compute_split_shapes_for_factors():
    # whole groups of 4: 10 groups over 3 shards (4, 4, 2), leftover 3 elements last
    assert es.helpers.compute_split_shapes_for_factors(43, 3, 4) == [16, 16, 11]
    assert es.helpers.compute_split_shapes_for_factors(13, 4, 1) == [4, 4, 4, 1]


def test_resolve_split_shapes(mesh_1d):
    group = mesh_1d["dp"].get_group()
    assert es.helpers.resolve_split_shapes(None, "dp", "a", group) is None
    assert es.helpers.resolve_split_shapes({"dp": {"a": [7]}}, "dp", "a", group) == [7]
    with pytest.raises(ValueError, match="passed shapes of size 2 not equal to 1"):
        es.helpers.resolve_split_shapes([3, 4], "dp", "a", group)


def test_einhalo_local_size_must_match_the_split_shape(mesh_1d):
    with pytest.raises(ValueError, match="Local tensor size 4 does not match split shape 5 for axis 'a'"):
        es.einhalo("a/dp b", torch.zeros(4, 2), {"a": 1}, mesh=mesh_1d, shapes=[5])


@pytest.mark.parametrize(
    "shapes, message",
    [
        ({"sp": [4]}, "Missing split shapes for mesh dimension 'dp'"),
        ({"dp": {"z": [4]}}, "Missing split shapes for axis 'a' on mesh dimension 'dp'"),
        ([2, 2], "passed shapes of size 2 not equal to 1"),
    ],
)
def test_einhalo_split_shapes_are_resolved_like_the_reference(mesh_1d, shapes, message):
    with pytest.raises(ValueError, match=message):
        es.einhalo("a/dp b", torch.zeros(4, 2), {"a": 1}, mesh=mesh_1d, shapes=shapes)


def test_einwindow_local_size_must_match_the_split_shape(mesh_1d):
    with pytest.raises(ValueError, match="Local tensor size 4 does not match split shape 3 for axis 'a'"):
        es.einwindow("a/dp b -> a/dp k b", torch.zeros(4, 1), {"a": "k"}, {"a": 1}, mesh=mesh_1d, shapes={"dp": [3]})


def test_matching_split_shapes_reach_the_device_check(mesh_1d):
    # the checks pass; the CPU tensor is then rejected (no CPU fallback)
    with pytest.raises(RuntimeError, match="MI355X"):
        es.einhalo("a/dp b", torch.zeros(4, 2), {"a": 1}, mesh=mesh_1d, shapes=[4])


def test_an_unpadded_sharded_axis_is_not_checked(mesh_1d):
    # the reference skips axes with no halo before looking at split shapes
    with pytest.raises(RuntimeError, match="MI355X"):
        es.einhalo("a/dp b", torch.zeros(4, 2), {"b": 1}, mesh=mesh_1d, shapes=[9])
