"""Host-side rules of non-local expressions on a one-rank mesh (no GPU needed).

Step names follow the reference's transition rules
(src/torch_einshard/symbolic.py:472-570) and the expectations its tests assert:
split / gather round trips (tests/test_distributed_unary.py:31, :35), owner
swaps (:200, :228, :293, :373), the row-parallel plan
(tests/test_distributed_binary.py:107-110, :129).  Errors: a sharded or partial
spec without a mesh (reference __init__.py:182-183), a mesh group with more
than one rank (this build runs on one GPU).
"""

import pytest
import torch

import torch_einshard as es
from torch_einshard.distributed import binary_plan_steps, unary_plan_steps
from torch_einshard.grammar import parse_sharding


def _unary(expr):
    x, _, z = parse_sharding(expr)
    return [name for name, _ in unary_plan_steps(list(x.axes), x.partials, list(z.axes), z.partials)]


def _binary(expr):
    x, y, z = parse_sharding(expr)
    return [name for name, _ in binary_plan_steps(list(x.axes), list(y.axes), list(z.axes), z.partials)]


@pytest.mark.parametrize(
    "expr, steps",
    [
        ("a b // tp -> a b", ["allreduce_forward_identity_backward"]),
        ("a b -> a b // tp", ["identity_forward_allreduce_backward"]),
        ("a b // tp -> a/tp b", ["reducescatter_forward_allgather_backward"]),
        ("a/tp b -> a b // tp", ["allgather_forward_reducescatter_backward"]),
        ("loss // (sp,dp) -> loss", ["allreduce_forward_identity_backward"] * 2),
        ("loss // dp-sp -> loss", ["allreduce_forward_identity_backward"]),
        ("a b // tp -> b a // tp", ["permute"]),
        ("a b -> a/dp b", ["split_forward_allgather_backward"]),
        ("a/dp b -> a b", ["allgather_forward_split_backward"]),
        # owner swaps (reference tests/test_distributed_unary.py:200, :228, :293, :373)
        ("a/dp b -> a/sp b", ["owner_swap"]),
        ("a/dp b/sp -> a/sp b/dp", ["owner_swap"]),
        ("a/dp b -> a/sp b/tp", ["owner_swap", "split_forward_allgather_backward"]),
        # an unchanged axis on an involved dim: gather / split instead (reference :249-262)
        ("a/dp c/sp b -> a/sp c/sp b", ["allgather_forward_split_backward", "split_forward_allgather_backward"]),
    ],
)
def test_unary_transition_steps(expr, steps):
    assert _unary(expr) == steps


def test_binary_plans():
    assert _binary("b n c/tp, h c/tp -> b n h") == ["rank_local_einsum", "allreduce_forward_identity_backward"]
    assert _binary("b n c/tp, h c/tp -> b n h // tp") == ["rank_local_einsum"]


def test_distributed_einshard_requires_mesh():
    # refused before any device check: the mesh is needed to plan at all
    with pytest.raises(ValueError, match="Distributed einshard operations require mesh"):
        es.einshard("a b -> a/dp b", torch.randn(4, 3))
    with pytest.raises(ValueError, match="Distributed einshard operations require mesh"):
        es.einshard("a b // tp -> a b", torch.randn(4, 3))
    with pytest.raises(ValueError, match="Distributed einshard operations require mesh"):
        es.einshard_like("a b -> a/dp b", torch.randn(4, 3))


def test_wrap_mesh_gives_a_compound_mesh(mesh_2d):
    # reference src/torch_einshard/mesh.py:15-70
    from torch_einshard.mesh_util import mesh_group_size

    wrapped = es.wrap_mesh(mesh_2d)
    assert isinstance(wrapped, es.CompoundDeviceMesh)
    assert es.wrap_mesh(wrapped) is wrapped
    assert wrapped.mesh_dim_names == ("dp", "sp")
    group = wrapped["dp-sp"].get_group()
    assert torch.distributed.get_world_size(group) == 1
    assert wrapped["sp-dp"].get_group() is group  # one group per set of dims
    assert wrapped["dp"].size() == 1
    for mesh in (wrapped, mesh_2d):
        assert mesh_group_size(mesh, "dp-sp") == 1
        assert mesh_group_size(mesh, "sp") == 1
    with pytest.raises(ValueError, match="cannot contain empty mesh dimensions"):
        wrapped["dp-"]
    with pytest.raises(ValueError, match="cannot repeat mesh dimensions"):
        wrapped["dp-dp"]


class _Names:
    """A mesh stand-in with the given dim names over a grid of matching rank."""

    def __init__(self, names, rank=None):
        self.mesh_dim_names = names
        n = rank if rank is not None else (len(names) if isinstance(names, tuple) else 1)
        self.mesh = torch.zeros((1,) * n, dtype=torch.int64)


@pytest.mark.parametrize(
    "names, error, message",
    [
        (("dp", 3), TypeError, "entries must be strings"),
        (torch.zeros(2), TypeError, "must be an iterable of strings"),
        (5, TypeError, "must be an iterable of strings"),
        (("dp", ""), ValueError, "must be non-empty strings"),
        (("dp-",), ValueError, "cannot contain empty compound components"),
        (("dp-dp",), ValueError, "cannot repeat compound components"),
        (("dp", "dp-sp"), ValueError, "cannot overlap compound components"),
        (("dp", "dp"), ValueError, "cannot overlap compound components"),
    ],
)
def test_compound_mesh_checks_dim_names(names, error, message):
    with pytest.raises(error, match=message):
        es.wrap_mesh(_Names(names, rank=2 if isinstance(names, tuple) and len(names) == 2 else 1))


def test_compound_mesh_needs_one_name_per_dim():
    with pytest.raises(ValueError, match="mesh_dim_names length must match mesh rank"):
        es.wrap_mesh(_Names(("dp", "sp"), rank=3))


class _Mesh:
    """A mesh stand-in: named dims of ``ranks`` ranks each."""

    def __init__(self, names, ranks):
        self.mesh_dim_names = names
        self.ranks = ranks

    def __getitem__(self, name):
        if name not in self.mesh_dim_names:
            raise KeyError(name)
        ranks = self.ranks

        class Sub:
            def size(self):
                return ranks

        return Sub()


def test_group_sizes_are_checked_before_any_work():
    with pytest.raises(NotImplementedError, match="more than one rank"):
        es.einshard("a b // tp -> a b", torch.randn(4, 3), mesh=_Mesh(("tp",), 2))
    with pytest.raises(ValueError, match="Unknown mesh dimension"):
        es.einshard("a b // xx -> a b", torch.randn(4, 3), mesh=_Mesh(("tp",), 1))
