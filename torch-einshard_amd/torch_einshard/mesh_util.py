"""Mesh helpers for the single-GPU build.

A mesh is accepted so that ``// tp`` partial specs and ``h/tp`` sharded specs
keep working (reference: src/torch_einshard/__init__.py:178-185,
src/torch_einshard/mesh.py:15-103), but every mesh group an operation uses
must have exactly one rank: collectives across GPUs are not part of this build.
On a one-rank group every collective of the reference is the identity on values
(an all-reduce of one contribution, a split into one piece, a gather of one
piece).
"""

__all__ = ["mesh_group_size", "mesh_dim_names", "require_single_rank"]


def mesh_dim_names(mesh):
    names = getattr(mesh, "mesh_dim_names", None)
    if names is None and hasattr(mesh, "mesh"):
        names = getattr(mesh.mesh, "mesh_dim_names", None)
    return tuple(names or ())


def _component_size(mesh, name):
    try:
        sub = mesh[name]
    except (KeyError, IndexError, TypeError, RuntimeError, ValueError) as error:
        raise ValueError(f"Unknown mesh dimension {name!r}") from error
    size = getattr(sub, "size", None)
    if callable(size):
        return int(size())
    if hasattr(sub, "get_group"):
        import torch.distributed as dist

        return dist.get_world_size(sub.get_group())
    raise ValueError(f"Cannot determine the size of mesh dimension {name!r}")


def mesh_group_size(mesh, name):
    """Ranks in the mesh group ``name``; a hyphenated name spans several dims."""
    names = mesh_dim_names(mesh)
    if name in names or "-" not in name:
        return _component_size(mesh, name)
    total = 1
    for part in name.split("-"):
        total *= _component_size(mesh, part)
    return total


def require_single_rank(mesh, groups, what):
    for group in groups:
        if mesh_group_size(mesh, group) != 1:
            raise NotImplementedError(
                f"{what}: mesh group {group!r} has more than one rank; this build runs on one GPU "
                "and supports meshes whose groups have one rank"
            )
