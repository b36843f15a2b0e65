"""Mesh helpers for the single-GPU build.

A mesh is accepted so that ``// tp`` partial specs and ``h/tp`` sharded specs
keep working (reference: src/torch_einshard/__init__.py:178-185,
src/torch_einshard/mesh.py:15-103), but every mesh group an operation uses
must have exactly one rank: collectives across GPUs are not part of this build.
On a one-rank group every collective of the reference is the identity on values
(an all-reduce of one contribution, a split into one piece, a gather of one
piece).
"""

__all__ = ["CompoundDeviceMesh", "mesh_group_size", "mesh_dim_names", "require_single_rank", "split_shapes", "wrap_mesh"]


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


_MISSING = object()


def split_shapes(shapes, shard_dim, axis_name, group_size):
    """The per-rank extents of ``axis_name`` on mesh dim ``shard_dim`` given by ``shapes``
    (a list, ``{dim: list}`` or ``{dim: {axis: list}}``), checked against the group
    size (not checked when it is None); None without ``shapes`` (reference
    helpers.py:312-333)."""
    if shapes is None:
        return None
    found = shapes
    if isinstance(found, dict):
        found = found.get(shard_dim, _MISSING)
        if found is _MISSING:
            raise ValueError(f"Missing split shapes for mesh dimension {shard_dim!r}")
    if isinstance(shapes, dict) and isinstance(found, dict):
        found = found.get(axis_name, _MISSING)
        if found is _MISSING:
            raise ValueError(f"Missing split shapes for axis {axis_name!r} on mesh dimension {shard_dim!r}")
    if group_size is not None and len(found) != group_size:
        raise ValueError(f"Error: passed shapes of size {len(found)} not equal to {group_size}")
    return found


def require_single_rank(mesh, groups, what):
    for group in groups:
        if mesh_group_size(mesh, group) != 1:
            raise NotImplementedError(
                f"{what}: mesh group {group!r} has more than one rank; this build runs on one GPU "
                "and supports meshes whose groups have one rank"
            )


class _MeshDim:
    """A mesh dimension standing for one process group (what ``mesh[name]`` gives)."""

    def __init__(self, group):
        self.group = group

    def get_group(self):
        return self.group

    def size(self):
        import torch.distributed as dist

        return dist.get_world_size(self.group)


def _checked_dim_names(names):
    """``mesh_dim_names`` as a tuple of strings, with the reference's checks and
    messages (reference src/torch_einshard/mesh.py:73-103): strings only, non-empty,
    hyphenated components non-empty and not repeated, no component shared by two
    entries, no entry twice."""
    import torch

    if names is None:
        return ()
    if isinstance(names, str):
        found = (names,)
    elif isinstance(names, torch.Tensor) or (hasattr(names, "shape") and hasattr(names, "dtype")):
        raise TypeError("mesh_dim_names must be an iterable of strings")
    else:
        try:
            found = tuple(names)
        except TypeError as error:
            raise TypeError("mesh_dim_names must be an iterable of strings") from error
    if not all(isinstance(name, str) for name in found):
        raise TypeError("mesh_dim_names entries must be strings")
    if not all(found):
        raise ValueError("mesh_dim_names entries must be non-empty strings")
    seen = set()
    for name in found:
        parts = name.split("-")
        if not all(parts):
            raise ValueError("mesh_dim_names entries cannot contain empty compound components")
        if len(set(parts)) != len(parts):
            raise ValueError("mesh_dim_names entries cannot repeat compound components")
        if seen & set(parts):
            raise ValueError("mesh_dim_names entries cannot overlap compound components")
        seen.update(parts)
    if len(set(found)) != len(found):
        raise ValueError("mesh_dim_names entries must be unique")
    return found


class CompoundDeviceMesh:
    """A device mesh whose hyphenated names (``"dp-sp"``) index the process group that
    spans those dims (reference src/torch_einshard/mesh.py:15-70).

    ``mesh["dp-sp"]`` gives an object with ``get_group()``: the ranks that share every
    other mesh coordinate with this one.  Such a group is created once per name, with
    ``torch.distributed.new_group`` called by every rank for every such rank set (a
    collective, as group creation is).  Plain names go to the wrapped mesh."""

    def __init__(self, device_mesh):
        self.device_mesh = device_mesh
        self.mesh = device_mesh.mesh
        self.mesh_dim_names = _checked_dim_names(device_mesh.mesh_dim_names)
        if len(self.mesh_dim_names) != self.mesh.dim():
            raise ValueError("mesh_dim_names length must match mesh rank")
        self._dim_of = {name: dim for dim, name in enumerate(self.mesh_dim_names)}
        self._groups = {}

    def __getitem__(self, name):
        if name in self._dim_of or "-" not in name:
            return self.device_mesh[name]
        parts = tuple(name.split("-"))
        if not all(parts):
            raise ValueError("Compound mesh groups cannot contain empty mesh dimensions")
        if len(set(parts)) != len(parts):
            raise ValueError("Compound mesh groups cannot repeat mesh dimensions")
        if not all(part in self._dim_of for part in parts):
            return self.device_mesh[name]
        return _MeshDim(self._group(parts))

    def _group(self, parts):
        import itertools

        import torch.distributed as dist

        dims = tuple(sorted(self._dim_of[part] for part in parts))
        if dims in self._groups:
            return self._groups[dims]
        if not dist.is_initialized():
            raise RuntimeError("Compound mesh groups require an initialized process group")
        grid = self.mesh.detach().cpu()
        fixed = [d for d in range(grid.dim()) if d not in dims]
        me = dist.get_rank()
        mine = None
        # one group per coordinate of the other dims, in the same order on every rank
        for coord in itertools.product(*(range(grid.shape[d]) for d in fixed)):
            index = [slice(None)] * grid.dim()
            for d, c in zip(fixed, coord):
                index[d] = c
            ranks = [int(r) for r in grid[tuple(index)].reshape(-1).tolist()]
            group = dist.new_group(ranks=ranks)
            if me in ranks:
                mine = group
        self._groups[dims] = mine
        return mine


def wrap_mesh(mesh):
    """A :class:`CompoundDeviceMesh` over ``mesh`` (``mesh`` itself when it is one),
    as the reference's ``wrap_mesh`` (mesh.py:66-70).  Every lookup in this package also
    resolves a hyphenated name on an unwrapped mesh (``mesh_group_size``)."""
    if isinstance(mesh, CompoundDeviceMesh):
        return mesh
    return CompoundDeviceMesh(mesh)
