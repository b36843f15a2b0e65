"""Split-shape helpers of the reference's ``torch_einshard.helpers`` that callers and
tests use to describe uneven shards (reference src/torch_einshard/helpers.py:312-361).
The reference's collective helpers in the same module (all-reduce, all-gather, halo and
roll exchanges) move data between ranks and have no counterpart in this one-GPU build.
"""

from .mesh_util import split_shapes

__all__ = ["compute_split_shapes", "compute_split_shapes_for_factors", "resolve_split_shapes"]


def compute_split_shapes(size, num_chunks):
    """Extents of ``num_chunks`` shards of an axis of ``size``: equal shards of
    ceil(size / num_chunks) with the remainder last, or, when that would leave the last
    shard empty, equal shards of floor(size / num_chunks) with the remainder last
    (reference helpers.py:336-351)."""
    if num_chunks == 1:
        return [size]
    each = -(-size // num_chunks)
    last = size - each * (num_chunks - 1)
    if last <= 0:
        each = size // num_chunks
        last = size - each * (num_chunks - 1)
    return [each] * (num_chunks - 1) + [last]


def compute_split_shapes_for_factors(size, num_chunks, factor):
    """compute_split_shapes over whole groups of ``factor`` elements, the leftover
    elements on the last shard (reference helpers.py:354-361)."""
    shards = compute_split_shapes(size // factor, num_chunks)
    if factor == 1:
        return shards
    shards = [extent * factor for extent in shards]
    shards[-1] += size % factor
    return shards


def resolve_split_shapes(shapes, shard_dim, axis_name, group=None):
    """The shard extents of ``axis_name`` on mesh dim ``shard_dim`` from ``shapes`` (a
    list, ``{dim: list}`` or ``{dim: {axis: list}}``), checked against the group's size
    when a process group is given (reference helpers.py:312-333)."""
    if group is None:
        if shapes is None:
            return None
        found = split_shapes(shapes, shard_dim, axis_name, None)
        return found
    import torch.distributed as dist

    return split_shapes(shapes, shard_dim, axis_name, dist.get_world_size(group))
