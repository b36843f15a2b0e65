"""Notation AST: axes, groups, ellipsis, partials and operand annotations.

Mirrors the observable behaviour of the reference's AST types
(reference: src/torch_einshard/sharding.py:4-232):

* ``Axis(name, shard_dim)`` compares and hashes on *both* fields, so ``a`` and
  ``a/tp`` are different axes (sharding.py:21-28).
* ``Axes`` is a list with ``local()`` / ``flat()`` / ``all_shard_dims()``
  (sharding.py:65-89).
* ``TensorSpec`` holds at most one ellipsis (sharding.py:205-210).
* Annotation dataclasses parse ``param`` / ``grad=`` / ``init_sync=`` items
  (sharding.py:92-202); their ``repr`` round-trips through the parser.
"""

from dataclasses import dataclass

__all__ = [
    "Axis",
    "EllipsisAxis",
    "AxisGroup",
    "Axes",
    "GradAnnotation",
    "InitSyncAnnotation",
    "TensorAnnotation",
    "TensorSpec",
]


class Axis:
    """A named axis, optionally sharded over a mesh dimension (``h/tp``)."""

    __slots__ = ("name", "shard_dim")

    def __init__(self, name: str, shard_dim: str = "") -> None:
        self.name = name
        self.shard_dim = shard_dim

    def local(self) -> bool:
        return self.shard_dim == ""

    def __repr__(self) -> str:
        return self.name if self.local() else f"{self.name} / {self.shard_dim}"

    def __hash__(self) -> int:
        return hash((Axis, self.name, self.shard_dim))

    def __eq__(self, other: object):
        if not isinstance(other, Axis):
            return NotImplemented
        return (self.name, self.shard_dim) == (other.name, other.shard_dim)


class EllipsisAxis:
    """``...``: the leading/trailing dimensions not named in the spec."""

    name = "..."
    shard_dim = ""

    def local(self) -> bool:
        return True

    def __repr__(self) -> str:
        return "..."

    def __hash__(self) -> int:
        return hash(EllipsisAxis)

    def __eq__(self, other: object):
        return isinstance(other, EllipsisAxis)


class Axes(list):
    """Ordered axes of one tensor spec (``Axis``, ``AxisGroup`` or ``EllipsisAxis``)."""

    def __repr__(self) -> str:
        return " × ".join(repr(axis) for axis in self)

    def local(self) -> bool:
        return all(axis.local() for axis in self)

    def all_shard_dims(self):
        dims = []
        for item in self:
            members = item.axes if isinstance(item, AxisGroup) else (item,)
            dims.extend(axis.shard_dim for axis in members if axis.shard_dim)
        return dims

    def flat(self) -> "Axes":
        out = Axes()
        for item in self:
            if isinstance(item, AxisGroup):
                out.extend(item.axes)
            else:
                out.append(item)
        return out


class AxisGroup:
    """A factored dimension ``(h p)``: one tensor dim holding several axes."""

    def __init__(self, axes) -> None:
        self.axes = Axes(axes)

    def local(self) -> bool:
        return self.axes.local()

    def __iter__(self):
        return iter(self.axes)

    def __len__(self) -> int:
        return len(self.axes)

    def __repr__(self) -> str:
        return "(" + " ".join(repr(axis) for axis in self.axes) + ")"


_GRAD_SUFFIX_BACKENDS = {"ddp": "ddp", "external": "external"}
_RESERVED_GRAD_WORDS = {"async", "ddp", "external", "none"}


@dataclass(frozen=True)
class GradAnnotation:
    """``grad=<value>`` of a ``[param, ...]`` annotation (reference sharding.py:92-139)."""

    mode: str = "inferred"
    mesh_dims: tuple = ()
    backend: str = "native"
    schedule: str = "backend_default"

    @classmethod
    def from_value(cls, value: str) -> "GradAnnotation":
        if ":" in value:
            mesh_dim, suffix = value.rsplit(":", 1)
            if not mesh_dim or not suffix:
                raise ValueError("Invalid grad annotation")
            if mesh_dim in _RESERVED_GRAD_WORDS:
                raise ValueError("Grad annotation suffix requires an explicit mesh group")
            if suffix == "async":
                return cls("explicit", (mesh_dim,), "native", "async")
            if suffix in _GRAD_SUFFIX_BACKENDS:
                return cls("explicit", (mesh_dim,), _GRAD_SUFFIX_BACKENDS[suffix])
            raise ValueError(f"Unknown grad annotation suffix {suffix!r}")
        if value == "async":
            return cls(schedule="async")
        if value in _GRAD_SUFFIX_BACKENDS:
            return cls(backend=_GRAD_SUFFIX_BACKENDS[value])
        if value == "none":
            return cls(mode="none", backend="none")
        return cls(mode="explicit", mesh_dims=(value,))

    def __repr__(self) -> str:
        if self.mode == "none":
            return "none"
        if self.mode == "inferred":
            if self.backend == "native" and self.schedule == "async":
                return "async"
            if self.backend in ("ddp", "external"):
                return self.backend
        if self.mode == "explicit" and self.mesh_dims:
            head = self.mesh_dims[0]
            if self.backend == "native" and self.schedule == "async":
                return f"{head}:async"
            if self.backend in ("ddp", "external"):
                return f"{head}:{self.backend}"
            return head
        return "inferred"


@dataclass(frozen=True)
class InitSyncAnnotation:
    """``init_sync=<value>`` of a ``[param, ...]`` annotation (reference sharding.py:142-162)."""

    mode: str = "inferred"
    mesh_dims: tuple = ()

    @classmethod
    def from_value(cls, value: str) -> "InitSyncAnnotation":
        if ":" in value:
            raise ValueError("init_sync annotations do not accept suffixes")
        if value in ("none", "external"):
            return cls(mode=value)
        return cls(mode="explicit", mesh_dims=(value,))

    def __repr__(self) -> str:
        if self.mode in ("none", "external"):
            return self.mode
        if self.mode == "explicit" and self.mesh_dims:
            return self.mesh_dims[0]
        return "inferred"


@dataclass(frozen=True)
class TensorAnnotation:
    """Operand annotation ``[param, grad=..., init_sync=...]`` (reference sharding.py:165-202)."""

    is_param: bool = False
    grad: object = None
    init_sync: object = None

    @classmethod
    def from_items(cls, items) -> "TensorAnnotation":
        fields = {}
        for key, value in items:
            if key in fields:
                raise ValueError(f"Duplicate tensor annotation {key!r}")
            if key == "param":
                fields[key] = True
            elif key == "grad":
                fields[key] = GradAnnotation.from_value(value)
            elif key == "init_sync":
                fields[key] = InitSyncAnnotation.from_value(value)
            else:
                raise ValueError(f"Unknown tensor annotation {key!r}")
        return cls(
            is_param=fields.get("param", False),
            grad=fields.get("grad"),
            init_sync=fields.get("init_sync"),
        )

    def __bool__(self) -> bool:
        return self.is_param or self.grad is not None or self.init_sync is not None

    def __repr__(self) -> str:
        parts = ["param"] if self.is_param else []
        if self.grad is not None:
            parts.append(f"grad={self.grad!r}")
        if self.init_sync is not None:
            parts.append(f"init_sync={self.init_sync!r}")
        return "[" + ", ".join(parts) + "]"


class TensorSpec:
    """One operand/result of an expression: axes, partial mesh dims, annotation."""

    def __init__(self, axes, partials=None, annotation=None) -> None:
        if sum(1 for axis in axes if isinstance(axis, EllipsisAxis)) > 1:
            raise ValueError("Tensor specs may contain at most one ellipsis")
        self.axes = axes
        self.partials = tuple(partials or ())
        self.annotation = annotation or TensorAnnotation()

    def local(self) -> bool:
        return self.axes.local() and not self.partials

    def __iter__(self):
        return iter(self.axes)

    def __len__(self) -> int:
        return len(self.axes)

    def __getitem__(self, key):
        return self.axes[key]

    def __repr__(self) -> str:
        text = repr(self.axes)
        if self.partials:
            if len(self.partials) == 1:
                text += f" // {self.partials[0]}"
            else:
                text += " // (" + ",".join(self.partials) + ")"
        if self.annotation:
            text += f" {self.annotation!r}"
        return text
