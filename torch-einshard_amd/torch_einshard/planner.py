"""Lowering of a labelled einsum onto the four device operations.

The reference hands ``"abkc,bcld->klda"``-style equations to ``torch.einsum``
(reference: src/torch_einshard/einsum.py:132).  Here the same semantics — the
subset of ``torch.einsum`` an einshard expression can produce — are lowered to
strided descriptors executed by the HIP library:

* ``GatherOp``    unary, nothing summed: permutation / diagonal / copy;
* ``ReduceOp``    unary with summed labels, or a binary contraction too thin for
                  a matrix tile (``min(M, N) < 16``): out = sum_red x (* y);
* ``BcastOp``     binary, nothing summed: out = x * y with broadcasting;
* ``ContractOp``  binary with summed labels: batched GEMM over label groups
                  {batch, M, N, K}, each a list of strided sub-axes.

``torch.einsum`` rules honoured (errors are ``RuntimeError`` like torch's):
ellipsis dims are right-aligned and broadcast across operands and summed when
the output has no ``...``; a label repeated inside one operand takes the
diagonal (its stride is the sum of the repeated dims' strides); a label of size
1 in one operand broadcasts against the other operand (stride 0).

Nothing is copied or transposed on the host: operands keep their own strides,
labels are grouped and adjacent labels are merged when every operand that
carries them agrees (``stride[outer] == stride[inner] * size[inner]``).
Outputs are always dense in output-label order.
"""

from dataclasses import dataclass, field

__all__ = [
    "ELLIPSIS",
    "SubAxis",
    "GatherOp",
    "ReduceOp",
    "BcastOp",
    "ContractOp",
    "EmptyOp",
    "lower_einsum",
    "dense_strides",
    "THIN_CONTRACTION",
]

ELLIPSIS = "..."
# below this many rows or columns a contraction is run as a product-reduction
THIN_CONTRACTION = 16


@dataclass
class SubAxis:
    """One (possibly merged) iteration axis: its extent and per-operand strides.

    ``a`` / ``b`` are the strides (in elements) in the first / second input of
    the device op and ``c`` the stride in the output; 0 means the operand does
    not vary along this axis.
    """

    size: int
    a: int = 0
    b: int = 0
    c: int = 0
    label: str = ""


@dataclass
class GatherOp:
    out_shape: tuple
    axes: list  # output order; a = source stride


@dataclass
class ReduceOp:
    out_shape: tuple
    keep: list  # output order (dense output); a = x stride, b = y stride
    red: list  # a = x stride, b = y stride
    has_y: bool


@dataclass
class BcastOp:
    out_shape: tuple
    axes: list  # output order; a = x stride, b = y stride


@dataclass
class ContractOp:
    out_shape: tuple
    swapped: bool  # True: device A operand is the second input
    batch: list = field(default_factory=list)
    m: list = field(default_factory=list)
    n: list = field(default_factory=list)
    k: list = field(default_factory=list)


@dataclass
class EmptyOp:
    out_shape: tuple


def dense_strides(shape):
    strides = []
    running = 1
    for size in reversed(shape):
        strides.append(running)
        running *= size
    return tuple(reversed(strides))


def _label_text(label):
    return label if isinstance(label, str) else str(label)


def _expand_operand(index, labels, shape, strides, ell_labels_total):
    """Return the operand's dims as (label, size, stride) with ``...`` expanded."""
    named = [label for label in labels if label != ELLIPSIS]
    has_ellipsis = len(named) != len(labels)
    rank = len(shape)
    if not has_ellipsis and len(named) != rank:
        raise RuntimeError(
            f"einsum(): the number of subscripts in the equation ({len(named)}) does not match "
            f"the number of dimensions ({rank}) for operand {index} and no ellipsis was given"
        )
    if has_ellipsis and len(named) > rank:
        raise RuntimeError(
            f"einsum(): the number of subscripts in the equation ({len(named)}) is more than "
            f"the number of dimensions ({rank}) for operand {index}"
        )
    ell_rank = rank - len(named)
    dims = []
    dim = 0
    for label in labels:
        if label == ELLIPSIS:
            first = ell_labels_total - ell_rank
            for j in range(ell_rank):
                dims.append((("...", first + j), shape[dim], strides[dim]))
                dim += 1
        else:
            dims.append((label, shape[dim], strides[dim]))
            dim += 1
    return dims


def _ellipsis_rank(labels, shape):
    named = sum(1 for label in labels if label != ELLIPSIS)
    return max(len(shape) - named, 0) if ELLIPSIS in labels else 0


def lower_einsum(input_labels, shapes, strides, output_labels):
    """Lower an einsum over one or two strided operands.

    ``input_labels``: per operand, a list of hashable labels, optionally with one
    ``ELLIPSIS``.  ``shapes`` / ``strides``: per operand, sizes and element
    strides.  ``output_labels``: labels of the result (may hold ``ELLIPSIS``).
    Returns one of the op dataclasses of this module.
    """
    n_ops = len(input_labels)
    if n_ops not in (1, 2):
        raise ValueError("einshard expressions take one or two inputs")
    ell_total = max(_ellipsis_rank(labels, shape) for labels, shape in zip(input_labels, shapes))
    operands = [
        _expand_operand(i, input_labels[i], tuple(shapes[i]), tuple(strides[i]), ell_total)
        for i in range(n_ops)
    ]

    # output labels with the ellipsis expanded
    out_labels = []
    for label in output_labels:
        if label == ELLIPSIS:
            out_labels.extend(("...", j) for j in range(ell_total))
        else:
            out_labels.append(label)
    seen = set()
    for label in out_labels:
        if label in seen:
            raise RuntimeError(
                f"einsum(): output subscript {_label_text(label)} appears more than once in the output"
            )
        seen.add(label)

    # per operand: label -> (size, summed stride)
    per_operand = []
    for index, dims in enumerate(operands):
        table = {}
        for label, size, stride in dims:
            if label in table:
                prev_size, prev_stride = table[label]
                if prev_size != size:
                    raise RuntimeError(
                        f"einsum(): subscript {_label_text(label)} is repeated for operand {index} "
                        f"but the sizes don't match, {prev_size} != {size}"
                    )
                table[label] = (size, prev_stride + stride)
            else:
                table[label] = (size, stride)
        per_operand.append(table)

    order = []  # all labels, first-seen order over inputs
    for table in per_operand:
        for label in table:
            if label not in order:
                order.append(label)
    for label in out_labels:
        if label not in order:
            raise RuntimeError(
                f"einsum(): output subscript {_label_text(label)} does not appear in the equation "
                f"for any input operand"
            )

    sizes = {}
    for label in order:
        candidates = {table[label][0] for table in per_operand if label in table}
        wide = candidates - {1}
        if len(wide) > 1:
            raise RuntimeError(
                "einsum(): operands do not broadcast with remapped shapes (original->remapped): "
                + " ".join(str(tuple(shape)) for shape in shapes)
            )
        sizes[label] = wide.pop() if wide else 1

    def stride_in(operand, label):
        table = per_operand[operand]
        if label not in table:
            return 0
        size, stride = table[label]
        if size == 1:
            return 0  # broadcast (or trivial) along this label
        return stride

    out_shape = tuple(sizes[label] for label in out_labels)
    out_strides = dict(zip(out_labels, dense_strides(out_shape)))
    if 0 in out_shape:
        return EmptyOp(out_shape)

    out_set = set(out_labels)
    live_out = [label for label in out_labels if sizes[label] != 1]
    summed = [label for label in order if label not in out_set and sizes[label] != 1]
    # a summed label of size 0 leaves a sum over nothing: kernels write zeros

    def sub(label, a_op=None, b_op=None, c=True):
        return SubAxis(
            size=sizes[label],
            a=stride_in(a_op, label) if a_op is not None else 0,
            b=stride_in(b_op, label) if b_op is not None else 0,
            c=out_strides[label] if c and label in out_strides else 0,
            label=_label_text(label),
        )

    if n_ops == 1:
        if not summed:
            axes = [sub(label, a_op=0) for label in live_out]
            return GatherOp(out_shape, _merge(axes, ("a", "c")))
        keep = [sub(label, a_op=0) for label in live_out]
        red = [sub(label, a_op=0, c=False) for label in summed]
        red.sort(key=lambda axis: -axis.a)
        return ReduceOp(out_shape, _merge(keep, ("a", "c")), _merge(red, ("a",)), has_y=False)

    x_has = {label for label in order if stride_in(0, label) != 0 or _trivially_present(per_operand[0], label, sizes)}
    y_has = {label for label in order if stride_in(1, label) != 0 or _trivially_present(per_operand[1], label, sizes)}

    if not summed:
        axes = [sub(label, a_op=0, b_op=1) for label in live_out]
        return BcastOp(out_shape, _merge(axes, ("a", "b", "c")))

    m_labels = [label for label in live_out if label in x_has and label not in y_has]
    n_labels = [label for label in live_out if label not in x_has and label in y_has]
    # batch: both operands vary along it — or neither does (an expanded view),
    # in which case every batch index recomputes and stores the same tile
    batch = [label for label in live_out if label not in m_labels and label not in n_labels]

    m_extent = _product(sizes[label] for label in m_labels)
    n_extent = _product(sizes[label] for label in n_labels)
    if min(m_extent, n_extent) < THIN_CONTRACTION:
        keep = [sub(label, a_op=0, b_op=1) for label in live_out]
        red = [sub(label, a_op=0, b_op=1, c=False) for label in summed]
        red.sort(key=lambda axis: (-axis.a, -axis.b))
        return ReduceOp(out_shape, _merge(keep, ("a", "b", "c")), _merge(red, ("a", "b")), has_y=True)

    # orientation: the output's innermost live label must be a device-N label
    swapped = bool(live_out) and live_out[-1] in m_labels
    a_op, b_op = (1, 0) if swapped else (0, 1)
    if swapped:
        m_labels, n_labels = n_labels, m_labels

    batch_axes = sorted((sub(label, a_op, b_op) for label in batch), key=lambda axis: -axis.c)
    m_axes = sorted((sub(label, a_op, b_op) for label in m_labels), key=lambda axis: (-axis.a, -axis.c))
    n_axes = sorted((sub(label, a_op, b_op) for label in n_labels), key=lambda axis: (-axis.c, -axis.b))
    k_axes = [sub(label, a_op, b_op, c=False) for label in summed]
    if any(axis.a == 1 for axis in k_axes):
        k_axes.sort(key=lambda axis: (-axis.a, -axis.b))
    else:
        k_axes.sort(key=lambda axis: (-axis.b, -axis.a))

    return ContractOp(
        out_shape,
        swapped,
        batch=_merge(batch_axes, ("a", "b", "c")),
        m=_merge(m_axes, ("a", "c")),
        n=_merge(n_axes, ("b", "c")),
        k=_merge(k_axes, ("a", "b")),
    )


def _trivially_present(table, label, sizes):
    # a label of global size 1 present in the operand: irrelevant for grouping
    return label in table and sizes[label] == 1


def _product(values):
    result = 1
    for value in values:
        result *= value
    return result


def _merge(axes, fields):
    """Merge neighbouring sub-axes (outer first) that form one strided run in every field."""
    merged = []
    for axis in axes:
        if merged:
            outer = merged[-1]
            if all(getattr(outer, f) == getattr(axis, f) * axis.size for f in fields):
                merged[-1] = SubAxis(
                    size=outer.size * axis.size,
                    a=axis.a,
                    b=axis.b,
                    c=axis.c,
                    label=outer.label + axis.label,
                )
                continue
        merged.append(SubAxis(axis.size, axis.a, axis.b, axis.c, axis.label))
    return merged
