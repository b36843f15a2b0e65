"""The lowering, checked on the CPU: the exact descriptors the GPU receives are
executed by a strided fp64 interpreter (test-only) and compared with the oracle.

This pins the planner — label grouping, stride arithmetic, axis merging,
operand orientation, ellipsis / diagonal / broadcast handling — independently
of the kernels, which the GPU tests then hold to the same oracle."""

import pytest
import torch

from oracle.einshard_oracle import einshard_cpu
from torch_einshard.einsum import plan_local
from torch_einshard.families import cached_expand_axis_families
from torch_einshard.grammar import parse_sharding
from torch_einshard.planner import BcastOp, ContractOp, EmptyOp, GatherOp, ReduceOp, lower_einsum

from conftest import randn


def _view(t, axes, field):
    sizes = [axis.size for axis in axes]
    strides = [getattr(axis, field) for axis in axes]
    return torch.as_strided(t, sizes, strides, t.storage_offset())


def interpret(op, xs):
    """Evaluate a planner op on CPU tensors in fp64 using only its descriptors."""
    xs = [x.to(torch.float64) if x.is_floating_point() else x for x in xs]
    if isinstance(op, EmptyOp):
        return torch.empty(op.out_shape, dtype=torch.float64)
    if isinstance(op, GatherOp):
        return _view(xs[0], op.axes, "a").reshape(op.out_shape)
    if isinstance(op, BcastOp):
        return (_view(xs[0], op.axes, "a") * _view(xs[1], op.axes, "b")).reshape(op.out_shape)
    if isinstance(op, ReduceOp):
        axes = op.keep + op.red
        term = _view(xs[0], axes, "a")
        if op.has_y:
            term = term * _view(xs[1], axes, "b")
        dims = list(range(len(op.keep), len(axes)))
        total = term.sum(dim=dims) if dims else term
        return total.reshape(op.out_shape)
    if isinstance(op, ContractOp):
        a, b = (xs[1], xs[0]) if op.swapped else (xs[0], xs[1])
        av = _view(a, op.batch + op.m + op.k, "a")
        bv = _view(b, op.batch + op.n + op.k, "b")
        nb, nm, nn, nk = (len(op.batch), len(op.m), len(op.n), len(op.k))
        size = lambda axes: int(torch.tensor([x.size for x in axes], dtype=torch.int64).prod().item()) if axes else 1
        am = av.reshape(size(op.batch), size(op.m), size(op.k))
        bm = bv.reshape(size(op.batch), size(op.n), size(op.k))
        c = torch.bmm(am, bm.transpose(1, 2))
        out = torch.zeros(op.out_shape, dtype=torch.float64)
        target = torch.as_strided(out, [x.size for x in op.batch + op.m + op.n], [x.c for x in op.batch + op.m + op.n])
        target.copy_(c.reshape([x.size for x in op.batch + op.m + op.n]))
        del nb, nm, nn, nk
        return out
    raise TypeError(type(op))


def _f64_view(x):
    """The same view (shape, strides, offset) over a float64 copy of x's storage."""
    if x.dtype == torch.float64:
        return x
    count = x.untyped_storage().nbytes() // x.element_size()
    base = torch.empty(0, dtype=x.dtype).set_(x.untyped_storage(), 0, (count,), (1,))
    return torch.as_strided(base.to(torch.float64), x.shape, x.stride(), x.storage_offset())


def check(expression, *xs, sizes=None, families=None, expect=None):
    xs = [_f64_view(x) for x in xs]
    text, sizes = cached_expand_axis_families(expression, sizes, families)
    shard = parse_sharding(text)
    op, packed = plan_local(shard, *xs, sizes=sizes)
    if expect is not None:
        assert isinstance(op, expect), type(op).__name__
    got = interpret(op, xs)
    if packed is not None:
        got = got.reshape(packed)
    want = einshard_cpu(text, *[x.to(torch.float64) for x in xs], sizes=sizes)
    assert tuple(got.shape) == tuple(want.shape)
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)
    return op


CASES = [
    ("a b, b c -> a c", [(24, 20), (20, 32)], ContractOp),
    ("a b k c, b c l d -> k l d a", [(4, 5, 8, 6), (5, 6, 8, 3)], ContractOp),
    ("b n c, h c -> b n h", [(2, 24, 16), (20, 16)], ContractOp),
    ("b i k, b k j -> b i j", [(3, 17, 9), (3, 9, 18)], ContractOp),
    ("b i k, b j k -> b j i", [(3, 17, 9), (3, 18, 9)], ContractOp),
    ("a b, c -> a c", [(20, 7), (18,)], ContractOp),
    ("i i j, j -> i", [(5, 5, 7), (7,)], ReduceOp),
    ("a b, a b -> a", [(9, 13), (9, 13)], ReduceOp),
    ("a b, b -> a", [(30, 13), (13,)], ReduceOp),
    ("p b n h -> b n h", [(3, 2, 5, 8)], ReduceOp),
    ("b n h -> b h", [(2, 5, 8)], ReduceOp),
    ("b n h -> b n", [(2, 5, 8)], ReduceOp),
    ("a b c -> b", [(3, 4, 5)], ReduceOp),
    ("b n h, h -> b n h", [(2, 5, 8), (8,)], BcastOp),
    ("i, j -> i j", [(3,), (4,)], BcastOp),
    ("a, a -> a", [(7,), (7,)], BcastOp),
    ("a b, c d -> d b c a", [(2, 3), (4, 5)], BcastOp),
    ("i i -> i", [(5, 5)], GatherOp),
    ("a b c -> c b a", [(3, 4, 5)], GatherOp),
    ("b t c h w -> b t h w c", [(2, 3, 4, 5, 6)], GatherOp),
    ("... c, c o -> ... o", [(2, 9, 4), (4, 20)], ContractOp),
    ("... c, c o -> ... o", [(2, 3, 4), (4, 5)], ReduceOp),
    ("... c -> c", [(2, 3, 4)], ReduceOp),
    ("b ... c -> ... b c", [(2, 3, 4, 5)], GatherOp),
    ("a b -> a b", [(6, 7)], GatherOp),
]


@pytest.mark.parametrize("expression, shapes, kind", CASES)
def test_planner_matches_oracle(expression, shapes, kind):
    xs = [randn(*shape, seed=11 + i) for i, shape in enumerate(shapes)]
    check(expression, *xs, expect=kind)


@pytest.mark.parametrize("expression, shapes, kind", CASES)
def test_planner_on_permuted_inputs(expression, shapes, kind):
    # non-contiguous operands: a transposed buffer viewed back to the logical shape
    xs = []
    for i, shape in enumerate(shapes):
        base = randn(*reversed(shape), seed=40 + i)
        xs.append(base.permute(*reversed(range(len(shape)))))
    check(expression, *xs, expect=kind)


def test_planner_with_expanded_operand():
    x = randn(1, 6, seed=3).expand(5, 6)  # stride 0 along a
    w = randn(6, 4, seed=4)
    check("a b, b c -> a c", x, w)
    check("a b -> b", x)
    check("a b, b -> a b", x, randn(6, seed=5))


def test_planner_size_one_broadcast_and_sliced_operand():
    x = randn(4, 1, 6, seed=3)
    y = randn(4, 5, 6, seed=4)
    check("a b c, a b c -> a b c", x, y)
    big = randn(10, 12, seed=7)
    check("a b, b c -> a c", big[1:9:2, 2:10], randn(8, 3, seed=8))


def test_planner_factored_and_family_forms():
    check("b (h p) c -> b h p c", randn(2, 12, 5), sizes={"p": 4})
    check("b h p c -> b (h p) c", randn(2, 3, 4, 5))
    check("b (h p) c -> b c h p", randn(2, 12, 5), sizes={"h": 3})
    check("... (h p) c -> ... h p c", randn(2, 3, 12, 5), sizes={"p": 4})
    families = {"spatial": ("h", "w"), "window": ("wh", "ww")}
    check(
        "b t [*spatial *window] c -> (b *spatial) t *window c",
        randn(2, 3, 8, 10, 5),
        families=families,
        sizes={"window": (4, 5)},
    )


def test_contraction_orientation_puts_contiguous_output_axis_in_n():
    x = randn(64, 32, 128, 64)
    y = randn(32, 64, 128, 16)
    shard = parse_sharding("a b k c, b c l d -> k l d a")
    op, _ = plan_local(shard, x, y)
    assert isinstance(op, ContractOp) and op.swapped
    assert op.n[-1].c == 1 and op.n[-1].size == 64  # output's innermost axis a
    assert [(ax.size, ax.a) for ax in op.m] == [(2048, 1)]  # (l d) merged, contiguous in y
    assert [(ax.size, ax.b) for ax in op.k] == [(32, 8192), (64, 1)]  # K contiguous in x


def test_config4_lowers_to_one_nt_gemm():
    x = torch.empty(8, 2048, 4096, device="meta")
    w = torch.empty(1792, 4096, device="meta")
    op = lower_einsum([list("abc"), list("dc")], [x.shape, w.shape], [x.stride(), w.stride()], list("abd"))
    assert isinstance(op, ContractOp) and not op.swapped and not op.batch
    assert [(a.size, a.a, a.c) for a in op.m] == [(16384, 4096, 1792)]
    assert [(a.size, a.b, a.c) for a in op.n] == [(1792, 4096, 1)]
    assert [(a.size, a.a, a.b) for a in op.k] == [(4096, 1, 1)]


@pytest.mark.parametrize(
    "labels, shapes, out, message",
    [
        ([list("ab")], [(3,)], list("a"), "does not match the number of dimensions"),
        ([list("ii")], [(3, 4)], list("i"), "repeated for operand 0"),
        ([list("a"), list("a")], [(3,), (4,)], list("a"), "do not broadcast"),
        ([list("a")], [(3,)], list("aa"), "appears more than once"),
        ([list("a")], [(3,)], list("b"), "does not appear in the equation"),
    ],
)
def test_einsum_errors_match_torch_wording(labels, shapes, out, message):
    strides = [torch.empty(s).stride() for s in shapes]
    with pytest.raises(RuntimeError, match=message):
        lower_einsum(labels, shapes, strides, out)


def test_zero_sized_operands():
    op = lower_einsum([list("ab"), list("bc")], [(0, 3), (3, 4)], [(3, 1), (4, 1)], list("ac"))
    assert isinstance(op, EmptyOp) and op.out_shape == (0, 4)
    # an empty summed axis leaves zeros: the kernels receive K = 0
    op = lower_einsum([list("ab"), list("bc")], [(20, 0), (0, 24)], [(1, 1), (24, 1)], list("ac"))
    assert isinstance(op, ContractOp) and [a.size for a in op.k] == [0]
    assert interpret(op, [torch.empty(20, 0), torch.empty(0, 24)]).abs().sum() == 0


# ---- split-K planning (host only) -----------------------------------------------------


def test_split_k_cuts_the_outermost_k_axis():
    from torch_einshard._exec import _split_k
    from torch_einshard.planner import ContractOp, SubAxis

    # the einconv weight gradient of the benchmark: 256 x 2304 outputs over 16 x 64 x 64 positions
    op = ContractOp((256, 2304), swapped=False, m=[SubAxis(256, a=1, c=2304)], n=[SubAxis(2304, b=1, c=1)],
                    k=[SubAxis(16, a=1048576, b=1115136), SubAxis(64, a=16384, b=16896), SubAxis(64, a=256, b=256)])
    split, parts = _split_k(op)
    assert parts == 8
    assert split.out_shape == (8, 256, 2304)
    # the split axis runs first in the batch group and steps over whole parts
    head = split.batch[0]
    assert (head.size, head.a, head.b, head.c) == (8, 2 * 1048576, 2 * 1115136, 256 * 2304)
    assert [(a.size, a.a, a.b) for a in split.k] == [(2, 1048576, 1115136), (64, 16384, 16896), (64, 256, 256)]


def test_split_k_leaves_busy_or_short_contractions_alone():
    from torch_einshard._exec import _split_k
    from torch_einshard.planner import ContractOp, SubAxis

    def op(m, n, k):
        return ContractOp((m, n), swapped=False, m=[SubAxis(m, a=k, c=n)], n=[SubAxis(n, b=k, c=1)],
                          k=[SubAxis(k, a=1, b=1)])

    assert _split_k(op(4096, 4096, 65536))[1] == 1  # enough tiles already
    assert _split_k(op(256, 256, 4096))[1] == 1     # K too short to pay
    assert _split_k(op(64, 64, 8191))[1] == 1       # a prime K has no divisor to cut at
    assert _split_k(op(64, 64, 16384))[1] == 32     # parts keep at least 512 of K


def test_split_k_planned_contraction_checks_its_arithmetic():
    # interpret the split op in fp64 on the CPU: partial sums over each part, then their sum
    import torch

    from torch_einshard._exec import _split_k
    from torch_einshard.planner import ContractOp, SubAxis

    m, n, k = 3, 5, 16384
    x = torch.randn(k, m, dtype=torch.float64)
    y = torch.randn(k, n, dtype=torch.float64)
    op = ContractOp((m, n), swapped=False, m=[SubAxis(m, a=1, c=n)], n=[SubAxis(n, b=1, c=1)],
                    k=[SubAxis(k, a=m, b=n)])
    split, parts = _split_k(op)
    head, rest = split.batch[0], split.k[0]
    xf, yf = x.reshape(-1), y.reshape(-1)
    partial = torch.zeros(parts, m, n, dtype=torch.float64)
    for s in range(parts):
        for r in range(rest.size):
            ia = s * head.a + r * rest.a
            ib = s * head.b + r * rest.b
            partial[s] += torch.outer(xf[ia : ia + m], yf[ib : ib + n])
    torch.testing.assert_close(partial.sum(0), x.T @ y)


def test_split_k_targets_the_pipelined_kernel_for_16_bit_weight_gradients():
    from torch_einshard._exec import _split_k
    from torch_einshard.planner import ContractOp, SubAxis

    # config 4's weight gradient (b n h, b n c -> h c): 7 x 16 tiles of 256 x 256 over
    # K = 16384, both operands contiguous along their rows.  Four parts make 448 tiles
    # for the pipelined kernel; without the element size only the 128 x 128 rule runs.
    def wgrad(m, n, k, k_inner_a=None):
        return ContractOp((m, n), swapped=False, m=[SubAxis(m, a=1, c=n)], n=[SubAxis(n, b=1, c=1)],
                          k=[SubAxis(k, a=k_inner_a or m, b=n)])

    split, parts = _split_k(wgrad(1792, 4096, 16384), 2)
    assert parts == 4
    assert [(a.size, a.a, a.b) for a in split.k] == [(4096, 1792, 4096)]
    head = split.batch[0]
    assert (head.size, head.a, head.b, head.c) == (4, 4096 * 1792, 4096 * 4096, 1792 * 4096)
    assert _split_k(wgrad(1792, 4096, 16384))[1] == 1
    # parts of at least 1024 of K, and enough tiles that every CU has one
    assert _split_k(wgrad(1024, 2048, 8192), 2)[1] == 8
    assert _split_k(wgrad(1024, 2048, 4096), 2)[1] == 1  # K shorter than the split minimum
    # operands the pipelined kernel cannot read in place keep the 128 x 128 rule:
    # row strides that are not a multiple of 8 elements
    assert _split_k(wgrad(1792, 4096, 16384, k_inner_a=1793), 2)[1] == 1
    # a whole number of 64-deep K tiles is required, in the whole K and in each part
    assert _split_k(wgrad(1792, 4096, 16383), 2)[1] == 1
    assert _split_k(wgrad(1792, 4096, 64 * 257), 2)[1] == 1  # 257 tiles: no whole-tile cut


def test_split_k_cut_through_two_k_axes_checks_its_arithmetic(monkeypatch):
    # A short outer K sub-axis is cut whole and the next one in parts (an einconv
    # weight gradient: 16 batch rows of positions).  Thresholds are lowered so that a
    # small case takes this cut; the split op is interpreted in fp64 from its
    # descriptors, and its partials must sum to the contraction.
    from torch_einshard import _exec

    monkeypatch.setattr(_exec, "_CU_TILES", 16)
    monkeypatch.setattr(_exec, "_PIPE_K_PART", 64)
    monkeypatch.setattr(_exec, "_PIPE_FIXED", 0)
    monkeypatch.setattr(_exec, "_SPLIT_MIN_K", 1024)
    b, h, w, o, t = 2, 16, 64, 256, 512
    gz = torch.randn(b, h, w + 8, o, dtype=torch.float64)[:, :, :w]  # K sub-axes that do not merge
    xp = torch.randn(b, h + 2, w, t, dtype=torch.float64)[:, :h]
    op = lower_einsum([list("bhwo"), list("bhwt")], [tuple(gz.shape), tuple(xp.shape)],
                      [gz.stride(), xp.stride()], list("ot"))
    assert [a.size for a in op.k] == [2, 16, 64]
    split, parts = _exec._split_k(op, 2)
    assert parts == 8  # 2 whole outer rows x 4 runs of the second sub-axis
    assert [a.size for a in split.batch] == [2, 4] and [a.size for a in split.k] == [4, 64]
    partial = interpret(split, [gz, xp])
    assert partial.shape == (8, o, t)
    torch.testing.assert_close(partial.sum(0), torch.einsum("bhwo,bhwt->ot", gz, xp))
    # every part covers a distinct quarter of one outer row
    for p in range(parts):
        i, j = divmod(p, 4)
        want = torch.einsum("hwo,hwt->ot", gz[i, 4 * j:4 * j + 4], xp[i, 4 * j:4 * j + 4])
        torch.testing.assert_close(partial[p], want)
