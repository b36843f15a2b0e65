"""GPU parity of es.einshard against the CPU oracle (the reference's CPU path).

The first block ports every local test of the reference's tests/test_einsum.py
onto device tensors; the rest sweeps dtypes, layouts, edge sizes and the four
kernel families.  Tolerances: fp32 1e-5 and bf16 2e-2 relative (with a scale
floor), bit-exact for copies and single-rounding products."""

import pytest
import torch

import torch_einshard as es
from oracle.einshard_oracle import einshard_cpu
from torch_einshard import _native
from torch_einshard.symbolic import last_plan

from conftest import TOL, assert_bitexact, assert_bitexact_nan, assert_rel, gen, on_device, randn

pytestmark = pytest.mark.gpu


def dev(t, gpu):
    return t.to(gpu)


# ---- reference tests/test_einsum.py, on the GPU ---------------------------------------


def test_contract_permute(gpu):
    x, y = randn(4, 5, 8, 6, seed=333), randn(5, 6, 8, 3, seed=334)
    z = es.einshard("a b k c, b c l d -> k l d a", dev(x, gpu), dev(y, gpu))
    assert z.is_cuda
    assert_rel(z, torch.einsum("abkc,bcld->klda", x, y), 1e-5)
    assert [step.name for step in last_plan()] == ["rank_local_einsum"]


def test_outer(gpu):
    x, y = randn(3, seed=1), randn(4, seed=2)
    assert_bitexact(es.einshard("i, j -> i j", dev(x, gpu), dev(y, gpu)), torch.einsum("i,j->ij", x, y))


def test_local_einshard_accepts_optimization_policy_arguments(gpu):
    x, y = dev(randn(3, seed=1), gpu), dev(randn(4, seed=2), gpu)
    want = torch.einsum("i,j->ij", x.cpu(), y.cpu())
    assert_bitexact(es.einshard("i, j -> i j", x, y, optimize="memory"), want)
    assert_bitexact(es.einshard("i, j -> i j", x, y, policy=es.PlanPolicy.from_mode("communication")), want)


def test_einshard_rejects_ambiguous_policy_arguments(gpu):
    with pytest.raises(ValueError, match="either optimize or policy"):
        es.einshard("i -> i", dev(randn(3), gpu), optimize="memory", policy=es.PlanPolicy.from_mode("training"))


def test_optimize_context_applies_to_existing_call_sites(gpu):
    x, y = dev(randn(3, seed=1), gpu), dev(randn(4, seed=2), gpu)
    with es.optimize("memory"):
        z = es.einshard("i, j -> i j", x, y)
    assert_bitexact(z, torch.einsum("i,j->ij", x.cpu(), y.cpu()))


def test_diagonal(gpu):
    x = randn(5, 5, seed=333)
    assert_bitexact(es.einshard("i i -> i", dev(x, gpu)), torch.einsum("ii->i", x))


def test_ellipsis_contract(gpu):
    x, w = randn(2, 3, 4, seed=1), randn(4, 5, seed=2)
    assert_rel(es.einshard("... c, c o -> ... o", dev(x, gpu), dev(w, gpu)), torch.einsum("...c,co->...o", x, w), 1e-5)


def test_ellipsis_reduction(gpu):
    x = randn(2, 3, 4, seed=1)
    assert_rel(es.einshard("... c -> c", dev(x, gpu)), torch.einsum("...c->c", x), 1e-5)


def test_ellipsis_permutation(gpu):
    x = randn(2, 3, 4, 5, seed=1)
    assert_bitexact(es.einshard("b ... c -> ... b c", dev(x, gpu)), torch.einsum("b...c->...bc", x))


def test_ellipsis_with_factored_axis(gpu):
    x = randn(2, 3, 12, 5)
    assert_bitexact(es.einshard("... (h p) c -> ... h p c", dev(x, gpu), sizes={"p": 4}), x.reshape(2, 3, 3, 4, 5))


def test_axis_families_window_partition_2d(gpu):
    x = randn(2, 3, 8, 10, 5)
    z = es.einshard(
        "b t [*spatial *window] c -> (b *spatial) t *window c",
        dev(x, gpu),
        families={"spatial": ("h", "w"), "window": ("wh", "ww")},
        sizes={"window": (4, 5)},
    )
    expected = x.reshape(2, 3, 2, 4, 2, 5, 5).permute(0, 2, 4, 1, 3, 5, 6).reshape(8, 3, 4, 5, 5)
    assert_bitexact(z, expected)


def test_axis_families_window_partition_3d(gpu):
    x = randn(2, 3, 8, 10, 6, 5)
    z = es.einshard(
        "b t [*spatial *window] c -> (b *spatial) t *window c",
        dev(x, gpu),
        families={"spatial": ("h", "w", "d"), "window": ("wh", "ww", "wd")},
        sizes={"window": (4, 5, 3)},
    )
    expected = x.reshape(2, 3, 2, 4, 2, 5, 2, 3, 5).permute(0, 2, 4, 6, 1, 3, 5, 7, 8).reshape(16, 3, 4, 5, 3, 5)
    assert_bitexact(z, expected)


def test_axis_families_window_reverse_3d(gpu):
    windows = randn(16, 3, 4, 5, 3, 5)
    z = es.einshard(
        "(b *spatial) t *window c -> b t [*spatial *window] c",
        dev(windows, gpu),
        families={"spatial": ("h", "w", "d"), "window": ("wh", "ww", "wd")},
        sizes={"b": 2, "h": 2, "w": 2, "d": 2},
    )
    expected = windows.reshape(2, 2, 2, 2, 3, 4, 5, 3, 5).permute(0, 4, 1, 5, 2, 6, 3, 7, 8).reshape(2, 3, 8, 10, 6, 5)
    assert_bitexact(z, expected)


def test_axis_family_sizes_expand_by_family_name(gpu):
    x = randn(2, 12, 5)
    z = es.einshard("b (*factors) c -> b *factors c", dev(x, gpu), families={"factors": ("h", "p")}, sizes={"factors": (3, 4)})
    assert_bitexact(z, x.reshape(2, 3, 4, 5))


def test_axis_family_rejects_mismatched_zipped_lengths(gpu):
    with pytest.raises(ValueError, match="matching lengths"):
        es.einshard(
            "b t [*spatial *window] c -> b t *spatial *window c",
            dev(randn(2, 3, 8, 10, 5), gpu),
            families={"spatial": ("h", "w"), "window": ("wh",)},
        )


def test_expand_factored_axis(gpu):
    x = randn(2, 12, 5)
    assert_bitexact(es.einshard("b (h p) c -> b h p c", dev(x, gpu), sizes={"p": 4}), x.reshape(2, 3, 4, 5))


def test_pack_factored_axis(gpu):
    x = randn(2, 3, 4, 5)
    assert_bitexact(es.einshard("b h p c -> b (h p) c", dev(x, gpu)), x.reshape(2, 12, 5))


def test_factored_axis_with_permutation(gpu):
    x = randn(2, 12, 5)
    z = es.einshard("b (h p) c -> b c h p", dev(x, gpu), sizes={"h": 3})
    assert_bitexact(z, x.reshape(2, 3, 4, 5).permute(0, 3, 1, 2))


def test_factored_axis_requires_unique_inference(gpu):
    with pytest.raises(ValueError, match="Cannot infer multiple factor sizes"):
        es.einshard("b (h p) c -> b h p c", dev(randn(2, 12, 5), gpu))


def test_factored_axis_allows_sharded_annotation_locally(gpu):
    x = randn(2, 12, 5)
    assert_bitexact(es.einshard("b (h/sp p) c -> b h/sp p c", dev(x, gpu), sizes={"p": 4}), x.reshape(2, 3, 4, 5))


def test_factored_axis_rejects_nonlocal_distributed_transform(gpu):
    with pytest.raises(NotImplementedError, match="local reshape operations"):
        es.einshard("b (h p) c -> b h/sp p c", dev(randn(2, 12, 5), gpu), sizes={"p": 4})


# ---- kernel families across dtypes and layouts -------------------------------------

FAMILY_CASES = [
    ("a b, b c -> a c", [(70, 45), (45, 90)]),
    ("a b k c, b c l d -> k l d a", [(16, 4, 24, 16), (4, 16, 24, 8)]),
    ("b n c, h c -> b n h", [(2, 96, 64), (80, 64)]),
    ("b i k, b k j -> b i j", [(3, 40, 24), (3, 24, 48)]),
    ("b i k, b j k -> b j i", [(3, 40, 24), (3, 48, 24)]),
    ("a b, a b -> a", [(33, 130), (33, 130)]),
    ("a b, b -> a", [(300, 70), (70,)]),
    ("p b n h -> b n h", [(4, 3, 20, 64)]),
    ("b n h -> b h", [(3, 50, 72)]),
    ("b n h -> b n", [(3, 50, 72)]),
    ("b n h, h -> b n h", [(3, 20, 64), (64,)]),
    ("i, j -> i j", [(30,), (41,)]),
    ("a b c -> c a b", [(5, 6, 7)]),
    ("i i j, j -> i", [(6, 6, 9), (9,)]),
]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("expression, shapes", FAMILY_CASES)
def test_family_parity(gpu, expression, shapes, dtype):
    xs = [randn(*s, seed=7 + i, dtype=dtype) for i, s in enumerate(shapes)]
    got = es.einshard(expression, *[dev(x, gpu) for x in xs])
    want = einshard_cpu(expression, *[x.float() for x in xs]).to(dtype)
    assert got.dtype == dtype
    assert_rel(got, want, TOL[dtype])
    if dtype != torch.float32:
        # also the reference's own path for 16-bit inputs: torch.einsum on the 16-bit
        # CPU tensors (reference src/torch_einshard/einsum.py:132)
        assert_rel(got, einshard_cpu(expression, *xs), TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("expression, shapes", FAMILY_CASES)
def test_family_parity_on_transposed_buffers(gpu, expression, shapes, dtype):
    xs = []
    for i, shape in enumerate(shapes):
        base = randn(*reversed(shape), seed=50 + i, dtype=dtype).to(gpu)
        xs.append(base.permute(*reversed(range(len(shape)))))
    got = es.einshard(expression, *xs)
    want = einshard_cpu(expression, *[x.cpu().float() for x in xs]).to(dtype)
    assert_rel(got, want, TOL[dtype])


GEMM_SHAPES = [(256, 256, 64), (512, 384, 256), (100, 130, 70), (33, 64, 192), (1000, 48, 512), (64, 2048, 128)]


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("layout", ["nt", "nn", "tn", "tt"])
@pytest.mark.parametrize("m, n, k", GEMM_SHAPES)
def test_gemm_layouts(gpu, m, n, k, layout, dtype):
    x = randn(m, k, seed=m + k, dtype=dtype)
    w = randn(n, k, seed=n + 3 * k, dtype=dtype)
    xd, wd = x.to(gpu), w.to(gpu)
    if layout[0] == "t":
        xd = x.t().contiguous().to(gpu).t()  # M contiguous
    if layout[1] == "n":
        wd = w.t().contiguous().to(gpu).t()  # N contiguous
    got = es.einshard("m k, n k -> m n", xd, wd)
    want = einshard_cpu("m k, n k -> m n", x.float(), w.float()).to(dtype)
    assert_rel(got, want, TOL[dtype])
    if dtype != torch.float32:
        assert_rel(got, einshard_cpu("m k, n k -> m n", x, w), TOL[dtype])  # the 16-bit CPU path


@pytest.mark.parametrize("layout", ["nt", "nn", "tn", "tt"])
@pytest.mark.parametrize("m, n, k", [(200, 136, 96), (64, 64, 32), (1024, 1024, 1024), (36, 1000, 4096)])
def test_fp32_64x64_kernels(gpu, m, n, k, layout):
    # fp32 on 64 x 64 tiles, both operands copied by LDS-DMA in their own layout
    # (K-contiguous or contiguous along M / N); ragged M and N edges.  A K-contiguous x
    # takes the four-wave pipelined kernel (w either way), an M-contiguous one the
    # eight-wave kernel of six stages
    x = randn(m, k, seed=m + 5 * k)
    w = randn(n, k, seed=n + 7 * k)
    xd = x.to(gpu) if layout[0] == "n" else x.t().contiguous().to(gpu).t()
    wd = w.to(gpu) if layout[1] == "t" else w.t().contiguous().to(gpu).t()
    got = es.einshard("m k, n k -> m n", xd, wd)
    want_kernel = "contract_f32_pipe_64x64" if layout[0] == "n" else "contract_f32_deep_64x64"
    assert _native.last_kernel() == want_kernel
    assert_rel(got, einshard_cpu("m k, n k -> m n", x, w), TOL[torch.float32])


@pytest.mark.parametrize("m, n", [(200, 135), (130, 67), (33, 250)])
def test_fp32_pipelined_kernel_element_stores(gpu, m, n):
    # an N that is not a multiple of 4 (both operands K-contiguous): the pipelined fp32
    # kernel writes the output one element at a time, the last column group partly
    x = randn(m, 96, seed=m + 11)
    w = randn(n, 96, seed=n + 13)
    got = es.einshard("m k, n k -> m n", x.to(gpu), w.to(gpu))
    assert _native.last_kernel() == "contract_f32_pipe_64x64", _native.last_kernel()
    assert_rel(got, einshard_cpu("m k, n k -> m n", x, w), TOL[torch.float32])


@pytest.mark.parametrize("w_layout", ["k", "n"])
@pytest.mark.parametrize("case", ["two K levels", "two M sub-axes", "both"])
def test_fp32_pipelined_kernel_walks(gpu, case, w_layout):
    # contract_f32_pipe's bounded walks: K in two sub-axes that do not merge (x stores b
    # outside m: K levels (b, c)), M in two (x's a and e swapped in memory), ragged edges;
    # w K-contiguous ([n, b, c]) or N-contiguous ([b, c, n])
    m_axes = "a e" if case != "two K levels" else "m"
    k_axes = "b c" if case != "two M sub-axes" else "c"
    sizes = {"m": 200, "a": 10, "e": 20, "b": 3, "c": 64, "n": 136}
    x_order = {"two K levels": "b m c", "two M sub-axes": "e a c", "both": "b e a c"}[case]
    x_base = randn(*[sizes[v] for v in x_order.split()], seed=91)
    x_logical = f"{m_axes} {k_axes}"
    xd = x_base.to(gpu).permute(*[x_order.split().index(v) for v in x_logical.split()])
    w_order = f"n {k_axes}" if w_layout == "k" else f"{k_axes} n"
    w_base = randn(*[sizes[v] for v in w_order.split()], seed=92)
    w_logical = f"n {k_axes}"
    wd = w_base.to(gpu).permute(*[w_order.split().index(v) for v in w_logical.split()])
    expr = f"{x_logical}, {w_logical} -> {m_axes} n"
    got = es.einshard(expr, xd, wd)
    assert _native.last_kernel() == "contract_f32_pipe_64x64", _native.last_kernel()
    want = einshard_cpu(expr, xd.cpu().contiguous(), wd.cpu().contiguous())
    assert_rel(got, want, TOL[torch.float32])


def test_gemm_uses_fast_layouts(gpu):
    x = randn(512, 256, dtype=torch.bfloat16).to(gpu)
    w = randn(384, 256, dtype=torch.bfloat16).to(gpu)
    es.einshard("m k, n k -> m n", x, w)
    assert _native.last_kernel().startswith("contract_") and "generic" not in _native.last_kernel()


def test_contraction_with_empty_sum_writes_zeros(gpu):
    x = torch.empty(40, 0, device=gpu)
    y = torch.empty(0, 24, device=gpu)
    z = es.einshard("a b, b c -> a c", x, y)
    assert z.shape == (40, 24) and torch.count_nonzero(z).item() == 0


def test_empty_output(gpu):
    x = torch.empty(0, 5, device=gpu)
    y = torch.empty(5, 3, device=gpu)
    assert es.einshard("a b, b c -> a c", x, y).shape == (0, 3)


def test_copies_are_bitexact_for_integer_and_double(gpu):
    for dtype in (torch.int32, torch.int64, torch.float64, torch.uint8, torch.int16):
        x = (randn(3, 4, 5) * 50).to(dtype)
        assert_bitexact(es.einshard("a b c -> c a b", x.to(gpu)), x.permute(2, 0, 1))


def test_broadcast_product_is_bitexact(gpu):
    for dtype in (torch.float32, torch.bfloat16, torch.float16):
        x = randn(6, 40, 64, dtype=dtype, seed=4)
        s = randn(64, dtype=dtype, seed=5)
        assert_bitexact(es.einshard("b n h, h -> b n h", x.to(gpu), s.to(gpu)), torch.einsum("bnh,h->bnh", x, s))


def test_unsupported_dtype_for_arithmetic(gpu):
    x = torch.ones(4, 4, dtype=torch.float64, device=gpu)
    with pytest.raises(NotImplementedError, match="not supported"):
        es.einshard("a b, b c -> a c", x, x)


def test_cpu_tensors_are_refused(gpu):
    with pytest.raises(RuntimeError, match="device tensors"):
        es.einshard("a b -> b a", torch.ones(2, 3))


# ---- prepared-launch replay -----------------------------------------------------------


def test_repeated_calls_replay_with_fresh_data_and_geometry(gpu):
    expr = "a b k c, b c l d -> k l d a"
    for seed in (40, 41):  # the second call replays the first call's prepared launch
        x, y = randn(4, 5, 8, 6, seed=seed), randn(5, 6, 8, 3, seed=seed + 100)
        assert_rel(es.einshard(expr, x.to(gpu), y.to(gpu)), einshard_cpu(expr, x, y), TOL[torch.float32])
        assert [step.name for step in last_plan()] == ["rank_local_einsum"]
    # same shapes, other strides: a new plan, not the cached one
    xt = randn(4, 5, 6, 8, seed=42).to(gpu).transpose(2, 3)
    y = randn(5, 6, 8, 3, seed=43)
    assert_rel(es.einshard(expr, xt, y.to(gpu)), einshard_cpu(expr, xt.cpu(), y), TOL[torch.float32])
    # same geometry on the host after a cached device call: still refused
    with pytest.raises(RuntimeError, match="device tensors"):
        es.einshard(expr, xt.cpu(), y)
    # a factored output packs on replay too
    x = randn(6, 4, seed=44)
    for _ in range(2):
        assert_bitexact(es.einshard("h p -> (p h)", x.to(gpu)), x.t().reshape(-1))


# ---- the 256 x 256 kernels (only chosen when they still give every CU a tile) -------


@pytest.mark.parametrize(
    "expr, shapes, kernel",
    [
        # K-contiguous operands: the software-pipelined kernels; ragged M and N,
        # an odd (3) and an even (4) number of 64-deep K tiles.  Both of these cut into
        # two rounds of one tile per CU with 256 x 224 tiles as with 256 x 256 ones,
        # so the narrower tiles are chosen.
        ("m k, n k -> m n", [(4136, 192), (4072, 192)], "contract_pipe_256x224"),
        ("m k, n k -> m n", [(4096, 256), (4200, 256)], "contract_pipe_256x224"),
        # 32 x 7 = 224 tiles of 256 x 256, fewer than the CUs: one round of 256 x 224
        # tiles beats four rounds of 128 x 128 ones (the host's cycle model)
        ("m k, n k -> m n", [(8192, 512), (1792, 512)], "contract_pipe_256x224"),
        # config 4's shape (N = 1792 = 8 x 224), and a ragged N edge inside a 224 tile
        ("b n c, h c -> b n h", [(8, 2048, 128), (1792, 128)], "contract_pipe_256x224"),
        ("m k, n k -> m n", [(16384, 192), (1700, 192)], "contract_pipe_256x224"),
        # two K sub-axes (the inner one exactly one K tile), batch offsets
        ("m a k, n a k -> m n", [(4096, 3, 64), (4096, 3, 64)], "contract_pipe_256x256"),
        ("b m k, b n k -> b m n", [(16, 1024, 128), (16, 1000, 128)], "contract_pipe_256x256"),
        # operands contiguous along M / N: read in place, fragments through transposing
        # LDS reads; ragged M and N edges
        ("k m, n k -> m n", [(128, 4096), (4096, 128)], "contract_pipe_256x256_mn_a"),
        ("m k, k n -> m n", [(4096, 128), (128, 4096)], "contract_pipe_256x256_mn_b"),
        ("k m, k n -> m n", [(192, 4096), (192, 4136)], "contract_pipe_256x256_mn_ab"),
        ("k m, n k -> m n", [(128, 4136), (4000, 128)], "contract_pipe_256x256_mn_a"),
        # more N rows than M rows: B takes the third LDS stage (K-contiguous operands, and
        # an N-contiguous B with a ragged N edge)
        ("m k, n k -> m n", [(2048, 192), (8192, 192)], "contract_pipe_256x256"),
        ("m k, k n -> m n", [(2048, 128), (128, 8104)], "contract_pipe_256x256_mn_b"),
    ],
)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_large_tiles(gpu, expr, shapes, kernel, dtype):
    x = randn(*shapes[0], seed=71, dtype=dtype)
    y = randn(*shapes[1], seed=72, dtype=dtype)
    got = es.einshard(expr, x.to(gpu), y.to(gpu))
    assert _native.last_kernel() == kernel
    assert_rel(got, einshard_cpu(expr, x, y), TOL[dtype])


# ---- several rounds of tiles per CU --------------------------------------------------
# Grids of two to three work-groups per CU on the 256-row kernels: ragged M and N edges
# in the last round, both tile widths, the three MN-contiguous layouts, two K levels and
# batch offsets.


def _sliced(full, index, seed, dtype):
    return randn(*full, seed=seed, dtype=dtype)[index]


@pytest.mark.parametrize(
    "expr, xs, ys, kernel",
    [
        # 96 x 8 = 768 tiles of 256 x 224, three rounds, ragged M and N
        ("m k, n k -> m n", ((24500, 512), ...), ((1704, 512), ...), "contract_pipe_256x224"),
        # 32 x 16 tiles of 256 x 256, two rounds
        ("m k, n k -> m n", ((8192, 256), ...), ((4096, 256), ...), "contract_pipe_256x256"),
        # batch offsets: 4 x 16 x 5 = 320 tiles, 10 K tiles
        ("b m k, b n k -> b m n", ((4, 4096, 640), ...), ((4, 1096, 640), ...), "contract_pipe_256x224"),
        # two K levels (a, then k sliced to 64 of 96): K tiles walk a
        ("m a k, n a k -> m n", ((4096, 4, 96), (slice(None), slice(None), slice(0, 64))),
         ((4200, 4, 96), (slice(None), slice(None), slice(0, 64))), "contract_pipe_256x224"),
        # operands contiguous along M / N (256 x 256 only)
        ("k m, n k -> m n", ((256, 8192), ...), ((4096, 256), ...), "contract_pipe_256x256_mn_a"),
        ("m k, k n -> m n", ((8192, 256), ...), ((256, 4096), ...), "contract_pipe_256x256_mn_b"),
        ("k m, k n -> m n", ((256, 8192), ...), ((256, 4136), ...), "contract_pipe_256x256_mn_ab"),
    ],
)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_multi_round_tiles(gpu, expr, xs, ys, kernel, dtype):
    x = _sliced(xs[0], xs[1], 171, dtype)
    y = _sliced(ys[0], ys[1], 172, dtype)
    got = es.einshard(expr, on_device(x, gpu), on_device(y, gpu))
    assert _native.last_kernel() == kernel
    assert_rel(got, einshard_cpu(expr, x, y), TOL[dtype])


def test_large_tiles_f32_m_contiguous(gpu):
    # fp32 keeps the 8-wave 256 x 256 kernel with its register-transposing loader
    x, y = randn(128, 4096, seed=73), randn(4096, 128, seed=74)
    got = es.einshard("k m, n k -> m n", x.to(gpu), y.to(gpu))
    assert _native.last_kernel() == "contract_256x256"
    assert_rel(got, einshard_cpu("k m, n k -> m n", x, y), TOL[torch.float32])


@pytest.mark.parametrize(
    "m, n, k, kernel",
    [
        (4096, 4096, 64, "contract_pipe_256x256"),
        (4096, 4096, 128, "contract_pipe_256x256"),
        (16384, 1792, 64, "contract_pipe_256x224"),
        (96, 80, 1, None),
    ],
)
def test_output_rounding_is_bitexact(gpu, m, n, k, kernel):
    # Only k = 0 carries values, so every output is one exact fp32 product x[m] * y[n]
    # (a bf16 x bf16 product has at most 16 significant bits) and the result is its one
    # rounding to bf16: nearest-even, overflow to inf, NaN stays NaN.
    g = gen(91)
    xv = torch.randn(m, generator=g) * 4
    yv = torch.randn(n, generator=g) * 4
    xv[3], xv[5], xv[11], yv[7] = float("inf"), float("nan"), 3e38, -float("inf")
    x = torch.zeros(m, k, dtype=torch.bfloat16)
    y = torch.zeros(n, k, dtype=torch.bfloat16)
    x[:, 0], y[:, 0] = xv.bfloat16(), yv.bfloat16()
    got = es.einshard("m k, n k -> m n", x.to(gpu), y.to(gpu))
    if kernel is not None:
        assert _native.last_kernel() == kernel
    want = (x[:, 0].float()[:, None] * y[:, 0].float()[None, :]).bfloat16()
    assert_bitexact_nan(got, want)


def test_c2_pattern_reads_the_n_contiguous_operand_in_place(gpu):
    # x is K-contiguous, y contiguous along its free axes; the planner makes y the
    # first operand (so the output's contiguous axis a is along N), read M-contiguous
    x = randn(64, 32, 128, 64, seed=75, dtype=torch.bfloat16)
    y = randn(32, 64, 128, 16, seed=76, dtype=torch.bfloat16)
    expr = "a b k c, b c l d -> k l d a"
    got = es.einshard(expr, x.to(gpu), y.to(gpu))
    assert _native.last_kernel() == "contract_pipe_256x256_mn_a"
    assert_rel(got, einshard_cpu(expr, x, y), TOL[torch.bfloat16])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mn_contiguous_operand_with_two_k_levels(gpu, dtype):
    # x sliced along its inner K axis: K stays two sub-axes (3 x 64), each K tile's 64
    # k-rows one stride apart, the outer level a jump
    big = randn(3, 80, 4096, seed=77, dtype=dtype)
    x = big[:, :64, :]
    y = randn(4096, 3, 64, seed=78, dtype=dtype)
    expr = "k j m, n k j -> m n"
    got = es.einshard(expr, on_device(x, gpu), y.to(gpu))
    assert _native.last_kernel() == "contract_pipe_256x256_mn_a"
    assert_rel(got, einshard_cpu(expr, x, y), TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_mn_contiguous_rows_in_groups(gpu, dtype):
    # x sliced along its unit-stride axis: M stays two sub-axes (200 x 24), so the
    # 8-row runs of a 32-row block cross from one group of 24 rows to the next
    x = randn(64, 200, 32, seed=79, dtype=dtype)[:, :, :24]
    y = randn(64, 4104, seed=80, dtype=dtype)
    expr = "k m a, k n -> m a n"
    got = es.einshard(expr, on_device(x, gpu), y.to(gpu))
    assert _native.last_kernel() == "contract_pipe_256x256_mn_ab"
    assert_rel(got, einshard_cpu(expr, x, y), TOL[dtype])


def test_mn_contiguous_output_rounding_is_bitexact(gpu):
    # as test_output_rounding_is_bitexact, with both operands read along M / N
    g = gen(92)
    m, n, k = 4096, 4096, 64
    xv, yv = torch.randn(m, generator=g) * 4, torch.randn(n, generator=g) * 4
    xv[3], xv[5], yv[7] = float("inf"), float("nan"), -float("inf")
    x = torch.zeros(k, m, dtype=torch.bfloat16)
    y = torch.zeros(k, n, dtype=torch.bfloat16)
    x[0], y[0] = xv.bfloat16(), yv.bfloat16()
    got = es.einshard("k m, k n -> m n", x.to(gpu), y.to(gpu))
    assert _native.last_kernel() == "contract_pipe_256x256_mn_ab"
    want = (x[0].float()[:, None] * y[0].float()[None, :]).bfloat16()
    assert_bitexact_nan(got, want)


# ---- transposes (pure permutations whose input unit-stride dim is not innermost) ----


@pytest.mark.parametrize(
    "expr, shape",
    [
        ("a b -> b a", (300, 200)),
        ("b t c h w -> b t h w c", (2, 3, 40, 5, 70)),
        ("a b c -> c a b", (33, 7, 129)),
        ("a b c d -> b d c a", (65, 3, 4, 70)),
    ],
)
@pytest.mark.parametrize("dtype", [torch.uint8, torch.bfloat16, torch.float32, torch.int64])
def test_transposes_are_bitexact(gpu, expr, shape, dtype):
    x = (randn(*shape, seed=81) * 50).to(dtype)
    got = es.einshard(expr, x.to(gpu))
    assert _native.last_kernel() == "gather_transpose"
    assert_bitexact(got, einshard_cpu(expr, x))


@pytest.mark.parametrize(
    "expr, shape, dtype",
    [
        ("o c kh kw -> o kh kw c", (256, 256, 3, 3), torch.bfloat16),  # a conv weight's taps behind its channels
        ("o c kh kw -> o kh kw c", (64, 48, 3, 3), torch.float32),
        ("o c k -> o k c", (128, 96, 7), torch.float16),
        ("a q p -> a p q", (32, 64, 5), torch.uint8),
        ("a q p -> a p q", (16, 30, 3), torch.int64),
        ("a b q p -> b a p q", (4, 8, 64, 9), torch.bfloat16),  # two outer dims, permuted
    ],
)
def test_short_transposes_move_whole_slabs(gpu, expr, shape, dtype):
    # P (the input's unit-stride dim) short and the (P, Q) slab dense and small in both
    # tensors: whole slabs through LDS with 16-byte accesses
    x = (randn(*shape, seed=83) * 50).to(dtype)
    got = es.einshard(expr, x.to(gpu))
    assert _native.last_kernel() == "gather_transpose_slab", _native.last_kernel()
    assert_bitexact(got, einshard_cpu(expr, x))
    # the same permutation of a misaligned view takes the tile kernel, with the same result
    flat = torch.zeros(x.numel() + 1, dtype=dtype, device=gpu)
    moved = flat[1:].view(shape)
    moved.copy_(x.to(gpu))
    again = es.einshard(expr, moved)
    assert _native.last_kernel() == "gather_transpose", _native.last_kernel()
    assert_bitexact(again, got)


@pytest.mark.parametrize(
    "expr, shape",
    [
        ("a b c d e -> a d c b e", (4, 1, 8, 1, 16)),  # unit dims swapped: a plain copy
        ("a b c d -> a c d b", (3, 5, 7, 64)),  # (c, d) move together behind a
        ("a b c d -> c d a b", (6, 10, 12, 9)),  # two merged pairs exchanged
        ("a b c -> b a c", (1, 40, 24)),  # a unit dim in front
        ("a b c d -> d a b c", (2, 3, 4, 70)),  # (a, b, c) merge: one 2-D transpose
    ],
)
@pytest.mark.parametrize("dtype", [torch.uint8, torch.bfloat16, torch.float32, torch.int64])
def test_permutations_with_mergeable_or_unit_dims(gpu, expr, shape, dtype):
    # es_gather merges output neighbours that are input neighbours and drops unit dims
    # before choosing its transpose; every permutation stays bit-exact
    x = (randn(*shape, seed=84) * 50).to(dtype)
    assert_bitexact(es.einshard(expr, x.to(gpu)), einshard_cpu(expr, x))
    # the same through a strided view: every other element along the last input dim
    wide = (randn(*shape[:-1], 2 * shape[-1], seed=85) * 50).to(dtype)
    view = wide.to(gpu)[..., ::2]
    assert_bitexact(es.einshard(expr, view), einshard_cpu(expr, wide[..., ::2].contiguous()))


@pytest.mark.parametrize("shape", [(16, 24, 40), (8, 33, 64), (3, 5, 7)])
def test_transposes_with_short_or_odd_dims(gpu, shape):
    # short P (tile depth below 64) and sizes that are not whole vectors
    for dtype in (torch.uint8, torch.bfloat16, torch.float32):
        x = (randn(*shape, seed=82) * 50).to(dtype)
        assert_bitexact(es.einshard("a p q -> a q p", x.to(gpu)), einshard_cpu("a p q -> a q p", x))


@pytest.mark.parametrize(
    "batch, m, n, k",
    [
        (1, 4096, 4136, 128),  # ragged N
        (4, 2048, 2000, 192),  # batched, ragged N, three 64-deep K tiles
        (1, 4104, 4096, 256),  # ragged M (a multiple of 8)
        (1, 4100, 4096, 128),  # M not a multiple of 8: element stores
    ],
)
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("bias", [False, True])
def test_output_contiguous_along_m(gpu, batch, m, n, k, dtype, bias):
    # out[b, n, m] = sum_k x[b, m, k] y[b, n, k] with M the A operand: the output is
    # contiguous along the tile's rows, so contract_pipe stages the tile transposed
    from torch_einshard._exec import launch, prepare_op
    from torch_einshard.planner import ContractOp, SubAxis

    x = randn(batch, m, k, seed=91, dtype=dtype)
    y = randn(batch, n, k, seed=92, dtype=dtype)
    b = randn(n, seed=93, dtype=dtype) if bias else None
    op = ContractOp(
        (batch, n, m),
        swapped=False,
        batch=[SubAxis(batch, a=m * k, b=n * k, c=n * m)],
        m=[SubAxis(m, a=k, c=1)],
        n=[SubAxis(n, b=k, c=m)],
        k=[SubAxis(k, a=1, b=1)],
    )
    prep = prepare_op(op, dtype, 2)
    got = launch(prep, (x.to(gpu), y.to(gpu)), gpu, dtype, bias=None if b is None else b.to(gpu))
    assert _native.last_kernel().startswith("contract_pipe"), _native.last_kernel()
    want = torch.matmul(y.float(), x.float().transpose(1, 2))  # [b, n, m]
    if b is not None:
        want = want + b.float()[None, :, None]
    assert_rel(got, want.to(dtype), TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("m, n, k", [(256, 512, 16384), (100, 300, 9000), (64, 64, 65536)])
def test_split_k(gpu, m, n, k, dtype):
    # few output tiles and a long K: partial contractions over parts of K, then their sum
    from torch_einshard._exec import _split_k
    from torch_einshard.planner import ContractOp, SubAxis

    _, parts = _split_k(ContractOp((m, n), swapped=False, m=[SubAxis(m, a=1, c=n)], n=[SubAxis(n, b=1, c=1)],
                                   k=[SubAxis(k, a=m, b=n)]))
    assert parts > 1
    x = randn(k, m, seed=95, dtype=dtype)
    y = randn(k, n, seed=96, dtype=dtype)
    got = es.einshard("k m, k n -> m n", x.to(gpu), y.to(gpu))
    assert _native.last_kernel().startswith("reduce"), _native.last_kernel()
    want = einshard_cpu("k m, k n -> m n", x.float(), y.float())
    assert_rel(got, want.to(dtype), TOL[dtype])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_split_k_on_the_pipelined_kernel(gpu, dtype):
    # a weight gradient with 4 x 8 tiles of 256 x 256 and K = 8192: eight parts of 1024
    # make 256 tiles for the pipelined kernel, both operands read along their rows
    from torch_einshard import _cache

    x = randn(8, 1024, 1024, seed=97, dtype=dtype)
    y = randn(8, 1024, 2048, seed=98, dtype=dtype)
    expr = "b n h, b n c -> h c"
    xs = [x.to(gpu), y.to(gpu)]
    got = es.einshard(expr, *xs)
    assert_rel(got, einshard_cpu(expr, x.float(), y.float()).to(dtype), TOL[dtype])
    prep, _ = _cache.lookup(_cache.call_key("einshard", xs, None, None, expr, None, None))
    parts = prep.split[0]
    assert parts == 8
    # the partial contractions alone: their kernel, and each part's fp32 sum (unrounded)
    assert prep.desc.out_f32 == 1 and prep.split[1].in_f32 == 1
    tmp = torch.empty((parts, 1024 * 2048), dtype=torch.float32, device=gpu)
    ptrs = [xs[i].data_ptr() for i in prep.order]
    assert _native.lib().es_contract(prep.ref, *ptrs, tmp.data_ptr(), _native.stream_of(tmp)) == 0
    assert _native.last_kernel() == "contract_pipe_256x256_mn_ab"
    for s in (0, parts - 1):
        want = einshard_cpu(expr, x[s:s + 1].float(), y[s:s + 1].float())
        assert_rel(tmp[s].view(1024, 2048), want, 1e-5)


@pytest.mark.parametrize("m, n", [(256, 512), (4096, 4096)])
def test_split_k_partials_do_not_overflow_f16(gpu, m, n):
    # The two halves of K cancel: each part's sum (512 or 1024 terms of +-256) is beyond
    # f16's range (65504) while the whole sum is small.  The partials are kept in fp32,
    # so the result is the single-pass one (a reference torch.einsum would accumulate
    # the whole sum before one rounding, too).  (256, 512): split for the 128 x 128
    # kernel; (4096, 4096) at K = 16384: no split, the plain pipelined kernel.
    k = 16384
    g = gen(99)
    x = torch.ones(k, m)
    y = torch.full((k, n), 256.0)
    y[k // 2:] = -256.0
    # the last 32 rows of each half carry random terms instead: the +-256 terms cancel
    # exactly and the result is the sum of those 64 products (~N(0, 1024^2) each, so the
    # fp32 ulp of a running sum near 2^21, 0.25, stays small against the result)
    for end in (k // 2, k):
        x[end - 32:end] = torch.randn(32, m, generator=g) * 32
        y[end - 32:end] = torch.randn(32, n, generator=g) * 32
    x16, y16 = x.half(), y.half()
    got = es.einshard("k m, k n -> m n", x16.to(gpu), y16.to(gpu))
    assert torch.isfinite(got).all().item()
    want = einshard_cpu("k m, k n -> m n", x16.float(), y16.float())
    assert_rel(got, want.half(), TOL[torch.float16])


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_split_k_through_two_k_axes_on_the_pipelined_kernel(gpu, dtype):
    # An einconv-weight-gradient geometry at the production thresholds: K = (16, 32, 64)
    # sub-axes that do not merge (both operands sliced), M x N = 256 x 2048 (8 tiles of
    # 256 x 256).  The outer sub-axis alone gives 16 parts (128 tiles), so the cut takes
    # it whole and halves the next one: 32 parts of K = 1024, 256 tiles on
    # contract_pipe_256x256_mn_ab, then one es_reduce over the fp32 partials.
    from torch_einshard import _cache

    gz = randn(16, 34, 72, 256, seed=101, dtype=dtype)[:, :32, :64]
    xp = randn(16, 34, 72, 2048, seed=102, dtype=dtype)[:, 1:33, 4:68]
    expr = "b h w o, b h w t -> o t"
    xs = [on_device(gz, gpu), on_device(xp, gpu)]
    got = es.einshard(expr, *xs)
    prep, _ = _cache.lookup(_cache.call_key("einshard", xs, None, None, expr, None, None))
    assert prep.split is not None and prep.split[0] == 32
    assert [prep.desc.batch[i].size for i in range(prep.desc.n_batch)] == [16, 2]
    assert _native.last_kernel().startswith("reduce"), _native.last_kernel()
    want = einshard_cpu(expr, gz.float(), xp.float())
    assert_rel(got, want.to(dtype), TOL[dtype])
    # the partial contractions alone run on the pipelined kernel
    tmp = torch.empty((32, 256 * 2048), dtype=torch.float32, device=gpu)
    ptrs = [xs[i].data_ptr() for i in prep.order]
    assert _native.lib().es_contract(prep.ref, *ptrs, tmp.data_ptr(), _native.stream_of(tmp)) == 0
    assert _native.last_kernel() == "contract_pipe_256x256_mn_ab"
    assert_rel(tmp.sum(0).view(256, 2048), want, 1e-5)
