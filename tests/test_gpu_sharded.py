"""The reference's sharded halo, window, convolution and tensor-parallel expectations at
world size 1, on the device, through a one-rank gloo mesh (the reference runs the same
tests at world size 1 under plain pytest, reference tests/conftest.py:16-41).

Ported: reference tests/test_halo.py:139-245 (a sharded halo with split shapes and its
gradient, a halo wider than the local shard, periodic wrap-and-accumulate, the empty
periodic axis, a sharded einwindow), tests/test_conv.py:105-137 (a sharded einconv with
bias and gradients) and tests/test_scigpt_patterns.py:11-99 (the tensor-parallel MLP
with and without an ellipsis, and the attention projection).  The expected values are
the reference tests' own: its split helpers (restated below), ``F.conv2d`` and
``torch.einsum`` on CPU tensors.  Copies are compared bit for bit, arithmetic within
the tolerances stated in each test.
"""

import pytest
import torch
import torch.nn.functional as F

import torch_einshard as es

from conftest import TOL, assert_rel

pytestmark = pytest.mark.gpu


def _extended_split(full, shapes, rank, left, right, *, fill=0):
    """Rows [start - left, end + right) of the full tensor, padded with fill past its
    ends (reference tests/test_halo.py:11-19)."""
    start = sum(shapes[:rank])
    end = start + shapes[rank]
    take_start = max(0, start - left)
    take_end = min(full.shape[0], end + right)
    result = full[take_start:take_end]
    if take_start > start - left or take_end < end + right:
        result = F.pad(result, (0, 0, take_start - (start - left), (end + right) - take_end), value=fill)
    return result


def _periodic_split(full, shapes, rank, left, right):
    """The same rows taken cyclically (reference tests/test_halo.py:22-26)."""
    start = sum(shapes[:rank])
    index = torch.arange(start - left, start + shapes[rank] + right).remainder(full.shape[0])
    return full.index_select(0, index)


def _split(full, shapes, rank, dim=0):
    return torch.split(full, shapes, dim=dim)[rank]


def _rank(mesh, name):
    import torch.distributed as dist

    group = mesh[name].get_group()
    return dist.get_rank(group), dist.get_world_size(group)


def test_sharded_einhalo_with_split_shapes(gpu, mesh_1d):
    # reference tests/test_halo.py:139-158
    rank, world = _rank(mesh_1d, "dp")
    shapes = es.helpers.compute_split_shapes(world * 3 + 1, world)
    full = torch.arange(sum(shapes) * 2, dtype=torch.float32).reshape(sum(shapes), 2)
    x = _split(full, shapes, rank).clone().to(gpu).requires_grad_(True)
    z = es.einhalo("a/dp b", x, {"a": 1}, mesh=mesh_1d, shapes=shapes, fill=-1)
    assert torch.equal(z.detach().cpu(), _extended_split(full, shapes, rank, 1, 1, fill=-1))
    z.sum().backward()
    full_grad = torch.zeros_like(full)
    for peer in range(world):
        start = sum(shapes[:peer])
        full_grad[max(0, start - 1):min(full.shape[0], start + shapes[peer] + 1)] += 1
    assert torch.equal(x.grad.cpu(), _split(full_grad, shapes, rank))


def test_sharded_einhalo_wider_than_the_local_shard(gpu, mesh_1d):
    # reference tests/test_halo.py:161-180
    rank, world = _rank(mesh_1d, "dp")
    shapes = [2] + [1] * (world - 1)
    full = torch.arange(sum(shapes) * 2, dtype=torch.float32).reshape(sum(shapes), 2)
    x = _split(full, shapes, rank).clone().to(gpu).requires_grad_(True)
    left, right = world + 1, world
    z = es.einhalo("a/dp b", x, {"a": (left, right)}, mesh=mesh_1d, shapes=shapes, fill=-3)
    assert torch.equal(z.detach().cpu(), _extended_split(full, shapes, rank, left, right, fill=-3))
    z.sum().backward()
    full_grad = torch.zeros_like(full)
    for peer in range(world):
        start = sum(shapes[:peer])
        full_grad[max(0, start - left):min(full.shape[0], start + shapes[peer] + right)] += 1
    assert torch.equal(x.grad.cpu(), _split(full_grad, shapes, rank))


def test_sharded_periodic_einhalo_wraps_and_accumulates(gpu, mesh_1d):
    # reference tests/test_halo.py:183-210: the left halo is wider than the whole axis,
    # so rows wrap more than once and their gradients add up
    rank, world = _rank(mesh_1d, "dp")
    shapes = [2] + [1] * (world - 1)
    full = torch.arange(sum(shapes) * 2, dtype=torch.float32).reshape(sum(shapes), 2)
    x = _split(full, shapes, rank).clone().to(gpu).requires_grad_(True)
    left, right = sum(shapes) + 1, world
    z = es.einhalo("a/dp b", x, {"a": (left, right)}, boundary="periodic", mesh=mesh_1d, shapes=shapes)
    assert torch.equal(z.detach().cpu(), _periodic_split(full, shapes, rank, left, right))
    z.sum().backward()
    full_grad = torch.zeros_like(full)
    for peer in range(world):
        index = torch.arange(sum(shapes[:peer]) - left, sum(shapes[:peer + 1]) + right).remainder(full.shape[0])
        full_grad.index_add_(0, index, torch.ones(index.shape[0], full.shape[1]))
    assert torch.equal(x.grad.cpu(), _split(full_grad, shapes, rank))


def test_sharded_periodic_einhalo_rejects_an_empty_axis(gpu, mesh_1d):
    # reference tests/test_halo.py:213-219
    _, world = _rank(mesh_1d, "dp")
    x = torch.empty(0, 2, device=gpu)
    with pytest.raises(ValueError, match="periodic-pad an empty axis"):
        es.einhalo("a/dp b", x, {"a": 1}, boundary="periodic", mesh=mesh_1d, shapes=[0] * world)


def test_sharded_einwindow_matches_full_tensor_windows(gpu, mesh_1d):
    # reference tests/test_halo.py:222-243
    rank, world = _rank(mesh_1d, "dp")
    shapes = es.helpers.compute_split_shapes(world * 3 + 1, world)
    full = torch.arange(sum(shapes), dtype=torch.float32).reshape(sum(shapes), 1)
    x = _split(full, shapes, rank).clone().to(gpu).requires_grad_(True)
    z = es.einwindow("a/dp b -> a/dp k b", x, {"a": "k"}, {"a": 1}, mesh=mesh_1d, shapes=shapes, fill=-1)
    expected = _extended_split(full, shapes, rank, 1, 1, fill=-1).unfold(0, 3, 1).permute(0, 2, 1)
    assert torch.equal(z.detach().cpu(), expected)
    # every row is read by its own window and its neighbours' (three times inside,
    # twice at the ends of the axis)
    z.sum().backward()
    want = torch.full((sum(shapes), 1), 3.0)
    want[0] = want[-1] = 2.0
    assert torch.equal(x.grad.cpu(), _split(want, shapes, rank))


def test_sharded_einwindow_checks_the_split_shapes(gpu, mesh_1d):
    x = torch.zeros(4, 1, device=gpu)
    with pytest.raises(ValueError, match="Local tensor size 4 does not match split shape 5 for axis 'a'"):
        es.einwindow("a/dp b -> a/dp k b", x, {"a": "k"}, {"a": 1}, mesh=mesh_1d, shapes=[5])


def test_sharded_einconv_matches_full_conv2d(gpu, mesh_1d):
    # reference tests/test_conv.py:105-137, with its tolerances for the gradient
    rank, world = _rank(mesh_1d, "dp")
    shapes = es.helpers.compute_split_shapes(world * 3 + 1, world)
    g = torch.Generator().manual_seed(105)
    full = torch.randn(2, sum(shapes), 5, 3, generator=g)
    weight = torch.randn(4, 3, 3, 3, generator=g)
    bias = torch.randn(4, generator=g)
    x = _split(full, shapes, rank, dim=1).contiguous().to(gpu).requires_grad_(True)
    z = es.einconv(
        "b h/dp w c, o c kh kw -> b h/dp w o",
        x,
        weight.to(gpu),
        {"h": "kh", "w": "kw"},
        bias=bias.to(gpu),
        mesh=mesh_1d,
        shapes=shapes,
    )
    expected = F.conv2d(full.permute(0, 3, 1, 2), weight, bias, padding=1).permute(0, 2, 3, 1)
    assert_rel(z, _split(expected, shapes, rank, dim=1), TOL[torch.float32])

    z.square().sum().backward()
    full_ref = full.clone().requires_grad_(True)
    F.conv2d(full_ref.permute(0, 3, 1, 2), weight, bias, padding=1).permute(0, 2, 3, 1).square().sum().backward()
    torch.testing.assert_close(x.grad.cpu(), _split(full_ref.grad, shapes, rank, dim=1), rtol=1e-4, atol=1e-5)


def test_sharded_einconv_checks_the_split_shapes(gpu, mesh_1d):
    x = torch.zeros(2, 4, 5, 3, device=gpu)
    w = torch.zeros(4, 3, 3, 3, device=gpu)
    with pytest.raises(ValueError, match="Local tensor size 4 does not match split shape 3 for axis 'h'"):
        es.einconv("b h/dp w c, o c kh kw -> b h/dp w o", x, w, {"h": "kh", "w": "kw"}, mesh=mesh_1d, shapes=[3])


def _tp_shards(mesh_tp):
    rank, size = _rank(mesh_tp, "tp")
    return rank, size


def test_tensor_parallel_mlp_pattern(gpu, mesh_tp):
    # reference tests/test_scigpt_patterns.py:11-38
    rank, size = _tp_shards(mesh_tp)
    batch, seq, channels, out_channels = 2, 3, 4, 5
    hidden = size * 3
    hidden_shapes = es.helpers.compute_split_shapes(hidden, size)
    g = torch.Generator().manual_seed(11)
    x = torch.randn(batch, seq, channels, generator=g)
    w1 = torch.randn(hidden, channels, generator=g)
    b1 = torch.randn(hidden, generator=g)
    w2 = torch.randn(out_channels, hidden, generator=g)
    b2 = torch.randn(out_channels, generator=g)
    w1_shard = torch.split(w1, hidden_shapes, dim=0)[rank].contiguous().to(gpu)
    b1_shard = torch.split(b1, hidden_shapes, dim=0)[rank].contiguous().to(gpu)
    w2_shard = torch.split(w2, hidden_shapes, dim=1)[rank].contiguous().to(gpu)

    h = es.einshard("b n c, h/tp c -> b n h/tp", x.to(gpu), w1_shard, mesh=mesh_tp)
    h = F.gelu(h + b1_shard)
    y_partial = es.einshard("b n h/tp, o h/tp -> b n o // tp", h, w2_shard, mesh=mesh_tp)
    y = es.einshard("b n o // tp -> b n o", y_partial, mesh=mesh_tp) + b2.to(gpu)

    expected = F.gelu(torch.einsum("bnc,hc->bnh", x, w1) + b1)
    expected = torch.einsum("bnh,oh->bno", expected, w2) + b2
    torch.testing.assert_close(y.cpu(), expected, rtol=1e-5, atol=1e-5)


def test_tensor_parallel_mlp_pattern_with_ellipsis(gpu, mesh_tp):
    # reference tests/test_scigpt_patterns.py:41-61
    rank, size = _tp_shards(mesh_tp)
    batch, seq, channels, out_channels = 2, 3, 4, 5
    hidden = size * 3
    hidden_shapes = es.helpers.compute_split_shapes(hidden, size)
    g = torch.Generator().manual_seed(41)
    x = torch.randn(batch, seq, channels, generator=g)
    w1 = torch.randn(hidden, channels, generator=g)
    w2 = torch.randn(out_channels, hidden, generator=g)
    w1_shard = torch.split(w1, hidden_shapes, dim=0)[rank].contiguous().to(gpu)
    w2_shard = torch.split(w2, hidden_shapes, dim=1)[rank].contiguous().to(gpu)

    h = es.einshard("... c, h/tp c -> ... h/tp", x.to(gpu), w1_shard, mesh=mesh_tp)
    y_partial = es.einshard("... h/tp, o h/tp -> ... o // tp", h, w2_shard, mesh=mesh_tp)
    y = es.einshard("... o // tp -> ... o", y_partial, mesh=mesh_tp)

    expected = torch.einsum("...c,hc->...h", x, w1)
    expected = torch.einsum("...h,oh->...o", expected, w2)
    torch.testing.assert_close(y.cpu(), expected, rtol=1e-5, atol=1e-5)


def test_tensor_parallel_attention_projection_pattern(gpu, mesh_tp):
    # reference tests/test_scigpt_patterns.py:64-99.  The attention between the
    # projections is the caller's own code; it runs on the CPU in fp32 here (torch's
    # device attention path is not part of this library).
    rank, size = _tp_shards(mesh_tp)
    batch, seq, channels, heads_per_rank, head_dim = 2, 5, 4, 2, 3
    heads = heads_per_rank * size
    embed = heads * head_dim
    embed_shapes = [heads_per_rank * head_dim for _ in range(size)]
    g = torch.Generator().manual_seed(64)
    x = torch.randn(batch, seq, channels, generator=g)
    wq = torch.randn(embed, channels, generator=g)
    wk = torch.randn(embed, channels, generator=g)
    wv = torch.randn(embed, channels, generator=g)
    wo = torch.randn(channels, embed, generator=g)
    shard = lambda w, dim: torch.split(w, embed_shapes, dim=dim)[rank].contiguous().to(gpu)
    xd = x.to(gpu)

    q = es.einshard("b l c, e/tp c -> b l e/tp", xd, shard(wq, 0), mesh=mesh_tp)
    k = es.einshard("b l c, e/tp c -> b l e/tp", xd, shard(wk, 0), mesh=mesh_tp)
    v = es.einshard("b l c, e/tp c -> b l e/tp", xd, shard(wv, 0), mesh=mesh_tp)
    heads_of = lambda t: t.cpu().reshape(batch, seq, heads_per_rank, head_dim).transpose(1, 2)
    attn = F.scaled_dot_product_attention(heads_of(q), heads_of(k), heads_of(v))
    attn = attn.transpose(1, 2).reshape(batch, seq, embed_shapes[rank]).contiguous().to(gpu)
    y_partial = es.einshard("b l e/tp, c e/tp -> b l c // tp", attn, shard(wo, 1), mesh=mesh_tp)
    y = es.einshard("b l c // tp -> b l c", y_partial, mesh=mesh_tp)

    full_heads = lambda w: torch.einsum("blc,ec->ble", x, w).reshape(batch, seq, heads, head_dim).transpose(1, 2)
    expected = F.scaled_dot_product_attention(full_heads(wq), full_heads(wk), full_heads(wv))
    expected = torch.einsum("ble,ce->blc", expected.transpose(1, 2).reshape(batch, seq, embed), wo)
    torch.testing.assert_close(y.cpu(), expected, rtol=1e-4, atol=1e-5)
