"""es_reduce_noalloc: es_reduce with its split partials in library-owned scratch.

Called through the C ABI and compared bit for bit with es_reduce on the same
descriptor (the same kernels and the same summation order), on two calls in a
row, the second on a smaller input, so the second call also runs over scratch
that still holds the first call's partials.  A descriptor needing more scratch
than ES_NOALLOC_SCRATCH_BYTES would be refused with ES_ERR_WORKSPACE before any
launch; no descriptor does (tests/test_abi.py checks the bound over a sweep).
A call captured into a HIP graph (after an eager first call on the device) is
replayed over new inputs and compared with es_reduce after every replay.
"""

import ctypes

import pytest
import torch

from torch_einshard import _native
from torch_einshard._exec import _set_axes
from torch_einshard.planner import SubAxis

from conftest import assert_bitexact

pytestmark = pytest.mark.gpu


def _middle_sum_desc(b, n, h, dtype, in_f32=False):
    """``b n h -> b h`` over a dense [b, n, h] input: a sum over the middle axis."""
    desc = _native.ReduceDesc()
    desc.dtype = _native.DTYPE_CODES[dtype]
    desc.in_f32 = 1 if in_f32 else 0
    desc.has_y = 0
    desc.n_keep = _set_axes(desc.keep, [SubAxis(b, a=n * h), SubAxis(h, a=1)], "test")
    desc.n_red = _set_axes(desc.red, [SubAxis(n, a=h)], "test")
    return desc


def _both(desc, x, out_shape, out_dtype):
    lib = _native.lib()
    stream = _native.stream_of(x)
    need = lib.es_reduce_workspace_bytes(ctypes.byref(desc))
    assert 0 < need <= _native.NOALLOC_SCRATCH_BYTES, need  # a split reduction that fits
    want = torch.empty(out_shape, dtype=out_dtype, device=x.device)
    ws = torch.empty(need, dtype=torch.uint8, device=x.device)
    assert lib.es_reduce(ctypes.byref(desc), x.data_ptr(), None, want.data_ptr(), ws.data_ptr(), need, stream) == 0
    got = torch.empty(out_shape, dtype=out_dtype, device=x.device)
    status = lib.es_reduce_noalloc(ctypes.byref(desc), x.data_ptr(), None, got.data_ptr(), stream)
    assert status == 0, lib.es_last_error().decode()
    assert _native.last_kernel() == "reduce_cols"
    return got, want


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_noalloc_reduce_matches_es_reduce_on_two_calls(gpu, dtype):
    g = torch.Generator(device=gpu).manual_seed(7)
    # first call: 16 x 1024 outputs, each a sum of 4096 terms, split 32 ways (2 MiB of
    # partials); second call: a smaller reduction over the same scratch
    for b, n, h in ((16, 4096, 1024), (3, 1000, 200)):
        x = (torch.rand(b, n, h, generator=g, device=gpu) * 2 - 1).to(dtype)
        got, want = _both(_middle_sum_desc(b, n, h, dtype), x, (b, h), dtype)
        torch.cuda.synchronize()
        assert_bitexact(got, want)
        ref = x.double().sum(1)
        assert (got.double() - ref).abs().max().item() <= 1e-5 * max(ref.abs().max().item(), 1.0) + (
            0 if dtype == torch.float32 else 1e-2 * ref.abs().max().item())


def test_noalloc_reduce_of_fp32_partials_to_bf16(gpu):
    # the split-K finish: fp32 partial results summed and rounded once to bf16
    g = torch.Generator(device=gpu).manual_seed(8)
    for b, n, h in ((8, 2048, 2048), (2, 1024, 512)):
        x = torch.randn(b, n, h, generator=g, device=gpu)
        got, want = _both(_middle_sum_desc(b, n, h, torch.bfloat16, in_f32=True), x, (b, h), torch.bfloat16)
        torch.cuda.synchronize()
        assert_bitexact(got, want)
        ref = x.double().sum(1)
        assert (got.double() - ref).abs().max().item() <= 2e-2 * ref.abs().max().item()


def test_noalloc_reduce_rejects_bad_descriptors_before_any_launch(gpu):
    lib = _native.lib()
    out = torch.empty(4, device=gpu)
    assert lib.es_reduce_noalloc(None, None, None, out.data_ptr(), None) == _native.ES_ERR_INVALID
    desc = _middle_sum_desc(1, 8, 4, torch.float32)
    desc.n_red = 9
    assert lib.es_reduce_noalloc(ctypes.byref(desc), None, None, out.data_ptr(), None) == _native.ES_ERR_INVALID


def test_noalloc_reduce_replays_from_a_captured_graph(gpu):
    # the entry point's intended caller: a HIP graph.  The first call on the device
    # (which looks up the scratch address) runs eagerly; the captured call is then
    # replayed five times over new inputs written between the replays, each replay
    # compared bit for bit with es_reduce on the same input.
    lib = _native.lib()
    b, n, h = 8, 2048, 1024
    desc = _middle_sum_desc(b, n, h, torch.float32)
    need = lib.es_reduce_workspace_bytes(ctypes.byref(desc))
    assert 0 < need <= _native.NOALLOC_SCRATCH_BYTES
    g = torch.Generator(device=gpu).manual_seed(9)
    x = torch.rand(b, n, h, generator=g, device=gpu) * 2 - 1
    out = torch.empty(b, h, device=gpu)
    assert lib.es_reduce_noalloc(ctypes.byref(desc), x.data_ptr(), None, out.data_ptr(), _native.stream_of(x)) == 0
    torch.cuda.synchronize()

    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        stream = ctypes.c_void_p(torch.cuda.current_stream(gpu).cuda_stream)
        status = lib.es_reduce_noalloc(ctypes.byref(desc), x.data_ptr(), None, out.data_ptr(), stream)
    assert status == 0, lib.es_last_error().decode()

    want = torch.empty(b, h, device=gpu)
    ws = torch.empty(need, dtype=torch.uint8, device=gpu)
    for replay in range(5):
        x.copy_(torch.rand(b, n, h, generator=g, device=gpu) * 2 - 1)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        stream = _native.stream_of(x)
        assert lib.es_reduce(ctypes.byref(desc), x.data_ptr(), None, want.data_ptr(), ws.data_ptr(), need, stream) == 0
        torch.cuda.synchronize()
        assert_bitexact(out, want)
