"""The C ABI boundary, checked without a GPU: the library loads, exports every
entry point include/einshard_hip.h declares, and rejects malformed
descriptors with a status code and message (no kernel is launched)."""

import ctypes
import os
import re
import subprocess

import pytest
import torch

from torch_einshard import _native

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "einshard_hip.h")


def declared_entry_points():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(es_[a-z0-9_]+)\s*\(", text)))


def test_header_declares_the_entry_points():
    names = declared_entry_points()
    for required in (
        "es_gather",
        "es_bcast",
        "es_reduce",
        "es_reduce_workspace_bytes",
        "es_contract",
        "es_contract_bias",
        "es_last_error",
    ):
        assert required in names


def test_library_exports_every_declared_symbol():
    path = _native.library_path()
    assert os.path.exists(path), "build libeinshard_hip.so first"
    out = subprocess.run(["nm", "-D", "--defined-only", path], capture_output=True, text=True, check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = [name for name in declared_entry_points() if name not in exported]
    assert not missing, missing


def test_library_loads_and_reports_version():
    lib = _native.lib()
    assert lib.es_abi_version() == _native.ABI_VERSION
    assert b"gfx950" in lib.es_version()
    for name in declared_entry_points():
        assert hasattr(lib, name)


def _integration_stub_classes():
    """The ctypes classes of the binding example in the repository's integration guide
    (the file read below), executed without the library (the CDLL line and everything
    after the classes are left out)."""
    doc = os.path.join(os.path.dirname(HEADER), os.pardir, "INTEGRATION.md")
    text = open(doc).read()
    block = next(b for b in re.findall(r"```python\n(.*?)```", text, flags=re.S) if "class es_axis" in b)
    start = block.index("class es_axis")
    end = block.index("_lib.es_contract.argtypes")
    scope = {"ctypes": ctypes}
    exec(block[start:end], scope)
    return scope["es_axis"], scope["es_contract_desc"]


def test_integration_stub_matches_the_abi_field_for_field():
    stub_axis, stub_desc = _integration_stub_classes()
    for stub, mirror in ((stub_axis, _native.EsAxis), (stub_desc, _native.ContractDesc)):
        assert ctypes.sizeof(stub) == ctypes.sizeof(mirror), stub.__name__
        names = [f[0] for f in stub._fields_]
        assert names == [f[0] for f in mirror._fields_], stub.__name__
        for name in names:
            a, b = getattr(stub, name), getattr(mirror, name)
            assert (a.offset, a.size) == (b.offset, b.size), (stub.__name__, name)


def test_descriptor_layouts_match_the_header():
    # sizes of the ctypes mirrors equal the C structs (int64 fields, 8 axes per group)
    assert ctypes.sizeof(_native.EsAxis) == 32
    assert ctypes.sizeof(_native.BcastDesc) == 8 + 8 * 32
    assert ctypes.sizeof(_native.ReduceDesc) == 24 + 2 * 8 * 32
    assert _native.ReduceDesc.keep.offset == 24 and _native.ContractDesc.batch.offset == 24
    assert _native.ContractDesc.out_f32.offset == 20 and _native.ReduceDesc.in_f32.offset == 16
    assert ctypes.sizeof(_native.ContractDesc) == 24 + 4 * 8 * 32
    assert ctypes.sizeof(_native.GatherDesc) == 24 + 4 * 8 * 8 + 2 * 8 * 4
    assert ctypes.sizeof(_native.HaloDim) == 32 and _native.HaloDim.extent.offset == 8
    assert ctypes.sizeof(_native.HaloDesc) == 8 + 2 * 32 and _native.HaloDesc.dim.offset == 8


def _status(entry, *args):
    lib = _native.lib()
    return getattr(lib, entry)(*args), lib.es_last_error().decode()


def test_null_descriptor_is_rejected():
    status, message = _status("es_gather", None, None, None, None)
    assert status == _native.ES_ERR_INVALID and "null descriptor" in message
    status, message = _status("es_contract", None, None, None, None, None)
    assert status == _native.ES_ERR_INVALID
    cdesc = _native.ContractDesc()
    cdesc.dtype = 1
    status, message = _status("es_contract_bias", ctypes.byref(cdesc), None, None, None, None, None)
    assert status == _native.ES_ERR_INVALID and "null bias" in message


def test_bad_descriptors_are_rejected_before_any_launch():
    desc = _native.GatherDesc()
    desc.elem_size = 3
    desc.out_rank = 1
    status, message = _status("es_gather", ctypes.byref(desc), None, None, None)
    assert status == _native.ES_ERR_INVALID and "elem_size" in message

    # an input dim fed twice by the same output dim is not a window
    desc.elem_size = 2
    desc.out_rank = 2
    desc.out_size[0] = desc.out_size[1] = 4
    desc.in_rank = 1
    desc.in_size[0] = 8
    desc.in_stride[0] = 1
    desc.pos[0] = desc.win[0] = 1
    status, message = _status("es_gather", ctypes.byref(desc), None, None, None)
    assert status == _native.ES_ERR_INVALID and "same output dim" in message

    cdesc = _native.ContractDesc()
    cdesc.dtype = 7
    status, message = _status("es_contract", ctypes.byref(cdesc), None, None, None, None)
    assert status == _native.ES_ERR_UNSUPPORTED and "dtype" in message

    cdesc.dtype = 1
    cdesc.n_m = 9  # more than ES_MAX_AXES
    status, message = _status("es_contract", ctypes.byref(cdesc), None, None, None, None)
    assert status == _native.ES_ERR_INVALID

    rdesc = _native.ReduceDesc()
    rdesc.dtype = 0
    rdesc.n_keep = 1
    rdesc.keep[0].size = -4
    status, message = _status("es_reduce_workspace_bytes", ctypes.byref(rdesc))
    assert status == _native.ES_ERR_INVALID


def _halo_conv(dtype=1, channels=64):
    """A 3 x 3 convolution over a 16 x 64 x 64 input as es_contract_halo's descriptors:
    M = (b, h, w), N = out channel, K = (kh, kw, c)."""
    desc = _native.ContractDesc()
    desc.dtype = dtype
    c = channels
    m = [(16, 64 * 64 * c, 64 * 64 * 256), (64, 64 * c, 64 * 256), (64, c, 256)]
    desc.n_m = len(m)
    for i, (size, a, cs) in enumerate(m):
        desc.m[i].size, desc.m[i].a, desc.m[i].c = size, a, cs
    desc.n_n = 1
    desc.n[0].size, desc.n[0].b, desc.n[0].c = 256, 9 * c, 1
    k = [(3, 64 * c, 3 * c), (3, c, c), (c, 1, 1)]
    desc.n_k = len(k)
    for i, (size, a, b) in enumerate(k):
        desc.k[i].size, desc.k[i].a, desc.k[i].b = size, a, b
    halo = _native.HaloDesc()
    halo.n = 2
    for s, axis in enumerate((1, 2)):
        halo.dim[s].m_axis, halo.dim[s].extent, halo.dim[s].dilation, halo.dim[s].pad = axis, 64, 1, 1
    return desc, halo


def _halo_status(desc, halo):
    # non-null, 16-byte aligned stand-ins that are never dereferenced: every case below
    # is rejected before a launch.  Where a GPU is present a regression would launch a
    # kernel on them, so these cases run on hosts without one only.
    if torch.cuda.device_count() > 0:
        pytest.skip("stand-in pointers are checked on hosts without a GPU")
    fake = [ctypes.c_void_p(0x10000 * (i + 1)) for i in range(3)]
    return _status("es_contract_halo", ctypes.byref(desc), halo if halo is None else ctypes.byref(halo),
                   fake[0], fake[1], None, fake[2], None)


def test_halo_descriptors_are_checked_before_any_launch():
    desc, halo = _halo_conv()
    status, message = _halo_status(desc, None)
    assert status == _native.ES_ERR_INVALID and "null halo" in message

    desc, halo = _halo_conv()
    halo.n = 3
    status, message = _halo_status(desc, halo)
    assert status == _native.ES_ERR_INVALID and "n must be 1 or 2" in message

    desc, halo = _halo_conv()
    halo.n = 1  # the K group then has one sub-axis too many
    status, message = _halo_status(desc, halo)
    assert status == _native.ES_ERR_INVALID and "taps followed by the channel" in message

    desc, halo = _halo_conv()
    halo.dim[1].m_axis = 1  # both dims on one position axis
    status, message = _halo_status(desc, halo)
    assert status == _native.ES_ERR_INVALID and "m_axis" in message

    desc, halo = _halo_conv()
    halo.dim[0].dilation = 2  # the tap stride says dilation 1
    status, message = _halo_status(desc, halo)
    assert status == _native.ES_ERR_INVALID and "dilation times the position stride" in message

    desc, halo = _halo_conv()
    halo.dim[1].pad = -1
    status, message = _halo_status(desc, halo)
    assert status == _native.ES_ERR_INVALID and "pad" in message


def test_halo_contractions_the_kernel_cannot_take_are_unsupported():
    # ES_ERR_UNSUPPORTED tells einconv to pad instead; nothing is launched
    desc, halo = _halo_conv(dtype=0)  # fp32
    status, message = _halo_status(desc, halo)
    assert status == _native.ES_ERR_UNSUPPORTED and "pipelined kernel" in message

    desc, halo = _halo_conv(channels=96)  # a channel count that is not a whole number of K tiles
    status, message = _halo_status(desc, halo)
    assert status == _native.ES_ERR_UNSUPPORTED

    desc, halo = _halo_conv()
    for s in range(2):  # 7 x 7 taps: more than one mask word
        desc.k[s].size = 7
        halo.dim[s].pad = 3
    status, message = _halo_status(desc, halo)
    assert status == _native.ES_ERR_UNSUPPORTED and "32 taps" in message


def test_empty_problems_need_no_pointers():
    # a zero-extent output returns ES_OK without touching the (null) buffers
    desc = _native.BcastDesc()
    desc.dtype = 0
    desc.rank = 1
    desc.axes[0].size = 0
    status, _ = _status("es_bcast", ctypes.byref(desc), None, None, None, None)
    assert status == _native.ES_OK


def test_reduce_workspace_query_is_pure():
    # few outputs, long rows: the reduction is split and asks for a workspace
    desc = _native.ReduceDesc()
    desc.dtype = 0
    desc.n_keep = 2
    desc.keep[0].size, desc.keep[0].a = 16, 4096 * 4096
    desc.keep[1].size, desc.keep[1].a = 4096, 1
    desc.n_red = 1
    desc.red[0].size, desc.red[0].a = 4096, 4096
    first = _native.lib().es_reduce_workspace_bytes(ctypes.byref(desc))
    second = _native.lib().es_reduce_workspace_bytes(ctypes.byref(desc))
    assert first == second and first > 0 and first % (16 * 4096 * 4) == 0


def test_missing_library_fails_loudly(monkeypatch, tmp_path):
    monkeypatch.setattr(_native, "_lib", None)
    monkeypatch.setenv("EINSHARD_HIP_LIB", str(tmp_path / "nope.so"))
    with pytest.raises(RuntimeError, match="not found"):
        _native.lib()


def test_every_reduction_fits_the_noalloc_scratch():
    # es_reduce_noalloc keeps split partials in ES_NOALLOC_SCRATCH_BYTES of device
    # memory: es_reduce's schedule must never ask for more (it splits only while its
    # grid has fewer than 2048 work-groups); the largest case is a 16-bit column sum
    from torch_einshard._exec import _set_axes
    from torch_einshard.planner import SubAxis
    lib = _native.lib()
    largest = 0
    for dtype in (0, 1, 2):
        for in_f32 in (0, 1):
            for b in (1, 3, 16, 64):
                for h in [2 ** i for i in range(16)] + [3, 100, 1000, 4000]:
                    for n in [2 ** i for i in range(0, 26, 3)]:
                        for rows in (False, True):
                            d = _native.ReduceDesc()
                            d.dtype, d.in_f32 = dtype, in_f32
                            keep = [SubAxis(b, a=n * h), SubAxis(h, a=n if rows else 1)]
                            d.n_keep = _set_axes(d.keep, keep, "t")
                            d.n_red = _set_axes(d.red, [SubAxis(n, a=1 if rows else h)], "t")
                            need = lib.es_reduce_workspace_bytes(ctypes.byref(d))
                            assert 0 <= need <= _native.NOALLOC_SCRATCH_BYTES, (dtype, in_f32, b, n, h, rows, need)
                            largest = max(largest, need)
    assert largest > _native.NOALLOC_SCRATCH_BYTES // 2  # the sweep reaches the bound's neighbourhood
