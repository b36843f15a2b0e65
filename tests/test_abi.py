"""The C ABI boundary, checked without a GPU: the library loads, exports every
entry point include/einshard_hip.h declares, and rejects malformed
descriptors with a status code and message (no kernel is launched)."""

import ctypes
import os
import re
import subprocess

import pytest

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


def test_descriptor_layouts_match_the_header():
    # sizes of the ctypes mirrors equal the C structs (int64 fields, 8 axes per group)
    assert ctypes.sizeof(_native.EsAxis) == 32
    assert ctypes.sizeof(_native.BcastDesc) == 8 + 8 * 32
    assert ctypes.sizeof(_native.ReduceDesc) == 16 + 2 * 8 * 32
    assert ctypes.sizeof(_native.ContractDesc) == 24 + 4 * 8 * 32
    assert ctypes.sizeof(_native.GatherDesc) == 24 + 4 * 8 * 8 + 2 * 8 * 4


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
