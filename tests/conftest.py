import os
import sys

import pytest
import torch

_REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (_REPO, os.path.join(_REPO, "torch-einshard_amd")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def gpu():
    """The device for GPU tests; the HIP library must load (no fallback)."""
    if not torch.cuda.is_available():
        pytest.skip("no ROCm device visible")
    from torch_einshard import _native

    _native.lib()  # raises if libeinshard_hip.so is missing
    return torch.device("cuda:0")


def gen(seed=1234):
    return torch.Generator().manual_seed(seed)


def randn(*shape, seed=1234, dtype=torch.float32, scale=1.0):
    """Seeded CPU normal draws (fp32, then cast) — the benchmark input recipe."""
    return (torch.randn(*shape, generator=gen(seed)) * scale).to(dtype)


def rel_error(actual, expected):
    """max |a - e| / max(max|e|, rms(e)): relative error with a scale floor."""
    a = actual.detach().cpu().to(torch.float64)
    e = expected.detach().cpu().to(torch.float64)
    if e.numel() == 0:
        return 0.0
    scale = max(e.abs().max().item(), e.pow(2).mean().sqrt().item(), 1e-30)
    return (a - e).abs().max().item() / scale


def assert_rel(actual, expected, tol):
    assert tuple(actual.shape) == tuple(expected.shape), (tuple(actual.shape), tuple(expected.shape))
    err = rel_error(actual, expected)
    assert err <= tol, f"relative error {err:.3e} > {tol:.1e}"
    return err


def assert_bitexact(actual, expected):
    a = actual.detach().cpu()
    e = expected.detach().cpu()
    assert tuple(a.shape) == tuple(e.shape), (tuple(a.shape), tuple(e.shape))
    assert a.dtype == e.dtype, (a.dtype, e.dtype)
    if a.numel():
        av = a.contiguous().view(torch.uint8) if a.element_size() == 1 else a.contiguous().view(
            {2: torch.int16, 4: torch.int32, 8: torch.int64}[a.element_size()]
        )
        ev = e.contiguous().view(torch.uint8) if e.element_size() == 1 else e.contiguous().view(
            {2: torch.int16, 4: torch.int32, 8: torch.int64}[e.element_size()]
        )
        differ = av != ev
        mismatches = differ.sum().item()
        if mismatches:
            where = differ.nonzero()[:4].tolist()
            shown = ", ".join(
                f"{tuple(i)}: {av[tuple(i)].item() & 0xffffffffffffffff:#x} != {ev[tuple(i)].item() & 0xffffffffffffffff:#x}"
                for i in where
            )
            raise AssertionError(f"{mismatches} of {a.numel()} elements differ bitwise; first at {shown}")


def assert_bitexact_nan(actual, expected):
    """Bit-exact except that a NaN only has to meet a NaN: contraction outputs are one
    rounding of the fp32 result, and torch itself rounds NaN to different bf16 bit
    patterns (0x7FC0 in scalar code, 0xFFFF in vectorised code)."""
    a = actual.detach().cpu()
    e = expected.detach().cpu()
    assert tuple(a.shape) == tuple(e.shape), (tuple(a.shape), tuple(e.shape))
    nan_a, nan_e = a.isnan(), e.isnan()
    assert torch.equal(nan_a, nan_e), f"NaN positions differ: {(nan_a != nan_e).sum().item()} elements"
    assert_bitexact(a.masked_fill(nan_a, 0), e.masked_fill(nan_e, 0))


# tolerances stated by the north star: fp32 1e-5 relative, bf16 2e-2 relative
TOL = {torch.float32: 1e-5, torch.bfloat16: 2e-2, torch.float16: 5e-3}
