"""Parity at the benchmark configurations' full sizes.

Every workload is launched at its exact shape and dtype, so the kernels, tile
shapes and split grids checked here are the ones the benchmark times.  The
reference computes each of them with one ``torch.einsum`` on CPU tensors
(reference src/torch_einshard/einsum.py:132); the oracle restates that call.

* C1 (fp32 1024^3): the whole output against the oracle at 1e-5, and both the
  device's and the reference CPU path's error against an fp64 einsum within 1e-5.
* C2 and C4 (bf16): against the reference's own bf16 path (``torch.einsum`` on
  bf16 CPU tensors) at 2e-2, and against an fp64 einsum of the same bf16 inputs,
  where the device result must be no less accurate than the reference's CPU
  result.  C4's whole output is also checked against the fp32 CPU product
  rounded to bf16; its bf16-path and fp64 comparisons use 512 rows, one in each
  run of 32, at every residue mod 32 (so every row position of a 16-row MFMA
  block and of a 32-row group) and 8 in each of the 64 M tiles.
* C5a / C5c (fp32 sums) at 1e-5 and C5b (one multiply per element) bit-exact,
  on the full-size launches, each compared on the slices b = 0, 7, 15 of its
  output; each slice's oracle runs on the matching input slice.

Every input follows the benchmark's recipe (bench.py): ``torch.Generator`` seed
1234 on the CPU, bf16 by casting fp32 draws, copied to the device.  C5a draws
x[8,16,4096,4096]; C5b draws y[16,4096,4096] then s[4096] from a fresh seed-1234
generator, and C5c sums that same y (its own fresh draw is the same tensor).
"""

import pytest
import torch

import torch_einshard as es
from oracle.einshard_oracle import einshard_cpu
from torch_einshard import _native

from conftest import TOL, assert_bitexact, assert_rel, rel_error

pytestmark = pytest.mark.gpu

SEED = 1234


def _cpu_gen():
    return torch.Generator().manual_seed(SEED)


def _fp64_errors(expr, got, cpu_out, inputs):
    """(device error, CPU error), each relative to an fp64 einsum of the same inputs."""
    ref = einshard_cpu(expr, *[x.double() for x in inputs])
    return rel_error(got, ref), rel_error(cpu_out, ref)


def test_c1_fp32_contraction_full_size(gpu):
    g = _cpu_gen()
    x = torch.randn(1024, 1024, generator=g)
    y = torch.randn(1024, 1024, generator=g)
    got = es.einshard("a b, b c -> a c", x.to(gpu), y.to(gpu))
    kernel = _native.last_kernel()
    assert kernel.startswith("contract_") and "generic" not in kernel, kernel
    want = einshard_cpu("a b, b c -> a c", x, y)
    assert_rel(got, want, TOL[torch.float32])
    # against the exact (fp64) result both are well inside the tolerance; the CPU's
    # blocked GEMM sums in shorter chains than the kernel's K-sequential fp32
    # accumulation (measured: 3.4e-7 against 1.2e-6)
    gpu_err, cpu_err = _fp64_errors("a b, b c -> a c", got, want, [x, y])
    print(f"C1 error vs fp64: device {gpu_err:.3e}, reference CPU path {cpu_err:.3e}")
    assert gpu_err <= TOL[torch.float32] and cpu_err <= TOL[torch.float32], (gpu_err, cpu_err)


def test_c2_permuted_contraction_against_the_bf16_cpu_path(gpu):
    g = _cpu_gen()
    x = torch.randn(64, 32, 128, 64, generator=g).to(torch.bfloat16)
    y = torch.randn(32, 64, 128, 16, generator=g).to(torch.bfloat16)
    expr = "a b k c, b c l d -> k l d a"
    got = es.einshard(expr, x.to(gpu), y.to(gpu))
    assert _native.last_kernel() == "contract_pipe_256x256_mn_a"
    cpu_bf16 = einshard_cpu(expr, x, y)  # the reference's own computation on bf16 tensors
    assert cpu_bf16.dtype == torch.bfloat16
    assert_rel(got, cpu_bf16, TOL[torch.bfloat16])
    gpu_err, cpu_err = _fp64_errors(expr, got, cpu_bf16, [x, y])
    print(f"C2 error vs fp64: device {gpu_err:.3e}, reference CPU path {cpu_err:.3e}")
    assert gpu_err <= 2 * cpu_err + 1e-4, (gpu_err, cpu_err)


def test_c4_headline_contraction_full_size(gpu):
    g = _cpu_gen()
    x = (torch.randn(8, 2048, 4096, generator=g) * 0.02).to(torch.bfloat16)
    w = (torch.randn(1792, 4096, generator=g) * 0.02).to(torch.bfloat16)
    got = es.einshard("b n c, h c -> b n h", x.to(gpu), w.to(gpu))
    assert _native.last_kernel() == "contract_pipe_256x224"
    assert got.shape == (8, 2048, 1792) and got.dtype == torch.bfloat16
    # every output element against the fp32 product on the CPU, rounded to bf16
    full32 = einshard_cpu("m c, h c -> m h", x.reshape(16384, 4096).float(), w.float())
    assert_rel(got.reshape(16384, 1792).cpu(), full32.to(torch.bfloat16), TOL[torch.bfloat16])
    del full32
    # 512 rows, row 32 i + (i mod 32): one in each run of 32 rows, every residue mod 32
    # (each row of a 16-row MFMA block and of a 32-row group), eight in each M tile
    i = torch.arange(512)
    rows = 32 * i + i % 32
    assert sorted(set((rows % 32).tolist())) == list(range(32))
    assert sorted(set((rows // 256).tolist())) == list(range(64))
    xs = x.reshape(16384, 4096)[rows]
    dev_rows = got.reshape(16384, 1792)[rows.to(gpu)].cpu()
    cpu_bf16 = einshard_cpu("m c, h c -> m h", xs, w)  # the reference's bf16 path on those rows
    assert_rel(dev_rows, cpu_bf16, TOL[torch.bfloat16])
    want32 = einshard_cpu("m c, h c -> m h", xs.float(), w.float()).to(torch.bfloat16)
    assert_rel(dev_rows, want32, TOL[torch.bfloat16])
    gpu_err, cpu_err = _fp64_errors("m c, h c -> m h", dev_rows, cpu_bf16, [xs, w])
    print(f"C4 error vs fp64: device {gpu_err:.3e}, reference CPU path {cpu_err:.3e}")
    assert gpu_err <= 2 * cpu_err + 1e-4, (gpu_err, cpu_err)
    # no row of the launch is left unwritten or non-finite
    assert torch.isfinite(got).all().item()


@pytest.fixture(scope="module")
def c5_runs(gpu):
    """The three config-5 launches at full size on the benchmark's inputs: partials
    p b n h -> b n h over x, the scale b n h, h -> b n h over (y, s), the sum
    b n h -> b h over y; slices b = 0, 7, 15 of every input and output on the host."""
    x = torch.rand(8, 16, 4096, 4096, generator=_cpu_gen()) * 2 - 1  # ~30 s of draws
    g = _cpu_gen()
    y = torch.rand(16, 4096, 4096, generator=g) * 2 - 1
    s = torch.rand(4096, generator=g) * 2 - 1
    bs = (0, 7, 15)
    out = {"s": s, "x": {b: x[:, b].clone() for b in bs}, "y": {b: y[b].clone() for b in bs}}
    xd = x.to(gpu)
    del x
    r_a = es.einshard("p b n h -> b n h", xd)
    k_a = _native.last_kernel()
    del xd
    yd, sd = y.to(gpu), s.to(gpu)
    del y
    r_b = es.einshard("b n h, h -> b n h", yd, sd)
    k_b = _native.last_kernel()
    r_c = es.einshard("b n h -> b h", yd)
    k_c = _native.last_kernel()
    torch.cuda.synchronize()
    out["kernels"] = (k_a, k_b, k_c)
    out["a"] = {b: r_a[b].cpu() for b in bs}
    out["b"] = {b: r_b[b].cpu() for b in bs}
    out["c"] = {b: r_c[b].cpu() for b in bs}
    del yd, sd, r_a, r_b, r_c
    torch.cuda.empty_cache()
    return out


def test_c5a_partial_sum_full_size(c5_runs):
    assert c5_runs["kernels"][0] == "reduce_cols"
    for b, got in c5_runs["a"].items():
        want = einshard_cpu("p n h -> n h", c5_runs["x"][b])
        assert_rel(got, want, TOL[torch.float32])


def test_c5b_scale_broadcast_full_size_is_bitexact(c5_runs):
    kernel = c5_runs["kernels"][1]
    assert kernel.startswith("bcast_") and kernel != "bcast_scalar", kernel  # 16-byte vectors
    for b, got in c5_runs["b"].items():
        assert_bitexact(got, einshard_cpu("n h, h -> n h", c5_runs["y"][b], c5_runs["s"]))


def test_c5c_middle_axis_sum_full_size(c5_runs):
    # [16, 4096, 4096] -> [16, 4096]: 16 x 4096 outputs split over the reduced axis
    # (reduce_cols writing partials, then reduce_finish), the grid the benchmark runs
    assert c5_runs["kernels"][2] == "reduce_cols"
    for b, got in c5_runs["c"].items():
        want = einshard_cpu("n h -> h", c5_runs["y"][b])
        assert_rel(got, want, TOL[torch.float32])
