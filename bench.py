"""Benchmark of torch_einshard's MI355X path (one JSON line per workload).

    python bench.py [--gpus 1] [--steps K] [--warmup W]
                    [--workload c4|c1|c2|c3|c5a|c5b|c5c|conv|partition|roll|all|...]

A step is one es.einshard / es.einwindow / es.einconv call over one batch of synthetic
input that is already resident in HBM.  The default workload is config 4 of
BASELINE.json — one rank's share of a tensor-parallel contraction,
es.einshard("b n c, h c -> b n h") with x[8,2048,4096], w[1792,4096] bf16 —
the configuration the north star's headline target (>= 70 % of bf16 MFMA peak)
is quoted on.  The other configs are parity cases; ``--workload`` measures them
individually with the same method.  ``conv`` (not a BASELINE config) measures
es.einconv, the halo + convolution the reference runs through F.conv2d;
``partition`` and ``roll`` are the reference's own local benchmarks of a family
permute and of einroll (benchmarks/bench_local.py, "large" size).  ``copy`` and
``dma_calib`` calibrate the traffic counters; ``vendor_c1``, ``vendor_c2`` and
``vendor_c4`` time torch's own GPU path (hipBLASLt) on configs 1, 2 and 4,
``vendor_conv`` the reference's GPU path of einconv (F.pad, F.conv2d on MIOpen),
``vendor_c3`` and ``vendor_c5a``/``b``/``c`` its torch calls for configs 3 and 5, and
``vendor_partition`` and ``vendor_roll`` torch's own device copy of the same bytes
as ``partition`` and ``roll``, as reference points.  ``all`` runs every workload but the calibrations and
reference points.  ``--vs-vendor`` (with any workload that has a ``vendor_`` point) times this library's launch and
the workload's reference point alternately on the same inputs, warm and flushed, the
order swapped every round, so both see the same clock and power state of the board
(dispatch times of either climb by up to 40 % and fall back over a run as the board
limits its power); it prints one line with both.

Timing: W untimed warm-up steps, then K back-to-back steps between two device
synchronisations (wall clock -> ms_per_step, value: host work included).  The
kernel's durations come from HIP events recorded on the stream the kernel runs on
(torch's current stream, which the library launches on):
  * roofline.kernel_ms / achieved / frac: K more launches, each after the 256 MB
    Infinity Cache and the L2s are flushed by a 512 MiB read -- cold operands,
    one launch's own ramp and drain included.  The time per launch is that of K x (flush, launch) minus that of
    K x flush, both queued behind the spin kernel (an event pair around each
    launch would add ~5-8 us of event overhead to every launch);
  * roofline.kernel_ms_warm / achieved_warm / frac_warm: K launches queued back to
    back behind a bounded spin kernel (no host gaps), operands resident in cache.
As in ``timeit``, Python's cyclic garbage collector is run before and switched
off during the timed loops: a full collection pauses the interpreter for tens of
milliseconds at a random call and has nothing to do with the library.

roofline.achieved uses algorithmic work only: 2*M*N*K flops for contractions
(for einconv, of the implicit GEMM alone, timed without the two gathers around it),
unique input bytes + output bytes for the copy / reduce / broadcast kernels.
cpu_baseline times the reference's CPU path as restated by oracle/ on the host
cores (torch.einsum / F.pad + unfold + permute on CPU tensors): on the whole
workload for configs 1, 2 and 4 (a few full-size calls), on a bounded sample of it
for the others, scaled to the same unit.  parity compares the device result on the
parity sample with the CPU path's (bit-exact for copies), and both with the same
computation in fp64.
"""

import argparse
import gc
import json
import os
import sys
import time

_REPO = os.path.dirname(os.path.abspath(__file__))
for _path in (os.path.join(_REPO, "torch-einshard_amd"), _REPO):
    if _path not in sys.path:
        sys.path.insert(0, _path)

import torch  # noqa: E402

# spin of the queue-priming kernel: ~10-25 ms, far longer than the host needs
# to enqueue K launches
PRIME_CYCLES = 50_000_000

METRIC = "einshard contraction TFLOP/s; einwindow/reduce GB/s; % of MI355X roofline"
PEAK = {
    "bf16": 2500.0,  # TFLOP/s, dense MFMA
    "f16": 2500.0,
    "f32": 157.3,  # TFLOP/s, fp32 MFMA
    "hbm": 8000.0,  # GB/s
}
SEED = 1234


def _gen():
    return torch.Generator().manual_seed(SEED)


# ---- workloads ---------------------------------------------------------------------------
# each returns dict(name, call(inputs)->out, inputs, flops|bytes, unit, bound, dtype, cpu)


def wl_c1(dev):
    g = _gen()
    x = torch.randn(1024, 1024, generator=g)
    y = torch.randn(1024, 1024, generator=g)
    return dict(
        key="c1",
        workload="config1: es.einshard('a b, b c -> a c') x,y [1024,1024] fp32",
        expr="a b, b c -> a c",
        host=[x, y],
        flops=2 * 1024**3,
        dtype="f32",
        bound="mfma",
        peak=PEAK["f32"],
        sample=lambda xs: ([xs[0], xs[1]], 1.0),
    )


def wl_c2(dev):
    g = _gen()
    x = torch.randn(64, 32, 128, 64, generator=g).to(torch.bfloat16)
    y = torch.randn(32, 64, 128, 16, generator=g).to(torch.bfloat16)
    return dict(
        key="c2",
        workload="config2: es.einshard('a b k c, b c l d -> k l d a') a=64 b=32 k=128 c=64 l=128 d=16 bf16",
        expr="a b k c, b c l d -> k l d a",
        host=[x, y],
        flops=2 * 8192 * 2048 * 2048,
        dtype="bf16",
        bound="mfma",
        peak=PEAK["bf16"],
        sample=lambda xs: ([xs[0][:8], xs[1]], 8 / 64),
        cpu_sample=lambda xs: (list(xs), 1.0),
    )


def wl_c4(dev):
    g = _gen()
    x = (torch.randn(8, 2048, 4096, generator=g) * 0.02).to(torch.bfloat16)
    w = (torch.randn(1792, 4096, generator=g) * 0.02).to(torch.bfloat16)
    return dict(
        key="c4",
        workload="config4: es.einshard('b n c, h c -> b n h') x[8,2048,4096] w[1792,4096] bf16 (one TP rank's share)",
        expr="b n c, h c -> b n h",
        host=[x, w],
        flops=2 * 16384 * 1792 * 4096,
        dtype="bf16",
        bound="mfma",
        peak=PEAK["bf16"],
        sample=lambda xs: ([xs[0][:1, :512], xs[1]], 512 / 16384),
        cpu_sample=lambda xs: (list(xs), 1.0),
    )


def wl_c3(dev):
    g = _gen()
    x = torch.randn(8, 256, 256, 64, generator=g).to(torch.bfloat16)
    return dict(
        key="c3",
        workload="config3: es.einwindow('b h w c -> b h w kh kw c', {h:kh, w:kw}, {h:1, w:1}) x[8,256,256,64] bf16",
        window=("b h w c -> b h w kh kw c", {"h": "kh", "w": "kw"}, {"h": 1, "w": 1}),
        copy_only=True,
        host=[x],
        bytes=8 * 256 * 256 * 64 * 2 + 8 * 256 * 256 * 9 * 64 * 2,
        dtype="bf16",
        bound="hbm",
        peak=PEAK["hbm"],
        sample=lambda xs: ([xs[0][:1]], 1 / 8),
    )


def _c5_input():
    g = _gen()
    return torch.rand(8, 16, 4096, 4096, generator=g) * 2 - 1


def wl_c5a(dev):
    x = _c5_input()
    return dict(
        key="c5a",
        workload="config5a: es.einshard('p b n h -> b n h') P=8 b=16 n=h=4096 fp32",
        expr="p b n h -> b n h",
        host=[x],
        bytes=8 * 16 * 4096 * 4096 * 4 + 16 * 4096 * 4096 * 4,
        dtype="f32",
        bound="hbm",
        peak=PEAK["hbm"],
        sample=lambda xs: ([xs[0][:, :1]], 1 / 16),
    )


def wl_c5b(dev):
    g = _gen()
    y = torch.rand(16, 4096, 4096, generator=g) * 2 - 1
    s = torch.rand(4096, generator=g) * 2 - 1
    return dict(
        key="c5b",
        workload="config5b: es.einshard('b n h, h -> b n h') b=16 n=h=4096 fp32",
        expr="b n h, h -> b n h",
        host=[y, s],
        bytes=2 * 16 * 4096 * 4096 * 4 + 4096 * 4,
        dtype="f32",
        bound="hbm",
        peak=PEAK["hbm"],
        sample=lambda xs: ([xs[0][:2], xs[1]], 2 / 16),
    )


def wl_c5c(dev):
    g = _gen()
    z = torch.rand(16, 4096, 4096, generator=g) * 2 - 1
    return dict(
        key="c5c",
        workload="config5c: es.einshard('b n h -> b h') b=16 n=h=4096 fp32",
        expr="b n h -> b h",
        host=[z],
        bytes=16 * 4096 * 4096 * 4 + 16 * 4096 * 4,
        dtype="f32",
        bound="hbm",
        peak=PEAK["hbm"],
        sample=lambda xs: ([xs[0][:2]], 2 / 16),
    )


def wl_conv(dev):
    g = _gen()
    x = torch.randn(16, 64, 64, 256, generator=g).to(torch.bfloat16)
    w = (torch.randn(256, 256, 3, 3, generator=g) * 0.02).to(torch.bfloat16)
    b = torch.randn(256, generator=g).to(torch.bfloat16)
    return dict(
        key="conv",
        workload=(
            "einconv: es.einconv('b h w c, o c kh kw -> b h w o', {h:kh, w:kw}, bias) x[16,64,64,256] "
            "w[256,256,3,3] bf16, same padding, forward (checkpoint=False)"
        ),
        conv=("b h w c, o c kh kw -> b h w o", {"h": "kh", "w": "kw"}),
        host=[x, w, b],
        flops=2 * (16 * 64 * 64) * 256 * (9 * 256),
        dtype="bf16",
        bound="mfma",
        peak=PEAK["bf16"],
        sample=lambda xs: ([xs[0][:1], xs[1], xs[2]], 1 / 16),
    )


def wl_partition(dev):
    g = _gen()
    x = torch.randn(4, 2, 128, 128, 128, generator=g)
    families = {"spatial": ("h", "w"), "window": ("wh", "ww")}
    return dict(
        key="partition",
        workload=(
            "window partition (reference benchmarks/bench_local.py:95-126, large): es.einshard('b t "
            "[*spatial *window] c -> (b *spatial) t *window c', families, sizes={window: (8, 8)}) "
            "x[4,2,128,128,128] fp32"
        ),
        gpu_call=lambda es, xs: es.einshard(
            "b t [*spatial *window] c -> (b *spatial) t *window c", xs[0], families=families, sizes={"window": (8, 8)}
        ),
        cpu_call=lambda xs: _oracle().einshard_cpu(
            "b t (h wh) (w ww) c -> (b h w) t wh ww c", xs[0], sizes={"wh": 8, "ww": 8}
        ),
        copy_only=True,
        host=[x],
        bytes=2 * 4 * 2 * 128 * 128 * 128 * 4,
        dtype="f32",
        bound="hbm",
        peak=PEAK["hbm"],
        sample=lambda xs: ([xs[0][:1]], 1 / 4),
    )


def wl_roll(dev):
    g = _gen()
    x = torch.randn(4, 128, 128, 128, generator=g)
    return dict(
        key="roll",
        workload=(
            "einroll (reference benchmarks/bench_local.py:212-229, large): es.einroll('b h w c', "
            "{h: 3, w: -5}) x[4,128,128,128] fp32"
        ),
        gpu_call=lambda es, xs: es.einroll("b h w c", xs[0], {"h": 3, "w": -5}),
        cpu_call=lambda xs: _oracle().einroll_cpu("b h w c", xs[0], {"h": 3, "w": -5}),
        copy_only=True,
        host=[x],
        bytes=2 * 4 * 128 * 128 * 128 * 4,
        dtype="f32",
        bound="hbm",
        peak=PEAK["hbm"],
        sample=lambda xs: ([xs[0][:1]], 1 / 4),
    )


def _oracle():
    from oracle import einshard_oracle

    return einshard_oracle


def wl_copy(dev):
    """Calibration: a plain 1 GiB copy through the same gather kernel (known traffic)."""
    x = torch.empty(16384, 16384, dtype=torch.float32).fill_(1.0)
    return dict(
        key="copy",
        workload="calibration: es.einshard('a b -> a b') x[16384,16384] fp32 (1 GiB read + 1 GiB write)",
        expr="a b -> a b",
        copy_only=True,
        host=[x],
        bytes=2 * 16384 * 16384 * 4,
        dtype="f32",
        bound="hbm",
        peak=PEAK["hbm"],
        sample=lambda xs: ([xs[0][:1024]], 1 / 16),
    )


def wl_dma_calib(dev):
    """Calibration of the traffic counters for LDS-DMA reads: a contraction whose 512 MiB
    first operand is read exactly once (one N tile), through global_load_lds_dwordx4."""
    g = _gen()
    x = (torch.randn(65536, 4096, generator=g) * 0.02).to(torch.bfloat16)
    w = (torch.randn(256, 4096, generator=g) * 0.02).to(torch.bfloat16)
    return dict(
        key="dma_calib",
        workload=("calibration: es.einshard('m k, n k -> m n') x[65536,4096] w[256,4096] bf16: x read once "
                  "by LDS-DMA (256 tiles of 256 x 256, one column), w from cache"),
        expr="m k, n k -> m n",
        host=[x, w],
        flops=2 * 65536 * 256 * 4096,
        bytes=65536 * 4096 * 2 + 256 * 4096 * 2 + 65536 * 256 * 2,
        dtype="bf16",
        bound="mfma",
        peak=PEAK["bf16"],
        sample=lambda xs: ([xs[0][:512], xs[1]], 512 / 65536),
    )


def wl_vendor_c4(dev):
    """Reference point, not this library: hipBLASLt (torch.matmul) on config 4's shape."""
    wl = wl_c4(dev)
    wl.update(
        key="vendor_c4",
        workload="reference: torch.matmul (hipBLASLt) on config 4's shape x[16384,4096] @ w[1792,4096]^T bf16",
        gpu_call=lambda es, xs: torch.matmul(xs[0].view(-1, 4096), xs[1].t()),
        kernel_name="torch.matmul (hipBLASLt)",
        cpu_call=lambda xs: torch.matmul(xs[0].reshape(-1, 4096), xs[1].t()),
    )
    return wl


def wl_vendor_c1(dev):
    """Reference point, not this library: hipBLASLt (torch.matmul, full fp32, no TF32) on
    config 1's shape."""
    wl = wl_c1(dev)

    def call(es, xs):
        assert not torch.backends.cuda.matmul.allow_tf32, "config 1 is full fp32"
        return torch.matmul(xs[0], xs[1])

    wl.update(
        key="vendor_c1",
        workload="reference: torch.matmul (hipBLASLt, fp32) on config 1's shape x,y [1024,1024]",
        gpu_call=call,
        kernel_name="torch.matmul (hipBLASLt)",
        cpu_call=lambda xs: torch.matmul(xs[0], xs[1]),
    )
    return wl


def wl_vendor_c2(dev):
    """Reference point, not this library: config 2 the way torch.einsum runs it on a GPU
    (operands permuted into one matrix product, torch.matmul, the result permuted back),
    with every operand of the product contiguous."""
    wl = wl_c2(dev)

    def call(es, xs):
        na, nb, nk, nc = xs[0].shape
        _, _, nl, nd = xs[1].shape
        a = xs[0].permute(0, 2, 1, 3).contiguous().view(na * nk, nb * nc)  # (a k, b c)
        prod = torch.matmul(a, xs[1].view(nb * nc, nl * nd))  # (a k, l d)
        return prod.view(na, nk, nl, nd).permute(1, 2, 3, 0).contiguous()  # k l d a

    wl.update(
        key="vendor_c2",
        workload=("reference: config 2 as torch.einsum runs it on a GPU (permute x, torch.matmul, "
                  "permute the result), bf16"),
        gpu_call=call,
        kernel_name="permute + torch.matmul (hipBLASLt) + permute",
        cpu_call=lambda xs: torch.einsum("abkc,bcld->klda", xs[0], xs[1]),
    )
    return wl


def wl_vendor_conv(dev):
    """Reference point, not this library: einconv's convolution the way the reference runs
    it on a GPU (conv.py:153-207): the halo padded (F.pad), the input permuted to
    (batch, channel, h, w), F.conv2d with padding 0 and the bias (MIOpen), the result
    permuted back."""
    wl = wl_conv(dev)

    def call(es, xs):
        x, w, b = xs
        z = torch.nn.functional.pad(x, (0, 0, 1, 1, 1, 1)).permute(0, 3, 1, 2).contiguous()
        return torch.nn.functional.conv2d(z, w, b, padding=0).permute(0, 2, 3, 1).contiguous()

    wl.update(
        key="vendor_conv",
        workload=("reference: einconv's convolution as the reference runs it on a GPU "
                  "(F.pad, permute, F.conv2d (MIOpen), permute), bf16"),
        gpu_call=call,
        kernel_name="F.pad + permute + F.conv2d (MIOpen) + permute",
        cpu_call=lambda xs: call(None, xs),
    )
    return wl


def _vendor_torch(wl, key, what, call):
    """Reference point, not this library: the workload the way the reference runs it on a
    GPU, through torch's own kernels."""
    wl.update(key=key, workload=f"reference: {what} (torch's own GPU kernels)", gpu_call=lambda es, xs: call(xs),
              kernel_name=what, cpu_call=call)
    return wl


def wl_vendor_c3(dev):
    # halo.py:402-418: F.pad, unfold along each windowed axis, permute, contiguous
    def call(xs):
        z = torch.nn.functional.pad(xs[0], (0, 0, 1, 1, 1, 1)).unfold(1, 3, 1).unfold(2, 3, 1)
        return z.permute(0, 1, 2, 4, 5, 3).contiguous()  # b h w c kh kw -> b h w kh kw c

    return _vendor_torch(wl_c3(dev), "vendor_c3", "F.pad + unfold + permute().contiguous()", call)


def wl_vendor_c5a(dev):
    return _vendor_torch(wl_c5a(dev), "vendor_c5a", "torch.sum over p", lambda xs: xs[0].sum(0))


def wl_vendor_c5b(dev):
    return _vendor_torch(wl_c5b(dev), "vendor_c5b", "torch.mul with broadcasting", lambda xs: xs[0] * xs[1])


def wl_vendor_c5c(dev):
    return _vendor_torch(wl_c5c(dev), "vendor_c5c", "torch.sum over n", lambda xs: xs[0].sum(1))


def _vendor_copy(wl, key, what):
    """Reference point, not this library: torch's own device copy (``Tensor.clone`` of a
    contiguous tensor, hipMemcpyAsync device to device) of the same bytes as ``wl``."""
    wl.update(
        key=key,
        workload=f"reference: torch clone (hipMemcpyAsync device to device) of {what}'s input, the same bytes",
        gpu_call=lambda es, xs: xs[0].clone(),
        kernel_name="torch clone (hipMemcpyAsync)",
        cpu_call=lambda xs: xs[0].clone(),
    )
    return wl


def wl_vendor_roll(dev):
    return _vendor_copy(wl_roll(dev), "vendor_roll", "roll")


def wl_vendor_partition(dev):
    return _vendor_copy(wl_partition(dev), "vendor_partition", "partition")


WORKLOADS = {
    "c1": wl_c1,
    "c2": wl_c2,
    "c3": wl_c3,
    "c4": wl_c4,
    "c5a": wl_c5a,
    "c5b": wl_c5b,
    "c5c": wl_c5c,
    "conv": wl_conv,
    "partition": wl_partition,
    "roll": wl_roll,
    "copy": wl_copy,
    "dma_calib": wl_dma_calib,
    "vendor_c1": wl_vendor_c1,
    "vendor_c2": wl_vendor_c2,
    "vendor_c3": wl_vendor_c3,
    "vendor_c4": wl_vendor_c4,
    "vendor_c5a": wl_vendor_c5a,
    "vendor_c5b": wl_vendor_c5b,
    "vendor_c5c": wl_vendor_c5c,
    "vendor_conv": wl_vendor_conv,
    "vendor_partition": wl_vendor_partition,
    "vendor_roll": wl_vendor_roll,
}


def _runner(es, wl):
    if "gpu_call" in wl:
        return lambda xs: wl["gpu_call"](es, xs)
    if "conv" in wl:
        expr, windows = wl["conv"]
        return lambda xs: es.einconv(expr, xs[0], xs[1], windows, bias=xs[2], checkpoint=False)
    if "window" in wl:
        expr, windows, radius = wl["window"]
        return lambda xs: es.einwindow(expr, xs[0], windows, radius)
    expr = wl["expr"]
    return lambda xs: es.einshard(expr, *xs)


def _kernel_runner(es, wl, xs):
    """The dominant kernel alone: for einconv the implicit GEMM read straight from the
    unpadded input (es_contract_halo, zero padding 1 on h and w), with the weight
    already in (out channel, kernel..., channel) order."""
    if "conv" not in wl:
        return _runner(es, wl), xs
    from torch_einshard.conv import _conv_launch, _halo_prepare

    wk = es.einshard("o c kh kw -> o kh kw c", xs[1])
    prep = _halo_prepare(xs[0], wk, (0, 1, 2, 3), ((1, 1), (1, 1)), (1, 1), (0, 1, 2, 3))
    return (lambda ys: _conv_launch(prep, ys[0], ys[1], ys[2])), [xs[0], wk, xs[2]]


def _cpu_runner(wl):
    from oracle.einshard_oracle import einconv_cpu, einshard_cpu, einwindow_cpu

    if "cpu_call" in wl:
        return wl["cpu_call"]
    if "conv" in wl:
        expr, windows = wl["conv"]
        return lambda xs: einconv_cpu(expr, xs[0], xs[1], windows, bias=xs[2])
    if "window" in wl:
        expr, windows, radius = wl["window"]
        return lambda xs: einwindow_cpu(expr, xs[0], windows, radius)
    expr = wl["expr"]
    return lambda xs: einshard_cpu(expr, *xs)


def measure_gpu(es, wl, dev, steps, warmup):
    gc.collect()
    gc.disable()
    try:
        return _measure_gpu(es, wl, dev, steps, warmup)
    finally:
        gc.enable()


def _measure_gpu(es, wl, dev, steps, warmup):
    xs = [t.to(dev) for t in wl["host"]]
    run = _runner(es, wl)
    for _ in range(warmup):
        run(xs)
    torch.cuda.synchronize(dev)
    t0 = time.perf_counter()
    for _ in range(steps):
        out = run(xs)
    torch.cuda.synchronize(dev)
    wall = time.perf_counter() - t0
    del out
    run, xs = _kernel_runner(es, wl, xs)
    run(xs)
    kernel_ms = _time_warm(run, xs, dev, steps)
    flush = _flush_buffer(dev)
    cold_ms = _time_flushed(run, xs, dev, steps, flush)
    del flush
    from torch_einshard import _native

    return dict(wall_s=wall, kernel_ms=kernel_ms, cold_ms=cold_ms, kernel=wl.get("kernel_name") or _native.last_kernel())


def _time_warm(run, xs, dev, steps):
    """ms per launch of K launches queued behind a bounded spin kernel, so that the host
    has enqueued all of them before the first starts and the two events bracket
    back-to-back kernels only (no host gaps)."""
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    torch.cuda._sleep(PRIME_CYCLES)
    start.record(stream)
    for _ in range(steps):
        out = run(xs)
    end.record(stream)
    torch.cuda.synchronize(dev)
    del out
    return start.elapsed_time(end) / steps


def _flush_buffer(dev):
    """512 MiB read by every flush: it evicts the 256 MB Infinity Cache and the L2s and
    leaves no dirty lines behind to be written back during the next launch (float32,
    since a sum of int32 would first convert to int64, writing 1 GiB)."""
    flush = torch.ones(512 * 1024 * 1024 // 4, dtype=torch.float32, device=dev)
    flush.sum()
    return flush


def _time_flushed(run, xs, dev, steps, flush):
    """ms per launch, each launch right after a flush: the difference of two batches timed
    the same way, K x (flush, launch) and K x flush, each queued behind the spin kernel.
    An event pair around every single launch would add ~5-8 us of event overhead per
    launch (checked against rocprofv3 kernel durations)."""
    stream = torch.cuda.current_stream(dev)
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)

    def batch(with_kernel):
        torch.cuda.synchronize(dev)
        torch.cuda._sleep(PRIME_CYCLES)
        start.record(stream)
        for _ in range(steps):
            flush.sum()
            if with_kernel:
                run(xs)
        end.record(stream)
        torch.cuda.synchronize(dev)
        return start.elapsed_time(end)

    both, alone = batch(True), batch(False)
    return (both - alone) / steps


def measure_vs_vendor(es, key, dev, steps, warmup, rounds):
    """This library's launch and torch's own GPU path for the same workload (``vendor_<key>``:
    hipBLASLt), timed alternately on the same inputs: each round times both, warm and
    flushed, the order swapped every round, so that both see the same clock and power
    state of the board.  Returns one JSON-ready dict with every round's figures."""
    wl, vendor = WORKLOADS[key](dev), WORKLOADS[f"vendor_{key}"](dev)
    xs = [t.to(dev) for t in wl["host"]]
    legs = {"einshard": _runner(es, wl), "vendor": _runner(es, vendor)}
    gc.collect()
    gc.disable()
    try:
        for _ in range(warmup):
            for run in legs.values():
                run(xs)
        from torch_einshard import _native

        legs["einshard"](xs)
        kernel = _native.last_kernel()
        flush = _flush_buffer(dev)
        times = {name: {"warm_ms": [], "flushed_ms": []} for name in legs}
        for r in range(rounds):
            order = list(legs) if r % 2 == 0 else list(legs)[::-1]
            for name in order:
                times[name]["warm_ms"].append(round(_time_warm(legs[name], xs, dev, steps), 5))
                times[name]["flushed_ms"].append(round(_time_flushed(legs[name], xs, dev, steps, flush), 5))
        del flush
    finally:
        gc.enable()
    med = lambda v: sorted(v)[len(v) // 2]
    out = {
        "metric": "kernel ms per launch, this library against torch's GPU path, timed alternately",
        "workload": wl["workload"],
        "reference": vendor["workload"],
        "steps": steps,
        "rounds": rounds,
        "kernel": kernel,
    }
    for name, t in times.items():
        out[name] = dict(t, warm_ms_median=med(t["warm_ms"]), flushed_ms_median=med(t["flushed_ms"]))
    for mode in ("warm", "flushed"):
        out[f"ratio_{mode}"] = round(out["einshard"][f"{mode}_ms_median"] / out["vendor"][f"{mode}_ms_median"], 4)
    return out


def measure_cpu(wl, budget_s=12.0):
    """Time the oracle (reference CPU path) on a bounded sample (``cpu_sample``: the whole
    workload, for the contractions that take well under a second on the host; else the
    parity ``sample``); returns per-unit rate."""
    threads = min(len(os.sched_getaffinity(0)), int(os.environ.get("OMP_NUM_THREADS", "64") or 64))
    torch.set_num_threads(max(threads, 1))
    run = _cpu_runner(wl)
    sample, fraction = wl.get("cpu_sample", wl["sample"])(wl["host"])
    sample = [t.contiguous() for t in sample]
    t0 = time.perf_counter()
    run(sample)  # warm-up
    first = time.perf_counter() - t0
    iters = max(1, min(20, int(budget_s / max(first, 1e-3))))
    t0 = time.perf_counter()
    for _ in range(iters):
        run(sample)
    per = (time.perf_counter() - t0) / iters
    work = wl.get("flops", wl.get("bytes")) * fraction
    if "flops" in wl:
        value = work / per / 1e12
        unit = "TFLOP/s"
    else:
        value = work / per / 1e9
        unit = "GB/s"
    shape = " x ".join(str(list(t.shape)) for t in sample)
    return dict(
        value=round(value, 4),
        unit=unit,
        cores=torch.get_num_threads(),
        kind="port",
        sample=f"{shape} ({fraction:.4g} of the workload), {iters} timed iterations of {per * 1e3:.1f} ms",
    )


def _rel_error(actual, expected):
    """max |a - e| / max(max |e|, rms(e)): the parity tests' relative error."""
    a, e = actual.double(), expected.double()
    scale = max(e.abs().max().item(), e.pow(2).mean().sqrt().item(), 1e-30)
    return (a - e).abs().max().item() / scale


def measure_parity(es, wl, dev):
    """Errors on the CPU-baseline sample: the device result and the reference CPU
    path's result, each against the same computation in fp64 (copies: bit-exactness
    of the device result against the CPU path)."""
    sample, _ = wl["sample"](wl["host"])
    sample = [t.contiguous() for t in sample]
    cpu_out = _cpu_runner(wl)(sample)
    gpu_out = _runner(es, wl)([t.to(dev) for t in sample]).cpu()
    out = dict(sample=" x ".join(str(list(t.shape)) for t in sample))
    if wl.get("copy_only") or not cpu_out.is_floating_point():
        out["bitexact"] = bool(torch.equal(gpu_out.view(torch.uint8) if gpu_out.element_size() == 1 else gpu_out,
                                           cpu_out.view(torch.uint8) if cpu_out.element_size() == 1 else cpu_out))
        return out
    exact = _cpu_runner(wl)([t.double() for t in sample])
    out["gpu_vs_fp64"] = float(f"{_rel_error(gpu_out, exact):.3e}")
    out["cpu_vs_fp64"] = float(f"{_rel_error(cpu_out, exact):.3e}")
    out["gpu_vs_cpu"] = float(f"{_rel_error(gpu_out, cpu_out):.3e}")
    return out


def bench_one(es, key, dev, steps, warmup, cpu=True):
    wl = WORKLOADS[key](dev)
    g = measure_gpu(es, wl, dev, steps, warmup)
    ms_per_step = g["wall_s"] * 1e3 / steps
    work = wl["flops"] if "flops" in wl else wl["bytes"]
    scale, unit = (1e12, "TFLOP/s") if "flops" in wl else (1e9, "GB/s")
    value = work / (ms_per_step / 1e3) / scale
    # achieved / frac: each launch timed alone after a cache flush (cold operands);
    # *_warm: back-to-back launches with the operands resident in cache
    achieved = work / (g["cold_ms"] / 1e3) / scale
    achieved_warm = work / (g["kernel_ms"] / 1e3) / scale
    roofline = dict(
        bound=wl["bound"],
        achieved=round(achieved, 2),
        peak=wl["peak"],
        unit=unit,
        frac=round(achieved / wl["peak"], 4),
        traffic=_traffic(key),
        **_mfma(key),
        kernel=g["kernel"],
        kernel_ms=round(g["cold_ms"], 5),
        achieved_warm=round(achieved_warm, 2),
        frac_warm=round(achieved_warm / wl["peak"], 4),
        kernel_ms_warm=round(g["kernel_ms"], 5),
    )
    line = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": unit,
        "n_gpus": 1,
        "steps": steps,
        "warmup": warmup,
        "ms_per_step": round(ms_per_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": wl["dtype"],
        "data": f"synthetic (torch.Generator seed {SEED}, generated on CPU, copied to HBM)",
        "config": {"workload": wl["workload"], "device": torch.cuda.get_device_name(dev)},
        "roofline": roofline,
        "cpu_baseline": measure_cpu(wl) if cpu else None,
    }
    if cpu:
        line["parity"] = measure_parity(es, wl, dev)
    return line


def _profile_rows(name, key_cells):
    """Rows of a markdown table in profiles/<name> keyed by their first cell."""
    path = os.path.join(_REPO, "profiles", name)
    if not os.path.exists(path):
        return None, {}
    header, rows = None, {}
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if header is None and all(k in cells for k in key_cells):
            header = cells
        elif header is not None and len(cells) == len(header) and not cells[0].startswith("---"):
            rows[cells[0]] = cells
    return header, rows


def _mfma(key):
    """Clock (GHz) and MFMA utilisation of a contraction workload's kernel, measured with
    the rocprofv3 counters GRBM_GUI_ACTIVE and SQ_VALU_MFMA_BUSY_CYCLES (profiles/mfma.md)."""
    header, rows = _profile_rows("mfma.md", ("clock GHz", "MFMA util"))
    if key not in rows:
        return {}
    cells = rows[key]
    try:
        return {
            "clock_ghz": float(cells[header.index("clock GHz")]),
            "mfma_util": round(float(cells[header.index("MFMA util")].rstrip(" %")) / 100, 4),
        }
    except ValueError:
        return {}


def _traffic(key):
    """HBM bytes per launch of the workload's dominant kernel, measured with the
    rocprofv3 FETCH_SIZE / WRITE_SIZE counters (profiles/traffic.md), else None."""
    path = os.path.join(_REPO, "profiles", "traffic.md")
    if not os.path.exists(path):
        return None
    header = None
    for line in open(path):
        cells = [c.strip() for c in line.strip().strip("|").split("|")]
        if header is None and "bytes/launch" in cells:
            header = cells
        elif header is not None and len(cells) == len(header) and cells[0] == key:
            try:
                return int(cells[header.index("bytes/launch")])
            except ValueError:
                return None
    return None


def main(argv=None):
    parser = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    parser.add_argument("--gpus", type=int, default=1)
    parser.add_argument("--steps", type=int, default=50)
    parser.add_argument("--warmup", type=int, default=10)
    parser.add_argument("--workload", default="c4", choices=sorted(WORKLOADS) + ["all"])
    parser.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    parser.add_argument(
        "--vs-vendor",
        action="store_true",
        help="time the workload (c1, c2 or c4) and torch's GPU path on it alternately; one JSON line",
    )
    parser.add_argument("--rounds", type=int, default=6, help="alternations of --vs-vendor")
    args = parser.parse_args(argv)
    if args.gpus != 1:
        print(
            f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
            "(collectives across GPUs are not part of it)",
            file=sys.stderr,
        )
        return 2
    if not torch.cuda.is_available():
        print("bench.py: no ROCm device visible", file=sys.stderr)
        return 2
    import torch_einshard as es

    dev = torch.device("cuda:0")
    if args.vs_vendor:
        if f"vendor_{args.workload}" not in WORKLOADS:
            print(f"bench.py: --vs-vendor needs a workload with a vendor_ reference point, not {args.workload}",
                  file=sys.stderr)
            return 2
        line = measure_vs_vendor(es, args.workload, dev, args.steps, args.warmup, args.rounds)
        print(json.dumps(line), flush=True)
        return 0
    calibration = ("copy", "dma_calib") + tuple(k for k in WORKLOADS if k.startswith("vendor_"))
    keys = [k for k in sorted(WORKLOADS) if k not in calibration] if args.workload == "all" else [args.workload]
    for key in keys:
        line = bench_one(es, key, dev, args.steps, args.warmup, cpu=not args.no_cpu)
        print(json.dumps(line), flush=True)
        torch.cuda.empty_cache()
    return 0


if __name__ == "__main__":
    sys.exit(main())
