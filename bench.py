#!/usr/bin/env python
"""Benchmark of the quantized-dtype hot path on one MI355X.

One step = BASELINE config [2]: a cast sweep over 2^28 fp32 elements held in
HBM: fp32 -> fp16 -> fp32, fp32 -> bf16 -> fp32, and for E4M3 and E5M2 the
per-tensor quantization (the amax pass, then the scaled cast, which derives
the scale from the amax itself) and the scaled dequantization back to fp32.
`value` is the algorithmic bytes of the step (52 B/element) over its wall
time, in GB/s, timed with nothing but the ops on the stream.  A second pass of
the same steps brackets each op with HIP events on its stream, which gives
the per-kernel roofline figures.  Further
legs, each with its own roofline: the FP8-weight Linear of config [4]
(x 2048x4096, W 4096x4096 E4M3) and its backward in TFLOP/s, the FP4 pack / unpack of config
[3] and the two FP4-weight convolutions of config [5] in GB/s.  The CPU
baseline is the C oracle on a bounded sample of the same sweep.

Prints ONE JSON line.  Usage: python bench.py [--gpus 1] [--steps K] [--warmup W]
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
FP8_PEAK_TFLOPS = 5000.0
BF16_PEAK_TFLOPS = 2500.0
METRIC = "cast GB/s (% HBM peak) at 256M elems; FP8-weight Linear TFLOP/s at 4096^2"

# (op name, algorithmic bytes per element); the sequence of one step
SWEEP = [
    ("f32->f16", 6), ("f16->f32", 6), ("f32->bf16", 6), ("bf16->f32", 6),
    # novaq_quantize: the amax pass (4 B/element), then the scaled cast (5 B)
    # deriving s = amax / 448 (57344) itself and writing it out
    ("quantize f32->e4m3 (amax + scaled cast)", 9), ("e4m3->f32 scaled", 5),
    ("quantize f32->e5m2 (amax + scaled cast)", 9), ("e5m2->f32 scaled", 5),
]
BYTES_PER_ELEM = sum(b for _, b in SWEEP)
# kernel behind each single-kernel op (rocprofv3 names), for the measured traffic
KERNEL_OF = {
    "f32->f16": "cast_kernel<0, 1, 0>", "f16->f32": "cast_kernel<1, 0, 0>",
    "f32->bf16": "cast_kernel<0, 2, 0>", "bf16->f32": "cast_kernel<2, 0, 0>",
    "f32->e4m3 scaled": "cast_kernel<0, 3, 1>", "e4m3->f32 scaled": "cast_kernel<3, 0, 1>",
    "f32->e5m2 scaled": "cast_kernel<0, 4, 1>", "e5m2->f32 scaled": "cast_kernel<4, 0, 1>",
}
FP4_KERNEL = {"pack f32->e2m1": "cast_kernel<0, 5, 1>", "unpack e2m1->f32": "cast_kernel<5, 0, 1>"}
CONV_KERNEL = {1: "conv2d_smallc_kernel<5, 0, true, true>", 32: "conv2d_band_kernel<5, 0, 1, true>"}
TRAFFIC_FILE = os.path.join(ROOT, "profiles", "traffic.json")


def measured_traffic(kernel: str):
    """HBM bytes per launch of `kernel` from the committed rocprofv3 FETCH_SIZE /
    WRITE_SIZE summary (profiles/traffic.json, copy-calibrated), or None."""
    try:
        with open(TRAFFIC_FILE) as f:
            return json.load(f)["bytes_per_launch"].get(kernel)
    except (OSError, ValueError, KeyError):
        return None


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


def make_sweep(n: int, dev):
    """Device buffers and the list of (name, bytes/elem, launch fn) of a step."""
    import torch

    from novann_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev)
    g.manual_seed(2)
    x = torch.empty(n, dtype=torch.float32, device=dev)
    x.uniform_(-20.0, 20.0, generator=g)
    x.exp2_()
    u = torch.empty(n, dtype=torch.float32, device=dev).uniform_(generator=g)
    x.copysign_(u - 0.5)  # random sign
    del u
    y = torch.empty_like(x)
    h = torch.empty(n, dtype=torch.int16, device=dev)
    q = torch.empty(n, dtype=torch.uint8, device=dev)
    amax_scale = torch.zeros(4, dtype=torch.float32, device=dev)  # (amax, s) per FP8 format
    stream = torch.cuda.current_stream(dev).cuda_stream
    P = lambda t: t.data_ptr()  # noqa: E731

    def cast(src, st, dst, dt, sc=None):
        return lambda: _lib.check(lib.novaq_cast(P(src), st, P(dst), dt, n, sc, stream), "cast")

    ops = [
        cast(x, 0, h, 1), cast(h, 1, y, 0), cast(x, 0, h, 2), cast(h, 2, y, 0),
    ]
    for k, dt in enumerate((3, 4)):
        as_ptr = P(amax_scale) + 8 * k
        ops += [
            lambda as_ptr=as_ptr, dt=dt: _lib.check(
                lib.novaq_quantize(P(x), 0, P(q), dt, n, as_ptr, stream), "quantize"),
            cast(q, dt, y, 0, as_ptr + 4),
        ]
    return [(name, b, fn) for (name, b), fn in zip(SWEEP, ops)], (x, y, h, q, amax_scale)


def bench_sweep(n: int, steps: int, warmup: int, dev):
    import torch
    ops, bufs = make_sweep(n, dev)
    for _ in range(warmup):
        for _, _, fn in ops:
            fn()
    torch.cuda.synchronize(dev)
    # the timed steps: the ops back to back, nothing else on the stream
    t0 = time.perf_counter()
    for s in range(steps):
        for _, _, fn in ops:
            fn()
    torch.cuda.synchronize(dev)
    t1 = time.perf_counter()
    # then, as diagnostics, the same number of steps with events around each op
    events = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
               for _ in ops] for _ in range(steps)]
    for s in range(steps):
        for (_, _, fn), (e0, e1) in zip(ops, events[s]):
            e0.record()
            fn()
            e1.record()
    torch.cuda.synchronize(dev)
    per_op = []
    for i, (name, b, _) in enumerate(ops):
        t = [events[s][i][0].elapsed_time(events[s][i][1]) for s in range(steps)]
        ms = sum(t) / steps
        gbs = b * n / (ms * 1e-3) / 1e9 if b else None
        per_op.append({"op": name, "ms": round(ms, 4), "median_ms": round(_median(t), 4),
                       "GB/s": None if gbs is None else round(gbs, 1),
                       "frac": None if gbs is None else round(gbs / HBM_PEAK_GBS, 4)})
    # after the timed steps, each op again with the MALL evicted before every
    # launch (its inputs then come from HBM, not from the op just before)
    flush = torch.zeros(1 << 27, dtype=torch.float32, device=dev)
    for p, (_, b, fn) in zip(per_op, ops):
        if not b:
            continue
        mean, med = _time_launches(dev, fn, max(steps, 5), 0, flush)
        p["evicted_median_ms"] = round(med, 4)
        p["evicted_GB/s"] = round(b * n / (med * 1e-3) / 1e9, 1)
    # context for the HBM roofline: the vendor's own conversion kernels (torch
    # copy_ between dtypes) on the same buffers, timed the same way
    x, y = bufs[0], bufs[1]
    h16 = {torch.float16: bufs[2].view(torch.float16), torch.bfloat16: bufs[2].view(torch.bfloat16)}
    vendor = {}
    for name, dt in (("f16", torch.float16), ("bf16", torch.bfloat16)):
        for label, fn in ((f"f32->{name}", lambda dt=dt: h16[dt].copy_(x)),
                          (f"{name}->f32", lambda dt=dt: y.copy_(h16[dt]))):
            med = _time_launches(dev, fn, max(steps, 5), 1, flush)[1]
            gbs = 6 * n / (med * 1e-3) / 1e9
            vendor[label] = {"evicted_median_ms": round(med, 4), "GB/s": round(gbs, 1),
                             "frac": round(gbs / HBM_PEAK_GBS, 4)}
    del bufs, flush, x, y, h16
    return (t1 - t0) * 1e3 / steps, per_op, vendor


def bench_linear(dev, iters: int = 20, warmup: int = 5):
    """Config [4]: y = x W^T + b, x (2048, 4096) fp32, W (4096, 4096) E4M3."""
    import torch

    from novann_amd import _lib, quant
    lib = _lib.load()
    M, K, N = 2048, 4096, 4096
    g = torch.Generator(device=dev)
    g.manual_seed(4)
    x = torch.randn((M, K), generator=g, device=dev, dtype=torch.float32)
    w = torch.randn((N, K), generator=g, device=dev, dtype=torch.float32) * (2.0 / K) ** 0.5
    wq = quant.quantize(w, "e4m3")
    b = torch.zeros(N, dtype=torch.float32, device=dev)
    y = torch.empty((M, N), dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def run():
        _lib.check(lib.novaq_linear_forward(x.data_ptr(), M, K, wq.data.data_ptr(), 3,
                                            wq.scale.data_ptr(), b.data_ptr(), N, y.data_ptr(),
                                            stream), "linear")
    try:
        run()
    except NotImplementedError:
        return None
    ms, med = _time_launches(dev, run, iters, warmup)
    # the same launches with the MALL evicted before each (x and W, 48 MB, are
    # otherwise still cached from the launch before)
    flush = torch.zeros(1 << 27, dtype=torch.float32, device=dev)
    _, emed = _time_launches(dev, run, iters, 0, flush)
    del flush
    flops = 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    # context: the vendor bf16 GEMM (torch -> hipBLASLt) on the same shape with
    # bf16 operands already in HBM (no fp32 x conversion, no W decode)
    xb, wb = x.to(torch.bfloat16), w.to(torch.bfloat16).contiguous()
    vms, _ = _time_launches(dev, lambda: torch.nn.functional.linear(xb, wb), iters, warmup)
    # the same product on x stored as E4M3 (amax-scaled, as a fused epilogue
    # writes activations): both operands' codes go to the FP8 MFMA
    xq = quant.quantize(x, "e4m3")

    def run8():
        _lib.check(lib.novaq_linear_forward_ex(
            xq.data.data_ptr(), _lib.E4M3, xq.scale.data_ptr(), M, K, wq.data.data_ptr(), 3,
            wq.scale.data_ptr(), b.data_ptr(), N, None, y.data_ptr(), stream), "linear fp8 x")
    ms8, _ = _time_launches(dev, run8, iters, warmup)
    tf8 = flops / (ms8 * 1e-3) / 1e12
    # x stored as bf16 (as a fused epilogue writes activations), and config
    # [4]'s fp32 x cast to bf16 by a separate launch first (both timed)
    x16 = torch.empty((M, K), dtype=torch.bfloat16, device=dev)

    def cast16():
        _lib.check(lib.novaq_cast(x.data_ptr(), _lib.F32, x16.data_ptr(), _lib.BF16, M * K, None,
                                  stream), "cast")

    def run16():
        _lib.check(lib.novaq_linear_forward_ex(
            x16.data_ptr(), _lib.BF16, None, M, K, wq.data.data_ptr(), 3, wq.scale.data_ptr(),
            b.data_ptr(), N, None, y.data_ptr(), stream), "linear bf16 x")
    cast16()
    ms16, _ = _time_launches(dev, run16, iters, warmup)
    mscast, _ = _time_launches(dev, lambda: (cast16(), run16()), iters, warmup)
    return {"metric": "FP8-weight Linear TFLOP/s at 4096^2", "value": round(tflops, 1),
            "unit": "TFLOP/s", "ms": round(ms, 4), "median_ms": round(med, 4),
            "evicted_median_ms": round(emed, 4),
            "vendor_bf16_gemm": {"what": "torch.nn.functional.linear, bf16 x and W in HBM",
                                 "ms": round(vms, 4),
                                 "TFLOP/s": round(flops / (vms * 1e-3) / 1e12, 1)},
            "e4m3_x": {"what": "config [4] with x stored as E4M3 (amax-scaled): "
                               "linear_f8_kernel, both operands on the FP8 MFMA",
                       "ms": round(ms8, 4), "TFLOP/s": round(tf8, 1),
                       "frac_bf16_peak": round(tf8 / BF16_PEAK_TFLOPS, 4),
                       "frac_fp8_peak": round(tf8 / FP8_PEAK_TFLOPS, 4),
                       "traffic": measured_traffic("linear_f8_kernel<3, 3>")},
            "bf16_x": {"what": "x stored as bf16 (a fused epilogue's output): "
                               "linear_pingpong_kernel<3, 2>, 16-byte x loads",
                       "ms": round(ms16, 4), "TFLOP/s": round(flops / (ms16 * 1e-3) / 1e12, 1)},
            "cast_then_bf16_x": {"what": "config [4]'s fp32 x cast to bf16 by novaq_cast, then "
                                         "the bf16-x product (both launches timed)",
                                 "ms": round(mscast, 4),
                                 "TFLOP/s": round(flops / (mscast * 1e-3) / 1e12, 1)},
            "config": {"workload": "BASELINE config [4]", "M": M, "K": K, "N": N,
                       "w_dtype": "e4m3", "mfma": "bf16"},
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / BF16_PEAK_TFLOPS, 4),
                         "traffic": measured_traffic("linear_pingpong_kernel<3, 0, false>")}}


def bench_linear_backward(dev, iters: int = 10, warmup: int = 3):
    """Linear.backward at config [4]'s shape (linear.py:85-108): grad_input
    = grad @ (s * dec(W)), grad_weight = grad^T @ x, grad_bias = column sums,
    E4M3 W; 2 x 68.72 GFLOP per call, all kernels (transposes included) timed."""
    import torch

    from novann_amd import _lib, quant
    lib = _lib.load()
    M, K, N = 2048, 4096, 4096  # batch, D_in, D_out
    g = torch.Generator(device=dev)
    g.manual_seed(6)
    x = torch.randn((M, K), generator=g, device=dev, dtype=torch.float32)
    w = torch.randn((N, K), generator=g, device=dev, dtype=torch.float32) * (2.0 / K) ** 0.5
    wq = quant.quantize(w, "e4m3")
    grad = torch.randn((M, N), generator=g, device=dev, dtype=torch.float32)
    gi = torch.empty((M, K), device=dev)
    gw = torch.empty((N, K), device=dev)
    gb = torch.empty(N, device=dev)
    nbytes = lib.novaq_linear_backward_workspace(M, K, N, 3)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def run():
        _lib.check(lib.novaq_linear_backward(
            grad.data_ptr(), x.data_ptr(), M, K, wq.data.data_ptr(), 3, wq.scale.data_ptr(), N,
            gi.data_ptr(), gw.data_ptr(), gb.data_ptr(), ws.data_ptr(), nbytes, stream),
            "linear backward")
    for _ in range(warmup):
        run()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize(dev)
    e0.record()
    for _ in range(iters):
        run()
    e1.record()
    torch.cuda.synchronize(dev)
    ms = e0.elapsed_time(e1) / iters
    flush = torch.zeros(1 << 27, dtype=torch.float32, device=dev)
    _, emed = _time_launches(dev, run, iters, 0, flush)  # MALL evicted before each call
    del flush
    flops = 2 * 2.0 * M * N * K
    tflops = flops / (ms * 1e-3) / 1e12
    return {"metric": "Linear backward TFLOP/s (grad_input + grad_weight) at config [4]",
            "value": round(tflops, 1), "unit": "TFLOP/s", "ms": round(ms, 4),
            "evicted_median_ms": round(emed, 4),
            "workspace_bytes": nbytes,
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1),
                         "peak": BF16_PEAK_TFLOPS, "unit": "TFLOP/s",
                         "frac": round(tflops / BF16_PEAK_TFLOPS, 4)}}


def bench_fp4(dev, n: int = 1 << 26, iters: int = 20, warmup: int = 3):
    """Config [3]: fp32 -> E2M1 pack and E2M1 -> fp32 unpack of 2^26 N(0,1)
    elements with the per-tensor scale s = amax / 6 (4.5 algorithmic bytes per
    element each way).  The 256 MiB input is at the MALL's size, so a 512 MiB
    read evicts it before every timed launch."""
    import torch

    from novann_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev)
    g.manual_seed(3)
    x = torch.randn(n, generator=g, device=dev, dtype=torch.float32)
    packed = torch.empty((n + 1) // 2, dtype=torch.uint8, device=dev)
    y = torch.empty_like(x)
    amax_scale = torch.empty(2, dtype=torch.float32, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    _lib.check(lib.novaq_amax(x.data_ptr(), 0, n, amax_scale.data_ptr(), stream), "amax")
    s_ptr = amax_scale.data_ptr() + 4
    _lib.check(lib.novaq_scale_from_amax(amax_scale.data_ptr(), 5, s_ptr, stream), "scale")
    ops = {
        "pack f32->e2m1": lambda: _lib.check(
            lib.novaq_pack_fp4(x.data_ptr(), n, s_ptr, packed.data_ptr(), stream), "pack"),
        "unpack e2m1->f32": lambda: _lib.check(
            lib.novaq_unpack_fp4(packed.data_ptr(), n, s_ptr, y.data_ptr(), stream), "unpack"),
    }
    flush = torch.zeros(1 << 27, dtype=torch.float32, device=dev)
    out = []
    for name, fn in ops.items():
        for _ in range(warmup):
            fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(iters)]
        torch.cuda.synchronize(dev)
        for e0, e1 in ev:
            _evict(flush)
            e0.record()
            fn()
            e1.record()
        torch.cuda.synchronize(dev)
        ms = sum(e0.elapsed_time(e1) for e0, e1 in ev) / iters
        gbs = 4.5 * n / (ms * 1e-3) / 1e9
        out.append({"op": name, "ms": round(ms, 4), "GB/s": round(gbs, 1),
                    "frac": round(gbs / HBM_PEAK_GBS, 4),
                    "traffic": measured_traffic(FP4_KERNEL[name]) if n == 1 << 26 else None})
    return {"workload": "BASELINE config [3]", "elements": n, "bytes_per_element": 4.5,
            "kernels": out}


def bench_conv(dev, iters: int = 20, warmup: int = 5):
    """Config [5]: MNIST-shaped conv1 (1->32) and conv2 (32->64), 3x3/s1/p1,
    E2M1 weights; HBM-bound, so reported as GB/s of algorithmic traffic
    (read x once, write y once)."""
    import torch

    from novann_amd import _lib, quant
    lib = _lib.load()
    g = torch.Generator(device=dev)
    g.manual_seed(5)
    N = 256
    x = torch.rand((N, 1, 28, 28), generator=g, device=dev, dtype=torch.float32)
    layers = []
    for cin, cout in ((1, 32), (32, 64)):
        w = torch.randn((cout, cin, 3, 3), generator=g, device=dev) * (2.0 / (cin * 9)) ** 0.5
        layers.append((cin, cout, quant.quantize(w.contiguous(), "e2m1")))
    y1 = torch.empty((N, 32, 28, 28), device=dev)
    y2 = torch.empty((N, 64, 28, 28), device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream

    def conv(src, dst, cin, cout, q):
        _lib.check(lib.novaq_conv2d_forward(src.data_ptr(), N, cin, 28, 28, q.data.data_ptr(), 5,
                                            q.scale.data_ptr(), cout, 3, 3, 1, 1, 1, 1, 0, None,
                                            dst.data_ptr(), stream), "conv2d")
    runs = [(x, y1) + layers[0], (y1, y2) + layers[1]]
    # a 512 MiB read between timed launches evicts the 256 MB MALL, so every
    # launch reads its input from HBM (the working sets would otherwise fit)
    flush = torch.zeros(1 << 27, dtype=torch.float32, device=dev)
    out = []
    for src, dst, cin, cout, q in runs:
        for _ in range(warmup):
            conv(src, dst, cin, cout, q)
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(iters)]
        torch.cuda.synchronize(dev)
        for e0, e1 in ev:
            _evict(flush)
            e0.record()
            conv(src, dst, cin, cout, q)
            e1.record()
        torch.cuda.synchronize(dev)
        ms = sum(e0.elapsed_time(e1) for e0, e1 in ev) / iters
        nbytes = (src.numel() + dst.numel()) * 4
        gbs = nbytes / (ms * 1e-3) / 1e9
        flops = 2.0 * N * 28 * 28 * cout * cin * 9
        out.append({"layer": f"conv {cin}->{cout}", "ms": round(ms, 4), "GB/s": round(gbs, 1),
                    "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                    "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2), "bytes": nbytes,
                    "traffic": measured_traffic(CONV_KERNEL[cin])})
    return {"workload": "BASELINE config [5]", "layers": out}


def bench_conv_backward(dev, iters: int = 20, warmup: int = 5):
    """Conv2d.backward (conv2d.py:179-207) for config [5]'s two layers, E2M1
    weights, all three gradients per call.  Algorithmic traffic: read grad
    twice (grad_input and grad_weight each need all of it) and x once, write
    grad_input once; the weight-sized arrays are negligible."""
    import torch

    from novann_amd import _lib, quant
    lib = _lib.load()
    g = torch.Generator(device=dev)
    g.manual_seed(7)
    N = 256
    stream = torch.cuda.current_stream(dev).cuda_stream
    flush = torch.zeros(1 << 27, dtype=torch.float32, device=dev)
    out = []
    for cin, cout in ((1, 32), (32, 64)):
        x = torch.rand((N, cin, 28, 28), generator=g, device=dev, dtype=torch.float32)
        w = torch.randn((cout, cin, 3, 3), generator=g, device=dev) * (2.0 / (cin * 9)) ** 0.5
        q = quant.quantize(w.contiguous(), "e2m1")
        grad = torch.randn((N, cout, 28, 28), generator=g, device=dev, dtype=torch.float32)
        gi = torch.empty_like(x)
        gw = torch.empty((cout, cin, 3, 3), device=dev)
        gb = torch.empty((cout, 1), device=dev)
        nbytes = lib.novaq_conv2d_backward_workspace(N, cin, cout, 3, 3, 5)
        ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)

        def run():
            _lib.check(lib.novaq_conv2d_backward(
                grad.data_ptr(), x.data_ptr(), N, cin, 28, 28, q.data.data_ptr(), 5,
                q.scale.data_ptr(), cout, 3, 3, 1, 1, 1, 1, 0, gi.data_ptr(), gw.data_ptr(),
                gb.data_ptr(), ws.data_ptr(), nbytes, stream), "conv2d backward")
        for _ in range(warmup):
            run()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(iters)]
        torch.cuda.synchronize(dev)
        for e0, e1 in ev:
            _evict(flush)
            e0.record()
            run()
            e1.record()
        torch.cuda.synchronize(dev)
        ms = sum(e0.elapsed_time(e1) for e0, e1 in ev) / iters
        nb = (2 * grad.numel() + 2 * x.numel()) * 4
        gbs = nb / (ms * 1e-3) / 1e9
        flops = 2 * 2.0 * N * 28 * 28 * cout * cin * 9
        out.append({"layer": f"conv {cin}->{cout} backward", "ms": round(ms, 4),
                    "GB/s": round(gbs, 1), "frac_hbm": round(gbs / HBM_PEAK_GBS, 4),
                    "TFLOP/s": round(flops / (ms * 1e-3) / 1e12, 2), "bytes": nb,
                    "workspace_bytes": nbytes})
        del x, grad, gi, ws
    return {"workload": "BASELINE config [5] shapes, backward", "layers": out}


def bench_epilogue(dev, iters: int = 20, warmup: int = 5):
    """Fused epilogues (eval BatchNorm + ReLU + bf16 store) on config [5]'s
    conv2 and config [4]'s Linear, each reading its input as the bf16 a
    previous fused layer stores; beside them the unfused equivalent of the
    same layer: the fp32-input product with an fp32 output, then a separate
    fp32 -> bf16 cast of y (the HBM round trip the fusion removes; the
    BatchNorm and ReLU would cost another such pass).  A 512 MiB read evicts
    the MALL before every timed launch."""
    import ctypes

    import torch

    from novann_amd import _lib, quant
    lib = _lib.load()
    g = torch.Generator(device=dev)
    g.manual_seed(8)
    stream = torch.cuda.current_stream(dev).cuda_stream
    flush = torch.zeros(1 << 27, dtype=torch.float32, device=dev)

    def timed(fn):
        for _ in range(warmup):
            fn()
        ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
              for _ in range(iters)]
        torch.cuda.synchronize(dev)
        for e0, e1 in ev:
            _evict(flush)
            e0.record()
            fn()
            e1.record()
        torch.cuda.synchronize(dev)
        return sum(e0.elapsed_time(e1) for e0, e1 in ev) / iters

    def bn_epilogue(C, out_dtype):
        mul = (torch.rand(C, generator=g, device=dev) + 0.5).contiguous()
        add = (torch.randn(C, generator=g, device=dev) * 0.1).contiguous()
        return _lib.Epilogue(mul.data_ptr(), add.data_ptr(), None, None, 1,
                             _lib.DTYPES[out_dtype]), (mul, add)

    out = {}
    # conv2 of config [5]: (256, 32, 28, 28) -> (256, 64, 28, 28), 3x3/s1/p1, E2M1
    N, C, Co, H = 256, 32, 64, 28
    x32 = torch.rand((N, C, H, H), generator=g, device=dev)
    x16 = x32.to(torch.bfloat16)
    w = torch.randn((Co, C, 3, 3), generator=g, device=dev) * (2.0 / (C * 9)) ** 0.5
    q = quant.quantize(w.contiguous(), "e2m1")
    y16 = torch.empty((N, Co, H, H), dtype=torch.bfloat16, device=dev)
    y32 = torch.empty((N, Co, H, H), dtype=torch.float32, device=dev)
    ep, keep = bn_epilogue(Co, "bf16")

    def conv_fused():
        _lib.check(lib.novaq_conv2d_forward_ex(
            x16.data_ptr(), _lib.BF16, None, N, C, H, H, q.data.data_ptr(), _lib.E2M1,
            q.scale.data_ptr(), Co, 3, 3, 1, 1, 1, 1, 0, None, ctypes.byref(ep), y16.data_ptr(),
            stream), "conv2d fused")

    def conv_unfused():
        _lib.check(lib.novaq_conv2d_forward(x32.data_ptr(), N, C, H, H, q.data.data_ptr(),
                                            _lib.E2M1, q.scale.data_ptr(), Co, 3, 3, 1, 1, 1,
                                            1, 0, None, y32.data_ptr(), stream), "conv2d")
        _lib.check(lib.novaq_cast(y32.data_ptr(), _lib.F32, y16.data_ptr(), _lib.BF16,
                                  y32.numel(), None, stream), "cast")
    ms_f, ms_u = timed(conv_fused), timed(conv_unfused)
    nb = (x16.numel() + y16.numel()) * 2
    out["conv2"] = {"layer": "conv 32->64 + BN + ReLU, bf16 in / bf16 out",
                    "ms": round(ms_f, 4), "GB/s": round(nb / (ms_f * 1e-3) / 1e9, 1),
                    "frac_hbm": round(nb / (ms_f * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": nb,
                    "unfused_ms": round(ms_u, 4),
                    "unfused": "fp32 conv (fp32 in / out) + fp32->bf16 cast of y"}
    del x32, x16, y16, y32
    # Linear of config [4]: x (2048, 4096) bf16, W (4096, 4096) E4M3
    M_, K, Nn = 2048, 4096, 4096
    x32 = torch.randn((M_, K), generator=g, device=dev)
    x16 = x32.to(torch.bfloat16)
    w = torch.randn((Nn, K), generator=g, device=dev) * (2.0 / K) ** 0.5
    wq = quant.quantize(w, "e4m3")
    y16 = torch.empty((M_, Nn), dtype=torch.bfloat16, device=dev)
    y32 = torch.empty((M_, Nn), dtype=torch.float32, device=dev)
    ep2, keep2 = bn_epilogue(Nn, "bf16")

    def lin_fused():
        _lib.check(lib.novaq_linear_forward_ex(
            x16.data_ptr(), _lib.BF16, None, M_, K, wq.data.data_ptr(), _lib.E4M3,
            wq.scale.data_ptr(), None, Nn, ctypes.byref(ep2), y16.data_ptr(), stream),
            "linear fused")

    def lin_unfused():
        _lib.check(lib.novaq_linear_forward(x32.data_ptr(), M_, K, wq.data.data_ptr(), _lib.E4M3,
                                            wq.scale.data_ptr(), None, Nn, y32.data_ptr(),
                                            stream), "linear")
        _lib.check(lib.novaq_cast(y32.data_ptr(), _lib.F32, y16.data_ptr(), _lib.BF16,
                                  y32.numel(), None, stream), "cast")
    ms_f, ms_u = timed(lin_fused), timed(lin_unfused)
    tf = 2.0 * M_ * Nn * K / (ms_f * 1e-3) / 1e12
    out["linear"] = {"layer": "Linear 4096x4096 E4M3 + BN1d + ReLU, bf16 in / bf16 out",
                     "ms": round(ms_f, 4), "TFLOP/s": round(tf, 1),
                     "frac_mfma": round(tf / BF16_PEAK_TFLOPS, 4), "unfused_ms": round(ms_u, 4),
                     "unfused": "fp32-input Linear (fp32 y) + fp32->bf16 cast of y"}
    return {"workload": "BASELINE configs [5] (conv2) and [4] with fused epilogues", **out}


def _evict(buf):
    """Evict the MALL (256 MB) and the L2s by reading a 512 MiB buffer: the
    caches then hold its clean lines, so the timed kernel reads its inputs
    from HBM without paying for an unrelated buffer's write-back (a 512 MiB
    write before each launch left 256 MB of dirty lines to drain during it)."""
    buf.amax()


def _median(v):
    s = sorted(v)
    k = len(s) // 2
    return s[k] if len(s) % 2 else 0.5 * (s[k - 1] + s[k])


def _time_launches(dev, fn, iters, warmup, flush=None):
    """(mean, median) ms of fn over `iters` launches, each bracketed by HIP
    events on the current stream (the one every entry point here is given);
    with `flush`, the MALL is evicted before each launch, outside the events."""
    import torch
    for _ in range(warmup):
        fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
          for _ in range(iters)]
    torch.cuda.synchronize(dev)
    for e0, e1 in ev:
        if flush is not None:
            _evict(flush)
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize(dev)
    t = [e0.elapsed_time(e1) for e0, e1 in ev]
    return sum(t) / len(t), _median(t)


def _timed_flush(dev, fn, iters, warmup):
    """Average ms of fn over iters launches, the MALL evicted before each."""
    import torch
    flush = torch.zeros(1 << 27, dtype=torch.float32, device=dev)
    return _time_launches(dev, fn, iters, warmup, flush)[0]


def bench_optim(dev, iters: int = 20, warmup: int = 3):
    """AdamW (adamw.py:41-65) on config [4]'s 4096 x 4096 weight: the fp32
    step alone (28 algorithmic bytes per element: w, g, m, v read, w, m, v
    written) and the step with re-quantization to E4M3 (+ 4 B read and 1 B
    written by the amax-scaled cast)."""
    import ctypes

    import torch

    from novann_amd import _lib
    lib = _lib.load()
    n = 4096 * 4096
    g = torch.Generator(device=dev)
    g.manual_seed(9)
    w = torch.randn(n, generator=g, device=dev) * 0.02
    grad = torch.randn(n, generator=g, device=dev)
    m = torch.zeros(n, device=dev)
    v = torch.zeros(n, device=dev)
    codes = torch.empty(n, dtype=torch.uint8, device=dev)
    st = torch.empty(2, device=dev)
    stream = torch.cuda.current_stream(dev).cuda_stream
    hp = _lib.AdamW(1e-3, 0.9, 0.999, 1e-8, 1e-2, 1, 1)

    def step():
        hp.step += 1
        _lib.check(lib.novaq_adamw_step(w.data_ptr(), grad.data_ptr(), m.data_ptr(),
                                        v.data_ptr(), n, ctypes.byref(hp), None, stream), "adamw")

    def requant():
        hp.step += 1
        _lib.check(lib.novaq_adamw_requantize(w.data_ptr(), grad.data_ptr(), m.data_ptr(),
                                              v.data_ptr(), n, ctypes.byref(hp),
                                              codes.data_ptr(), _lib.E4M3, st.data_ptr(),
                                              stream), "adamw requantize")
    ms_s = _timed_flush(dev, step, iters, warmup)
    ms_r = _timed_flush(dev, requant, iters, warmup)
    gs = 28.0 * n / (ms_s * 1e-3) / 1e9
    gr = 33.0 * n / (ms_r * 1e-3) / 1e9
    return {"workload": "AdamW on BASELINE config [4]'s 4096x4096 weight", "elements": n,
            "step": {"ms": round(ms_s, 4), "GB/s": round(gs, 1),
                     "frac": round(gs / HBM_PEAK_GBS, 4), "bytes_per_element": 28},
            "step_requantize_e4m3": {"ms": round(ms_r, 4), "GB/s": round(gr, 1),
                                     "frac": round(gr / HBM_PEAK_GBS, 4),
                                     "bytes_per_element": 33}}


def bench_pool(dev, iters: int = 20, warmup: int = 3):
    """MaxPool2d(2, 2) and GlobalAvgPool2d on a config [5]-sized activation
    (256, 64, 28, 28) in fp32 and bf16, and GlobalAvgPool2d on main.py's 7x7
    map at batch 256: algorithmic bytes = read x once + write y once; their
    backward passes on the same activation: read x (MaxPool2d) and the output
    gradient once, write the fp32 input gradient once."""
    import torch

    from novann_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev)
    g.manual_seed(10)
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = []
    x32 = torch.randn((256, 64, 28, 28), generator=g, device=dev)
    for name, x, dt in (("f32", x32, _lib.F32), ("bf16", x32.to(torch.bfloat16), _lib.BF16)):
        y = torch.empty((256, 64, 14, 14), dtype=x.dtype, device=dev)
        fn = lambda x=x, y=y, dt=dt: _lib.check(lib.novaq_max_pool2d(  # noqa: E731
            x.data_ptr(), dt, 256, 64, 28, 28, 2, 2, 2, 2, 0, 0, 0, y.data_ptr(), stream),
            "max_pool2d")
        ms = _timed_flush(dev, fn, iters, warmup)
        nb = (x.numel() + y.numel()) * x.element_size()
        out.append({"op": f"max_pool2d 2x2/2 (256,64,28,28) {name}", "ms": round(ms, 4),
                    "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                    "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    for shape in ((256, 64, 28, 28), (256, 64, 7, 7)):
        x = torch.randn(shape, generator=g, device=dev)
        y = torch.empty(shape[:2], device=dev)
        fn = lambda x=x, y=y, s=shape: _lib.check(lib.novaq_global_avg_pool2d(  # noqa: E731
            x.data_ptr(), _lib.F32, None, *s, y.data_ptr(), stream), "avg_pool2d")
        ms = _timed_flush(dev, fn, iters, warmup)
        nb = (x.numel() + y.numel()) * 4
        out.append({"op": f"global_avg_pool2d {shape} f32", "ms": round(ms, 4),
                    "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                    "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    # backward passes on the same activation: MaxPool2d(2, 2) reads x and the
    # (256, 64, 14, 14) grad and writes the fp32 input gradient; GlobalAvgPool2d
    # reads the (256, 64) grad and writes the input gradient
    gy = torch.randn((256, 64, 14, 14), generator=g, device=dev)
    for name, x, dt in (("f32", x32, _lib.F32), ("bf16", x32.to(torch.bfloat16), _lib.BF16)):
        gi = torch.empty((256, 64, 28, 28), device=dev)
        fn = lambda x=x, gi=gi, dt=dt: _lib.check(lib.novaq_max_pool2d_backward(  # noqa: E731
            gy.data_ptr(), x.data_ptr(), dt, 256, 64, 28, 28, 2, 2, 2, 2, 0, 0, 0,
            gi.data_ptr(), stream), "max_pool2d_backward")
        ms = _timed_flush(dev, fn, iters, warmup)
        nb = x.numel() * x.element_size() + gy.numel() * 4 + gi.numel() * 4
        out.append({"op": f"max_pool2d_backward 2x2/2 (256,64,28,28) x {name}",
                    "ms": round(ms, 4), "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                    "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    gp = torch.randn((256, 64), generator=g, device=dev)
    gi = torch.empty((256, 64, 28, 28), device=dev)
    fn = lambda: _lib.check(lib.novaq_global_avg_pool2d_backward(  # noqa: E731
        gp.data_ptr(), 256, 64, 28, 28, gi.data_ptr(), stream), "avg_pool2d_backward")
    ms = _timed_flush(dev, fn, iters, warmup)
    nb = (gp.numel() + gi.numel()) * 4
    out.append({"op": "global_avg_pool2d_backward (256, 64, 28, 28) f32", "ms": round(ms, 4),
                "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4)})
    return {"workload": "pools on config [5]-sized and main.py activations (forward and backward)",
            "kernels": out}


def bench_extras(dev, iters: int = 20, warmup: int = 3):
    """The arrays conv2d / max_pool2d return with extras=True, materialised on
    the device: the column matrix of config [5]'s conv2 (x (256, 32, 28, 28)
    fp32, col 288 x 200704 fp32 = 231 MB) and the padded copy behind the
    pooling window view of a (256, 64, 28, 28) activation padded by 1.
    Algorithmic bytes: read x once, write the output once; the MALL is evicted
    before each launch."""
    import torch

    from novann_amd import _lib
    lib = _lib.load()
    g = torch.Generator(device=dev)
    g.manual_seed(12)
    stream = torch.cuda.current_stream(dev).cuda_stream
    out = []
    x = torch.randn((256, 32, 28, 28), generator=g, device=dev)
    col = torch.empty((288, 256 * 28 * 28), device=dev)
    fn = lambda: _lib.check(lib.novaq_im2col(  # noqa: E731
        x.data_ptr(), _lib.F32, None, 256, 32, 28, 28, 3, 3, 1, 1, 1, 1, 0, col.data_ptr(),
        stream), "im2col")
    ms = _timed_flush(dev, fn, iters, warmup)
    nb = (x.numel() + col.numel()) * 4
    out.append({"op": "im2col config [5] conv2 (col 288 x 200704 fp32)", "ms": round(ms, 4),
                "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": nb})
    del col
    x = torch.randn((256, 64, 28, 28), generator=g, device=dev)
    xp = torch.empty((256, 64, 30, 30), device=dev)
    fn = lambda: _lib.check(lib.novaq_pad2d(  # noqa: E731
        x.data_ptr(), _lib.F32, 256, 64, 28, 28, 1, 1, 0, xp.data_ptr(), stream), "pad2d")
    ms = _timed_flush(dev, fn, iters, warmup)
    nb = (x.numel() + xp.numel()) * 4
    out.append({"op": "pad2d (256,64,28,28) -> (256,64,30,30) f32", "ms": round(ms, 4),
                "GB/s": round(nb / (ms * 1e-3) / 1e9, 1),
                "frac": round(nb / (ms * 1e-3) / 1e9 / HBM_PEAK_GBS, 4), "bytes": nb})
    return {"workload": "extras=True arrays of conv2d / max_pool2d", "kernels": out}


def cpu_baseline(sample: int, min_seconds: float = 10.0):
    """The C oracle running the same sweep on a bounded sample (all host cores)."""
    import numpy as np

    import oracle as O
    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count() or 1
    rng = np.random.default_rng(2)
    x = (np.exp2(rng.uniform(-20, 20, sample)) * np.where(rng.random(sample) < 0.5, -1, 1)
         ).astype(np.float32)
    # whole sweeps over the sample until about min_seconds of CPU work are done
    passes = 0
    t0 = time.perf_counter()
    while True:
        for st in (O.F16, O.BF16):
            O.cast(O.cast(x, O.F32, st, nthreads=threads), st, O.F32, n=sample, nthreads=threads)
        for dt in (O.E4M3, O.E5M2):
            s = O.scale_from_amax(O.amax(x, nthreads=threads), dt)
            q = O.cast(x, O.F32, dt, scale=s, nthreads=threads)
            O.cast(q, dt, O.F32, n=sample, scale=s, nthreads=threads)
        passes += 1
        dt_s = time.perf_counter() - t0
        if dt_s >= min_seconds:
            break
    return {"value": round(BYTES_PER_ELEM * sample * passes / dt_s / 1e9, 3), "unit": "GB/s",
            "cores": threads, "kind": "port",
            "sample": f"config [2] sweep (52 B/element) repeated {passes}x on {sample >> 20}M "
                      f"elements, C oracle, {threads} OpenMP threads, {dt_s:.1f} s"}


def _cpu_info():
    """(BLAS threads numpy uses, CPU model, nproc) of this host."""
    import numpy as np  # noqa: F401  (loads the BLAS threadpoolctl reports)
    threads = None
    try:
        import threadpoolctl
        info = [i for i in threadpoolctl.threadpool_info() if i.get("user_api") == "blas"]
        threads = info[0]["num_threads"] if info else None
    except ImportError:
        pass
    model = None
    try:
        with open("/proc/cpuinfo") as f:
            model = next((ln.split(":", 1)[1].strip() for ln in f
                          if ln.startswith("model name")), None)
    except OSError:
        pass
    return threads, model, os.cpu_count()


def _cpu_reps(fn, min_reps: int = 5, max_seconds: float = 12.0):
    """Median and count of repeated host timings of fn (one untimed warm-up)."""
    fn()
    t, start = [], time.perf_counter()
    while len(t) < min_reps or (time.perf_counter() - start < 2.0 and len(t) < 50):
        t0 = time.perf_counter()
        fn()
        t.append(time.perf_counter() - t0)
        if time.perf_counter() - start > max_seconds and len(t) >= 3:
            break
    return _median(t), len(t)


def cpu_linear_baseline():
    """The reference's own Linear arithmetic on the host: numpy
    ``x @ W.T`` then ``+= b`` (novann/functional.py:160-162, restated in
    oracle.functional_ref.linear) at config [4], W the E4M3-quantized weight
    dequantized to fp32 by the C oracle.  Median of >= 5 repetitions."""
    import numpy as np

    import oracle as O
    from oracle import functional_ref as R
    M, K, N = 2048, 4096, 4096
    rng = np.random.default_rng(4)
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = rng.standard_normal((N, K), dtype=np.float32) * np.float32((2.0 / K) ** 0.5)
    s = O.scale_from_amax(O.amax(w), O.E4M3)
    wd = O.cast(O.cast(w, O.F32, O.E4M3, scale=s), O.E4M3, O.F32, n=w.size,
                scale=s).reshape(N, K)
    b = np.zeros((1, N), dtype=np.float32)
    med, reps = _cpu_reps(lambda: R.linear(x, wd, b))
    threads, model, ncpu = _cpu_info()
    return {"value": round(2.0 * M * N * K / med / 1e12, 4), "unit": "TFLOP/s",
            "ms": round(med * 1e3, 3), "cores": threads, "nproc": ncpu, "cpu": model,
            "kind": "port",
            "sample": f"config [4] at full size (x {M}x{K} fp32, dequantized E4M3 W {N}x{K}), "
                      f"numpy x @ W.T + b (OpenBLAS sgemm, {threads} threads), "
                      f"median of {reps}"}


def cpu_conv_baseline():
    """The reference's own Conv2d arithmetic on the host: numpy.pad +
    as_strided im2col + one GEMM + bias + NCHW view (novann/functional.py:
    346-382, restated in oracle.functional_ref.conv2d) for config [5]'s two
    layers, E2M1-quantized weights dequantized by the C oracle.  Median of
    >= 5 repetitions per layer."""
    import numpy as np

    import oracle as O
    from oracle import functional_ref as R
    rng = np.random.default_rng(5)
    x = rng.random((256, 1, 28, 28), dtype=np.float32)
    threads, model, ncpu = _cpu_info()
    out = []
    for cin, cout in ((1, 32), (32, 64)):
        w = rng.standard_normal((cout, cin, 3, 3), dtype=np.float32) * np.float32(
            (2.0 / (cin * 9)) ** 0.5)
        s = O.scale_from_amax(O.amax(w), O.E2M1)
        wd = O.cast(O.cast(w, O.F32, O.E2M1, scale=s), O.E2M1, O.F32, n=w.size,
                    scale=s).reshape(w.shape)
        b = np.zeros((cout, 1), dtype=np.float32)
        y = None

        def run(x=x, wd=wd, b=b):
            nonlocal y
            y = R.conv2d(x, wd, (1, 1), (1, 1), "zeros", b)
        med, reps = _cpu_reps(run)
        nbytes = (x.size + 256 * cout * 28 * 28) * 4
        out.append({"layer": f"conv {cin}->{cout}", "ms": round(med * 1e3, 3),
                    "GB/s": round(nbytes / med / 1e9, 3), "reps": reps})
        x = np.ascontiguousarray(y)
    return {"layers": out, "unit": "GB/s", "cores": threads, "nproc": ncpu, "cpu": model,
            "kind": "port",
            "sample": f"config [5] at full size (batch 256), numpy im2col + GEMM "
                      f"(OpenBLAS, {threads} threads), median per layer"}


LEGS = ("sweep", "linear", "linear_backward", "conv", "conv_backward", "epilogue", "adamw",
        "pool", "extras", "fp4", "cpu")


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--elems", type=int, default=1 << 28)
    ap.add_argument("--cpu-sample", type=int, default=1 << 26)
    ap.add_argument("--only", default="",
                    help="comma-separated subset of legs to run (profiling runs): "
                         + ", ".join(LEGS))
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-linear", action="store_true")
    ap.add_argument("--copy-probe", action="store_true",
                    help="also run one fp32->fp32 copy of the sweep input (known bytes), "
                         "the reference dispatch for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE")
    ap.add_argument("--no-conv", action="store_true")
    ap.add_argument("--no-fp4", action="store_true")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(run with --gpus 1)", file=sys.stderr)
        return 2
    legs = set(args.only.split(",")) if args.only else set(LEGS)
    unknown = legs - set(LEGS)
    if unknown:
        print(f"bench.py: unknown legs {sorted(unknown)}; known: {', '.join(LEGS)}",
              file=sys.stderr)
        return 2
    if args.no_linear:
        legs -= {"linear", "linear_backward"}
    if args.no_conv:
        legs -= {"conv", "conv_backward", "epilogue", "adamw", "pool", "extras"}
    if args.no_fp4:
        legs.discard("fp4")
    if args.no_cpu:
        legs.discard("cpu")
    import torch
    dev = torch.device("cuda", 0)
    torch.cuda.set_device(dev)
    if args.copy_probe:
        from novann_amd import _lib
        src = torch.empty(args.elems, dtype=torch.float32, device=dev).fill_(1.0)
        dst = torch.empty_like(src)
        _lib.check(_lib.load().novaq_cast(src.data_ptr(), 0, dst.data_ptr(), 0, args.elems, None,
                                          torch.cuda.current_stream(dev).cuda_stream), "copy")
        torch.cuda.synchronize(dev)
        del src, dst
    ms = value = None
    per_op, roof, vendor_casts = None, None, None
    if "sweep" in legs:
        log(f"sweep: {args.elems} elements, {args.steps} steps, {args.warmup} warmup")
        ms, per_op, vendor_casts = bench_sweep(args.elems, args.steps, args.warmup, dev)
        value = BYTES_PER_ELEM * args.elems / (ms * 1e-3) / 1e9
        # dominant single-kernel op (the amax op also launches a 1-thread fill kernel)
        kernels = [p for p in per_op if p["op"] in KERNEL_OF]
        dom = max(kernels, key=lambda p: p["ms"])
        dom_bpe = dict(SWEEP)[dom["op"]]
        roof = {"bound": "hbm", "kernel": f'{dom["op"]} ({KERNEL_OF[dom["op"]]})',
                "achieved": dom["GB/s"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                "frac": dom["frac"],
                "traffic": (measured_traffic(KERNEL_OF[dom["op"]])
                            if args.elems == 1 << 28 else None),
                "bytes_per_launch": dom_bpe * args.elems}
        log(f"sweep done: {ms:.3f} ms/step, {value:.1f} GB/s")
    run = {}
    for leg, fn in (("linear", bench_linear), ("linear_backward", bench_linear_backward),
                    ("conv", bench_conv), ("conv_backward", bench_conv_backward),
                    ("epilogue", bench_epilogue), ("adamw", bench_optim),
                    ("pool", bench_pool), ("extras", bench_extras), ("fp4", bench_fp4)):
        run[leg] = fn(dev) if leg in legs else None
        log(f"{leg}: {run[leg]}")
    cpu = None
    if "cpu" in legs:
        cpu = cpu_baseline(args.cpu_sample)
        log(f"cpu baseline: {cpu}")
        if run["linear"] is not None:
            run["linear"]["cpu_baseline"] = cpu_linear_baseline()
            log(f"linear cpu baseline: {run['linear']['cpu_baseline']}")
        if run["conv"] is not None:
            run["conv"]["cpu_baseline"] = cpu_conv_baseline()
            log(f"conv2d cpu baseline: {run['conv']['cpu_baseline']}")
    out = {
        "metric": METRIC, "value": None if value is None else round(value, 1), "unit": "GB/s",
        "n_gpus": 1, "steps": args.steps, "warmup": args.warmup,
        "ms_per_step": None if ms is None else round(ms, 4),
        "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
        "dtype": "f32<->{f16,bf16,e4m3,e5m2}", "data": "synthetic",
        "config": {"workload": "BASELINE config [2]: cast sweep, amax-scaled FP8",
                   "elements": args.elems, "bytes_per_element": BYTES_PER_ELEM},
        "roofline": roof,
        "kernels": per_op,
        "vendor_casts": vendor_casts,
        "linear": run["linear"],
        "linear_backward": run["linear_backward"],
        "conv2d": run["conv"],
        "conv2d_backward": run["conv_backward"],
        "epilogue": run["epilogue"],
        "adamw": run["adamw"],
        "pool": run["pool"],
        "extras": run["extras"],
        "fp4": run["fp4"],
        "cpu_baseline": cpu,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
