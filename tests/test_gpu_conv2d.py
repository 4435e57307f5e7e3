"""Quantized Conv2d on the GPU vs the CPU oracle (direct fp64 loops and the
numpy im2col restatement of novann/functional.py:275-385).

Tolerance: normwise max|y - r| / max|r| <= 1e-2 against fp64 on the same fp32
input and the dequantized fp32 weights."""
import numpy as np
import pytest
import torch

import oracle as O
from oracle import functional_ref as R
from novann_amd import _lib
from novann_amd import functional as F
from novann_amd.module import Conv2d, Parameters, QuantizedParameters
from tests.gpu_util import bf16_round, error_report, to_dev

pytestmark = pytest.mark.gpu

TOL = 1e-2
QCODE = {"e4m3": O.E4M3, "e5m2": O.E5M2, "e2m1": O.E2M1, "bf16": O.BF16, "f16": O.F16,
         "f32": O.F32}


def normwise(y, r):
    return float(np.abs(y.astype(np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


def run_conv(x, codes, wdt, wshape, scale, bias, stride, padding, mode):
    N, C, H, W = x.shape
    C_out, _, KH, KW = wshape
    sh, sw = stride
    ph, pw = padding
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    wd = to_dev(codes, QCODE[wdt])
    sd = None if scale is None else torch.tensor([scale], dtype=torch.float32, device="cuda")
    bd = None if bias is None else torch.from_numpy(np.ascontiguousarray(bias, np.float32)).cuda()
    yd = torch.empty((N, C_out, OH, OW), dtype=torch.float32, device="cuda")
    rc = _lib.load().novaq_conv2d_forward(
        xd.data_ptr(), N, C, H, W, wd.data_ptr(), _lib.DTYPES[wdt],
        None if sd is None else sd.data_ptr(), C_out, KH, KW, sh, sw, ph, pw,
        _lib.PAD_MODES[mode], None if bd is None else bd.data_ptr(), yd.data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "conv2d")
    torch.cuda.synchronize()
    return yd.cpu().numpy()


def quantize_weights(w, wdt):
    c = QCODE[wdt]
    if wdt in ("e4m3", "e5m2", "e2m1"):
        s = O.scale_from_amax(O.amax(w), c)
        codes = O.cast(w.reshape(-1), O.F32, c, scale=s)
        wdeq = O.cast(codes, c, O.F32, n=w.size, scale=s).reshape(w.shape)
        return codes, s, wdeq
    if wdt == "f32":
        return w.reshape(-1).view(np.uint32), None, w
    codes = O.cast(w.reshape(-1), O.F32, c)
    return codes, None, O.cast(codes, c, O.F32).reshape(w.shape)


def test_golden_fixture_all_padding_modes(golden):
    g = golden["products"]
    x = g["conv_x"]
    for mode in ("zeros", "reflect", "replicate", "circular"):
        want = g[f"conv_y_{mode}"]
        y = run_conv(x, g["conv_packed"], "e2m1", (5, 3, 3, 3), float(g["conv_scale"][0]),
                     g["conv_bias"], (2, 1), (2, 1), mode)
        assert y.shape == want.shape
        assert normwise(y, want.astype(np.float64)) <= TOL, mode


@pytest.mark.parametrize("wdt", ["e2m1", "e4m3", "e5m2", "bf16", "f16", "f32"])
@pytest.mark.parametrize("mode", ["zeros", "reflect", "replicate", "circular"])
@pytest.mark.parametrize("case", [
    # (N, C, H, W, C_out, KH, KW, sh, sw, ph, pw)
    (2, 3, 16, 16, 4, 3, 3, 1, 1, 1, 1),
    (2, 2, 20, 20, 4, 5, 5, 2, 2, 0, 0),
    (3, 2, 16, 16, 4, 3, 5, 2, 1, 1, 2),
    (1, 1, 8, 8, 2, 3, 3, 1, 1, 2, 2),
    (2, 9, 11, 13, 70, 3, 3, 1, 1, 1, 1),
    (1, 70, 9, 7, 33, 3, 3, 1, 1, 1, 1),
    (2, 16, 31, 33, 64, 1, 1, 1, 1, 0, 0),
    # 3x3 with C a multiple of 8 (the constant-shift weight regrouping) and a
    # partial output-channel block
    (2, 16, 12, 12, 40, 3, 3, 1, 1, 1, 1),
    (1, 8, 9, 16, 70, 3, 3, 2, 2, 1, 1),
    # few input channels, stride 1 (the VALU small-channel kernel): config
    # [5]'s conv1 shape at batch 3, widths that are no multiple of 4, 5 x 5 /
    # 7 x 7 / non-square windows, more than 8 output channels
    (3, 1, 28, 28, 32, 3, 3, 1, 1, 1, 1),
    (2, 4, 13, 10, 9, 5, 5, 1, 1, 2, 2),
    (1, 2, 9, 7, 3, 7, 7, 1, 1, 3, 3),
    (2, 3, 6, 6, 12, 2, 4, 1, 1, 0, 3),
    # batch x channel groups large enough for two 8-channel groups per
    # workgroup, the last group partial (37 = 4 x 8 + 5)
    (208, 2, 6, 6, 37, 3, 3, 1, 1, 1, 1),
    # one output channel (an MFMA tile's 16 columns hold 1): 5 x 5 and 3 x 8
    # windows, C no multiple of 8, W no multiple of 4
    (2, 32, 12, 16, 1, 3, 3, 1, 1, 1, 1),
    (2, 5, 9, 8, 1, 5, 5, 1, 1, 2, 2),
    (1, 70, 10, 12, 1, 3, 8, 1, 1, 1, 3),
    (2, 16, 7, 7, 1, 3, 3, 1, 1, 1, 1),
])
def test_shapes_and_modes_vs_oracle(wdt, mode, case):
    N, C, H, W, C_out, KH, KW, sh, sw, ph, pw = case
    rng = np.random.default_rng(sum(case) + len(mode))
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = (rng.standard_normal((C_out, C, KH, KW)) * np.sqrt(2.0 / (C * KH * KW))).astype(np.float32)
    b = rng.standard_normal(C_out).astype(np.float32)
    codes, s, wdeq = quantize_weights(w, wdt)
    y = run_conv(x, codes, wdt, w.shape, s, b, (sh, sw), (ph, pw), mode)
    r = O.conv2d_f64(x, wdeq, (sh, sw), (ph, pw), mode, b)
    assert normwise(y, r.astype(np.float64)) <= TOL
    # the numpy im2col restatement agrees with the direct loops
    r2 = R.conv2d(x.astype(np.float64), wdeq.astype(np.float64), (sh, sw), (ph, pw), mode,
                  b.astype(np.float64))
    assert np.allclose(r, r2, rtol=1e-5, atol=1e-5)


@pytest.mark.parametrize("case", [
    # (N, C, H, W, KH, KW, ph, pw, mode)
    (4, 32, 28, 28, 3, 3, 1, 1, "zeros"),     # config [5] conv1's input gradient, 4 images
    (2, 37, 13, 20, 2, 5, 0, 2, "reflect"),   # C no multiple of 8
    (3, 8, 30, 8, 7, 7, 3, 3, "circular"),    # 7 x 7, rows wider than the image's 8 columns
    (1, 6, 70, 4, 3, 1, 1, 0, "replicate"),   # narrow rows: many rows per band
    # zero padding, W a multiple of 4: the taps as the MFMA's N
    (2, 64, 10, 12, 4, 4, 2, 1, "zeros"),     # 16 taps, two channel steps of 32
    (3, 37, 13, 8, 1, 8, 0, 4, "zeros"),      # a 1 x 8 window, C no multiple of 8
    (2, 8, 40, 20, 2, 2, 0, 0, "zeros"),      # 13-row bands
])
def test_one_output_channel_exact_operands(case):
    """C_out = 1 (the input gradient of a one-channel convolution is one)
    against the fp64 convolution of the operands the kernel multiplies (x
    rounded to bf16, the dequantized E4M3 weight) within 1e-5: a staging slip
    (a row, column or channel dropped or shifted) costs far more."""
    N, C, H, W, KH, KW, ph, pw, mode = case
    print(f"conv2d C_out=1 {case}", flush=True)
    rng = np.random.default_rng(sum(case[:8]))
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = (rng.standard_normal((1, C, KH, KW)) * 0.3).astype(np.float32)
    codes, s, wdeq = quantize_weights(w, "e4m3")
    y = run_conv(x, codes, "e4m3", w.shape, s, None, (1, 1), (ph, pw), mode)
    r = R.conv2d(bf16_round(x).astype(np.float64), wdeq.astype(np.float64), (1, 1), (ph, pw), mode)
    assert normwise(y, r) <= 1e-5


def test_config5_mnist_two_layers():
    """BASELINE config [5]: x (256, 1, 28, 28) U[0,1]; conv1 1->32 and conv2
    32->64, 3x3 / stride 1 / pad 1, Kaiming-normal weights in E2M1 with
    per-tensor scale, bias zero, conv2 applied to conv1's fp32 output."""
    rng = np.random.default_rng(5)
    x = rng.uniform(0, 1, (256, 1, 28, 28)).astype(np.float32)
    w1 = (rng.standard_normal((32, 1, 3, 3)) * np.sqrt(2.0 / 9)).astype(np.float32)
    w2 = (rng.standard_normal((64, 32, 3, 3)) * np.sqrt(2.0 / 288)).astype(np.float32)
    q1 = QuantizedParameters.from_float(w1, "e2m1")
    q2 = QuantizedParameters.from_float(w2, "e2m1")
    b1 = Parameters(np.zeros((32, 1), np.float32))
    b2 = Parameters(np.zeros((64, 1), np.float32))
    xd = torch.from_numpy(x).cuda()
    y1 = F.conv2d(xd, q1, 3, 1, 1, bias=b1)
    y2 = F.conv2d(y1, q2, 3, 1, 1, bias=b2)
    torch.cuda.synchronize()
    w1d = q1.dequantize().cpu().numpy()
    w2d = q2.dequantize().cpu().numpy()
    y1h, y2h = y1.cpu().numpy(), y2.cpu().numpy()
    r1 = O.conv2d_f64(x, w1d, (1, 1), (1, 1))
    rep1 = error_report(y1h, r1.astype(np.float64))
    assert rep1["normwise"] <= TOL, rep1
    # layer 2 checked on the GPU's own layer-1 output (isolates layer 2's error)
    r2 = O.conv2d_f64(y1h, w2d, (1, 1), (1, 1))
    rep2 = error_report(y2h, r2.astype(np.float64))
    assert rep2["normwise"] <= TOL, rep2
    # and end to end against the all-fp64 chain
    r2_chain = O.conv2d_f64(r1, w2d, (1, 1), (1, 1))
    assert normwise(y2h, r2_chain.astype(np.float64)) <= TOL
    # against the fp64 convolution of the operands the kernels multiply (the
    # input rounded to bf16, W decoded exactly): fp32 summation error only
    e1 = error_report(y1h, O.conv2d_f64(bf16_round(x), w1d, (1, 1), (1, 1)).astype(np.float64))
    e2 = error_report(y2h, O.conv2d_f64(bf16_round(y1h), w2d, (1, 1), (1, 1)).astype(np.float64))
    print(f"config [5] conv1 vs fp32-input fp64: {rep1}; exact-operand: {e1}", flush=True)
    print(f"config [5] conv2 vs fp32-input fp64: {rep2}; exact-operand: {e2}", flush=True)
    assert e1["normwise"] <= 1e-5 and e2["normwise"] <= 1e-5, (e1, e2)


def test_layer_shape_contracts_like_reference():
    """novann tests/layers/conv/test_conv2d.py:10-43, :87-132 shape contracts."""
    rng = np.random.RandomState(0)
    layer = Conv2d(3, 16, kernel_size=3, stride=1, padding=1, bias=True, weight_dtype="e2m1")
    out = layer(rng.randn(4, 3, 32, 32).astype(np.float32))
    assert out.shape == (4, 16, 32, 32) and out.dtype == np.float32
    layer = Conv2d(2, 4, kernel_size=5, stride=2, padding=0, bias=False, weight_dtype="e4m3")
    assert layer.bias is None
    assert layer(rng.randn(2, 2, 20, 20).astype(np.float32)).shape == (2, 4, 8, 8)
    for k, s, p in [(3, 1, 0), (5, 2, 1), ((3, 5), (2, 1), (1, 2))]:
        layer = Conv2d(2, 4, kernel_size=k, stride=s, padding=p, bias=False)
        out = layer(rng.randn(3, 2, 16, 16).astype(np.float32))
        assert out.shape[:2] == (3, 4) and out.shape[2] > 0 and out.shape[3] > 0
    for mode in ("zeros", "reflect", "replicate", "circular"):
        layer = Conv2d(1, 2, kernel_size=3, padding=2, padding_mode=mode, bias=False)
        out = layer(np.ones((1, 1, 8, 8), dtype=np.float32))
        assert out.shape[:2] == (1, 2)


@pytest.mark.parametrize("wdt,mode,xs,ws,stride,pad", [
    ("e2m1", "zeros", (1, 64, 3, 4096), (8, 64, 3, 3), (1, 1), (1, 1)),
    ("e4m3", "reflect", (2, 3, 4, 3000), (5, 3, 3, 5), (1, 2), (1, 2)),
    ("f32", "circular", (1, 80, 2, 2500), (3, 80, 2, 3), (1, 1), (0, 1)),
])
def test_rows_too_wide_for_lds(wdt, mode, xs, ws, stride, pad):
    """Images whose padded rows do not fit in LDS take the direct-gather
    kernel (no NOVAQ_ENOTSUP), within the same tolerance, with an epilogue."""
    print(f"conv2d wide rows {wdt} {mode} {xs} {ws}", flush=True)
    rng = np.random.default_rng(xs[3])
    x = rng.uniform(-1, 1, xs).astype(np.float32)
    w = (rng.standard_normal(ws) * np.sqrt(2.0 / np.prod(ws[1:]))).astype(np.float32)
    codes, s, wdeq = quantize_weights(w, wdt)
    b = rng.standard_normal(ws[0]).astype(np.float32)
    y = run_conv(x, codes, wdt, ws, s, b, stride, pad, mode)
    r = O.conv2d_f64(x, wdeq, stride, pad, mode, b)
    assert y.shape == r.shape and normwise(y, r) <= TOL
    # the same launch through the layer path with a ReLU epilogue
    wq = Parameters(wdeq) if wdt == "f32" else QuantizedParameters(
        to_dev(codes, QCODE[wdt]), ws, wdt, torch.tensor([s], device="cuda"))
    yr = F.conv2d(x, wq, ws[2:], stride, pad, bias=Parameters(b.reshape(-1, 1)),
                  padding_mode=mode, epilogue=F.Epilogue(relu=True))
    assert normwise(yr, np.maximum(r, 0.0)) <= TOL


def test_backward_rows_too_wide_for_lds():
    """Conv2d.backward on a wide image: grad_input's flipped-weight convolution
    falls back to the direct gather; all gradients within tolerance."""
    N, C, H, W, Co = 1, 64, 3, 4096, 8
    rng = np.random.default_rng(5)
    x = rng.uniform(-1, 1, (N, C, H, W)).astype(np.float32)
    w = (rng.standard_normal((Co, C, 3, 3)) * np.sqrt(2.0 / (C * 9))).astype(np.float32)
    codes, s, wdeq = quantize_weights(w, "e2m1")
    wq = QuantizedParameters(to_dev(codes, O.E2M1), w.shape, "e2m1",
                             torch.tensor([s], device="cuda"))
    g = rng.standard_normal((N, Co, H, W)).astype(np.float32)
    gi, gw, gb = F.conv2d_backward(g, x, wq, 3, 1, 1, bias=True)
    ri, rw, rb = R.conv2d_backward(g.astype(np.float64), x.astype(np.float64),
                                   wdeq.astype(np.float64), (1, 1), (1, 1))
    assert normwise(gi, ri) <= TOL and normwise(gw, rw) <= TOL
    assert normwise(gb.reshape(-1), rb.reshape(-1)) <= TOL
