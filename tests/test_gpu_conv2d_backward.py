"""Backward products of the quantized Conv2d on the GPU (through the C ABI) vs
the CPU restatement of Conv2d.backward and _col2im
(novann/layers/convolutional/conv2d.py:117-148, 179-207).

Tolerance: normwise max|g - r| / max|r| <= 1e-2 against fp64 on the same fp32
grad and input and the dequantized weight (the BASELINE tolerance of the
forward products).  grad_bias is an fp32 sum, so it is held to 1e-5."""
import numpy as np
import pytest
import torch

from oracle import functional_ref as R
from novann_amd import _lib
from novann_amd import functional as F
from novann_amd.module import Conv2d, Parameters, QuantizedParameters

pytestmark = pytest.mark.gpu

TOL = 1e-2


def normwise(g, r):
    return float(np.abs(g.astype(np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


def weight_of(w, wdt):
    if wdt in ("e4m3", "e5m2", "e2m1"):
        q = QuantizedParameters.from_float(w, wdt)
        return q, q.dequantize().cpu().numpy().astype(np.float64).reshape(w.shape)
    return Parameters(w), w.astype(np.float64)


def check_case(N, C, H, W, C_out, KH, KW, stride, pad, wdt, mode="zeros", seed=0):
    print(f"conv2d_backward N={N} C={C} H={H} W={W} C_out={C_out} k={KH}x{KW} s={stride} "
          f"p={pad} {wdt} {mode}", flush=True)
    rng = np.random.default_rng(seed + N * 7 + C * 11 + C_out * 13 + KH)
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = (rng.standard_normal((C_out, C, KH, KW)) * np.sqrt(2.0 / (C * KH * KW))).astype(np.float32)
    OH = (H + 2 * pad[0] - KH) // stride[0] + 1
    OW = (W + 2 * pad[1] - KW) // stride[1] + 1
    g = rng.standard_normal((N, C_out, OH, OW)).astype(np.float32)
    weight, wdeq = weight_of(w, wdt)
    gi, gw, gb = F.conv2d_backward(torch.from_numpy(g).cuda(), torch.from_numpy(x).cuda(),
                                   weight, (KH, KW), stride, pad, bias=True, padding_mode=mode)
    torch.cuda.synchronize()
    ri, rw, rb = R.conv2d_backward(g.astype(np.float64), x.astype(np.float64), wdeq, stride,
                                   pad, mode)
    assert gi.shape == (N, C, H, W) and gw.shape == (C_out, C, KH, KW) and gb.shape == (C_out, 1)
    ei, ew = normwise(gi.cpu().numpy(), ri), normwise(gw.cpu().numpy(), rw)
    assert ei <= TOL, f"grad_input {ei}"
    assert ew <= TOL, f"grad_weight {ew}"
    np.testing.assert_allclose(gb.cpu().numpy(), rb, rtol=1e-5,
                               atol=1e-5 * np.sqrt(N * OH * OW))


GEOMETRIES = [
    # N, C, H, W, C_out, KH, KW, stride, pad
    (2, 2, 6, 6, 3, 3, 3, (1, 1), (1, 1)),       # reference test_conv2d.py:44-86 shape
    (4, 8, 12, 12, 16, 3, 3, (1, 1), (1, 1)),    # grad_input on the forward band kernel
    (3, 5, 9, 11, 70, 3, 3, (2, 2), (1, 1)),     # stride 2: direct grad_input; C_out > 64
    (2, 3, 10, 10, 7, 5, 5, (1, 1), (2, 2)),     # 5x5; E2M1 weight count odd (525)
    (2, 4, 7, 9, 6, 3, 2, (1, 1), (3, 2)),       # padding >= kernel: direct grad_input
    (1, 16, 16, 16, 8, 1, 1, (1, 1), (0, 0)),    # 1x1
    (5, 64, 9, 9, 24, 3, 3, (1, 2), (0, 1)),     # mixed strides, C = 64
    (2, 3, 33, 70, 65, 3, 3, (1, 1), (1, 1)),    # long rows (OW > 64), many pixels per image
]


@pytest.mark.parametrize("wdt", ["e4m3", "e5m2", "e2m1", "f32"])
@pytest.mark.parametrize("geom", GEOMETRIES, ids=lambda g: "x".join(map(str, g[:7])))
def test_conv2d_backward_vs_oracle(geom, wdt):
    check_case(*geom, wdt)


# grad_weight and grad_bias on the stride-1 rows kernel (8 to 12 taps, at
# most 8 columns, output rows of at most 64 pixels, 16 or more input
# channels, at most 5 staged slots per lane), and shapes just outside it
ROWS_GEOMETRIES = [
    (2, 40, 13, 15, 70, 3, 3, (1, 1), (1, 1)),   # 16-pixel rows, last band partial, both channel blocks partial
    (2, 17, 9, 50, 33, 3, 3, (1, 1), (0, 2)),    # 52-pixel rows (two per band)
    (2, 16, 10, 12, 8, 3, 4, (1, 1), (1, 2)),    # 12 taps: even and odd column shifts
    (2, 16, 9, 9, 8, 2, 4, (1, 1), (1, 2)),      # 8 taps
    (3, 16, 10, 12, 8, 4, 4, (1, 1), (2, 1)),    # 16 taps: the general kernel
    (1, 16, 6, 20, 8, 2, 8, (1, 1), (0, 3)),     # 8 columns, 16 taps: the general kernel
    (2, 96, 7, 30, 130, 3, 3, (1, 1), (1, 1)),   # three input and three output channel blocks
]


@pytest.mark.parametrize("wdt", ["e4m3", "e2m1"])
@pytest.mark.parametrize("geom", ROWS_GEOMETRIES, ids=lambda g: "x".join(map(str, g[:7])))
def test_conv2d_backward_rows_path(geom, wdt):
    check_case(*geom, wdt)


# zero padding, W and OW multiples of 4: the rows kernel stages with 16-byte
# loads (N, C, H, W, C_out, KH, KW, pad)
VEC_GEOMETRIES = [
    (2, 16, 12, 12, 8, 3, 3, (1, 1)),    # input column 0 at staged column 2 (pw 1)
    (2, 16, 12, 8, 8, 8, 1, (0, 0)),     # 8 x 1 window, pw 0
    (2, 16, 10, 16, 8, 2, 5, (1, 2)),    # pw 2
    (2, 16, 9, 20, 8, 3, 3, (1, 3)),     # pw 3: staged column 4
    (1, 16, 6, 60, 8, 3, 3, (1, 1)),     # 60-pixel rows, 3 input quads per lane
    (3, 24, 13, 16, 40, 3, 3, (1, 1)),   # 16-pixel rows, last band partial, partial blocks
    (2, 48, 8, 8, 80, 3, 3, (1, 1)),     # two input and two output channel blocks
    (2, 64, 6, 60, 128, 4, 3, (2, 1)),   # 12 taps, 4 input quads per lane, two blocks each
]


def backward_bits(g, x, N, C, H, W, w, C_out, KH, KW, pad, outs, mode="zeros"):
    """One C ABI call (grad_weight and / or grad_bias per outs) -> host arrays."""
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    code = _lib.DTYPES["e2m1"]
    nbytes = lib.novaq_conv2d_backward_workspace(N, C, C_out, KH, KW, code)
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    gw = torch.full((C_out, C, KH, KW), 7.0, device="cuda")
    gb = torch.full((C_out,), 7.0, device="cuda")
    _lib.check(lib.novaq_conv2d_backward(
        g.data_ptr(), x.data_ptr(), N, C, H, W, w.codes.data_ptr(), code, w.scale.data_ptr(),
        C_out, KH, KW, 1, 1, pad[0], pad[1], _lib.PAD_MODES[mode], None,
        gw.data_ptr() if "w" in outs else None, gb.data_ptr() if "b" in outs else None,
        ws.data_ptr(), nbytes, st), "conv2d backward")
    torch.cuda.synchronize()
    return gw.cpu().numpy().view(np.int32), gb.cpu().numpy()


def bf16_round(a):
    """fp32 -> nearest bf16 (ties to even), as fp32 (finite inputs)."""
    u = np.ascontiguousarray(a, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    return u.astype(np.uint32).view(np.float32)


@pytest.mark.parametrize("geom", VEC_GEOMETRIES, ids=lambda g: "x".join(map(str, g[:7])))
def test_conv2d_backward_rows_vec_staging(geom):
    """The 16-byte staging against the oracle, and grad_weight against the
    fp64 product of the operands the MFMAs multiply (grad and input rounded to
    bf16) within 1e-5: a staging slip (a pixel, row or channel dropped or
    shifted) costs more.  A bias-only and a weight-only call give the full
    call's bits."""
    N, C, H, W, C_out, KH, KW, pad = geom
    check_case(N, C, H, W, C_out, KH, KW, (1, 1), pad, "e2m1")
    rng = np.random.default_rng(sum(geom[:7]))
    OH, OW = H + 2 * pad[0] - KH + 1, W + 2 * pad[1] - KW + 1
    assert W % 4 == 0 and OW % 4 == 0
    xh = rng.standard_normal((N, C, H, W)).astype(np.float32)
    gh = rng.standard_normal((N, C_out, OH, OW)).astype(np.float32)
    x, g = torch.from_numpy(xh).cuda(), torch.from_numpy(gh).cuda()
    w = QuantizedParameters.from_float(
        (rng.standard_normal((C_out, C, KH, KW)) * 0.2).astype(np.float32), "e2m1")
    wv, bv = backward_bits(g, x, N, C, H, W, w, C_out, KH, KW, pad, "wb")
    wdeq = w.dequantize().cpu().numpy().astype(np.float64).reshape(C_out, C, KH, KW)
    _, rw, _ = R.conv2d_backward(bf16_round(gh).astype(np.float64),
                                 bf16_round(xh).astype(np.float64), wdeq, (1, 1), pad, "zeros")
    assert normwise(wv.view(np.float32), rw) <= 1e-5
    assert np.array_equal(backward_bits(g, x, N, C, H, W, w, C_out, KH, KW, pad, "w")[0], wv)
    assert np.array_equal(backward_bits(g, x, N, C, H, W, w, C_out, KH, KW, pad, "b")[1], bv)


# one input channel, stride 1, at most 16 taps, OW a multiple of 4 and at
# most 64, C_out <= 64: grad_weight with the taps as the GEMM's N
# (N, H, W, C_out, KH, KW, pad, mode)
C1_GEOMETRIES = [
    (2, 12, 16, 8, 3, 3, (1, 1), "zeros"),
    (3, 9, 20, 40, 3, 5, (1, 2), "reflect"),      # 15 taps, three channel tiles
    (1, 17, 39, 64, 4, 4, (2, 2), "replicate"),   # 16 taps, 40-pixel rows (two k-steps a row)
    (2, 7, 8, 33, 2, 3, (0, 1), "circular"),      # a partial last channel tile
    (5, 30, 28, 32, 3, 3, (1, 1), "zeros"),       # config [5] conv1's shape, 5 images
]


@pytest.mark.parametrize("geom", C1_GEOMETRIES, ids=lambda g: "x".join(map(str, g[:6])))
def test_conv2d_backward_one_input_channel(geom):
    """Against the oracle, grad_weight against the fp64 product of the
    operands the MFMAs multiply (grad and input rounded to bf16) within 1e-5,
    and a bias-only and a weight-only call give the full call's bits."""
    N, H, W, C_out, KH, KW, pad, mode = geom
    check_case(N, 1, H, W, C_out, KH, KW, (1, 1), pad, "e2m1", mode=mode)
    rng = np.random.default_rng(sum(geom[:6]) + 3)
    OH, OW = H + 2 * pad[0] - KH + 1, W + 2 * pad[1] - KW + 1
    assert OW % 4 == 0
    xh = rng.standard_normal((N, 1, H, W)).astype(np.float32)
    gh = rng.standard_normal((N, C_out, OH, OW)).astype(np.float32)
    x, g = torch.from_numpy(xh).cuda(), torch.from_numpy(gh).cuda()
    w = QuantizedParameters.from_float(
        (rng.standard_normal((C_out, 1, KH, KW)) * 0.3).astype(np.float32), "e2m1")
    wv, bv = backward_bits(g, x, N, 1, H, W, w, C_out, KH, KW, pad, "wb", mode)
    wdeq = w.dequantize().cpu().numpy().astype(np.float64).reshape(C_out, 1, KH, KW)
    _, rw, _ = R.conv2d_backward(bf16_round(gh).astype(np.float64),
                                 bf16_round(xh).astype(np.float64), wdeq, (1, 1), pad, mode)
    assert normwise(wv.view(np.float32), rw) <= 1e-5
    assert np.array_equal(backward_bits(g, x, N, 1, H, W, w, C_out, KH, KW, pad, "w", mode)[0], wv)
    assert np.array_equal(backward_bits(g, x, N, 1, H, W, w, C_out, KH, KW, pad, "b", mode)[1], bv)


@pytest.mark.parametrize("mode", ["zeros", "reflect", "replicate", "circular"])
@pytest.mark.parametrize("geom", [(2, 3, 8, 9, 5, 3, 3, (1, 1), (1, 2)),
                                  (2, 4, 11, 10, 6, 3, 3, (2, 1), (2, 1)),
                                  (2, 16, 8, 9, 5, 3, 3, (1, 1), (1, 2))],
                         ids=["s1", "s2", "s1rows"])
def test_conv2d_backward_padding_modes(geom, mode):
    """grad_weight reads the input padded in the forward's mode; grad_input is
    the cropped col2im, the same in every mode (conv2d.py:141-148)."""
    check_case(*geom, "e4m3", mode=mode)


@pytest.mark.parametrize("layer,cin,cout", [("conv1", 1, 32), ("conv2", 32, 64)])
def test_conv2d_backward_mnist_shapes(layer, cin, cout):
    """Config [5]'s two convolutions (batch 256, 28x28, 3x3/s1/p1, FP4 E2M1)."""
    check_case(256, cin, 28, 28, cout, 3, 3, (1, 1), (1, 1), "e2m1")


def test_conv2d_backward_deterministic_and_partial_outputs():
    rng = np.random.default_rng(5)
    N, C, H, W, C_out = 8, 16, 14, 14, 32
    x = torch.from_numpy(rng.standard_normal((N, C, H, W)).astype(np.float32)).cuda()
    g = torch.from_numpy(rng.standard_normal((N, C_out, H, W)).astype(np.float32)).cuda()
    w = QuantizedParameters.from_float(
        (rng.standard_normal((C_out, C, 3, 3)) * 0.1).astype(np.float32), "e4m3")
    a = F.conv2d_backward(g, x, w, 3, 1, 1)
    b = F.conv2d_backward(g, x, w, 3, 1, 1)
    torch.cuda.synchronize()
    for u, v in zip(a, b):
        assert torch.equal(u, v)
    # one output at a time through the C ABI gives the same bits
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    nbytes = lib.novaq_conv2d_backward_workspace(N, C, C_out, 3, 3, _lib.DTYPES["e4m3"])
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    outs = [torch.full_like(t, 7.0) for t in a]
    for k in range(3):
        ptrs = [None, None, None]
        ptrs[k] = outs[k].data_ptr()
        _lib.check(lib.novaq_conv2d_backward(
            g.data_ptr(), x.data_ptr(), N, C, H, W, w.codes.data_ptr(), _lib.DTYPES["e4m3"],
            w.scale.data_ptr(), C_out, 3, 3, 1, 1, 1, 1, _lib.PAD_MODES["zeros"], *ptrs,
            ws.data_ptr(), nbytes, st), "conv2d backward")
    torch.cuda.synchronize()
    for u, v in zip(a, outs):
        assert torch.equal(u, v)


def test_conv2d_backward_empty_batch():
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    C, C_out = 4, 6
    w = QuantizedParameters.from_float(np.ones((C_out, C, 3, 3), np.float32), "e2m1")
    nbytes = lib.novaq_conv2d_backward_workspace(0, C, C_out, 3, 3, _lib.DTYPES["e2m1"])
    ws = torch.empty(nbytes, dtype=torch.uint8, device="cuda")
    gw = torch.full((C_out, C, 3, 3), 7.0, device="cuda")
    gb = torch.full((C_out, 1), 7.0, device="cuda")
    _lib.check(lib.novaq_conv2d_backward(None, None, 0, C, 5, 5, w.codes.data_ptr(),
                                         _lib.DTYPES["e2m1"], w.scale.data_ptr(), C_out, 3, 3,
                                         1, 1, 1, 1, 0, None, gw.data_ptr(), gb.data_ptr(),
                                         ws.data_ptr(), nbytes, st), "conv2d backward")
    torch.cuda.synchronize()
    assert torch.count_nonzero(gw).item() == 0 and torch.count_nonzero(gb).item() == 0


def test_layer_backward_like_reference():
    """novann tests/layers/conv/test_conv2d.py:44-86 on the quantized layer:
    gradients against the oracle (whose finite-difference agreement is pinned
    on the CPU) and the grad_input shape."""
    rng = np.random.RandomState(0)
    layer = Conv2d(in_channels=2, out_channels=3, kernel_size=3, stride=1, padding=1,
                   bias=True, weight_dtype="e4m3")
    x = rng.randn(2, 2, 6, 6).astype(np.float32) * 0.1
    out = layer(x)
    G = rng.randn(*out.shape).astype(np.float32) * 0.1
    grad_input = layer.backward(G)
    wdeq = layer.weight.dequantize().cpu().numpy().astype(np.float64).reshape(3, 2, 3, 3)
    ri, rw, rb = R.conv2d_backward(G.astype(np.float64), x.astype(np.float64), wdeq, 1, 1)
    assert isinstance(grad_input, np.ndarray) and grad_input.shape == x.shape
    assert layer.weight.grad.shape == (3, 2, 3, 3) and layer.bias.grad.shape == (3, 1)
    assert normwise(layer.weight.grad, rw) <= TOL
    assert np.abs(layer.bias.grad - rb).max() < 5e-3
    assert normwise(grad_input, ri) <= TOL
