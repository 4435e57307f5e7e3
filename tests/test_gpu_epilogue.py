"""Fused epilogues of the forward products on the GPU (through the C ABI).

Bit-exact checks: the epilogue's fp32 steps equal the oracle's fp32 restatement
applied to the unfused kernel output (every Linear and Conv2d kernel path);
bf16 / f16 / FP8 stores equal the oracle cast of those fp32 values; the output
amax equals max |v|.  Reference-path check: conv / linear -> eval BatchNorm
(fp64, the reference's formula) -> ReLU within normwise 1e-2 of the fused
result (the BASELINE tolerance of the products)."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from oracle import functional_ref as R
from novann_amd import _lib
from novann_amd import functional as F
from novann_amd.module import QuantizedParameters
from tests.gpu_util import to_dev, to_host

pytestmark = pytest.mark.gpu

TOL = 1e-2
OUT = {"f32": O.F32, "f16": O.F16, "bf16": O.BF16, "e4m3": O.E4M3, "e5m2": O.E5M2}
TORCH_OUT = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16,
             "e4m3": torch.uint8, "e5m2": torch.uint8}


def stream():
    return torch.cuda.current_stream().cuda_stream


def quantized_codes(w, wdt, rng):
    """Raw codes (device) of a weight, its scale tensor and the dequantized fp64 matrix."""
    if wdt in ("e4m3", "e5m2", "e2m1"):
        c = {"e4m3": O.E4M3, "e5m2": O.E5M2, "e2m1": O.E2M1}[wdt]
        s = O.scale_from_amax(O.amax(w), c)
        codes = O.cast(w.reshape(-1), O.F32, c, scale=s)
        deq = O.cast(codes, c, O.F32, n=w.size, scale=s).reshape(w.shape)
        return to_dev(codes, c), torch.tensor([s], dtype=torch.float32, device="cuda"), deq
    if wdt in ("bf16", "f16"):
        c = O.BF16 if wdt == "bf16" else O.F16
        codes = O.cast(w.reshape(-1), O.F32, c)
        return to_dev(codes, c), None, O.cast(codes, c, O.F32).reshape(w.shape)
    return torch.from_numpy(w).cuda(), None, w


class Epi:
    """ctypes epilogue + the device tensors it points at."""

    def __init__(self, C, rng, relu=True, out="f32", out_scale=None, amax=True, mul=True,
                 add=True, mul_vals=None, add_vals=None):
        self.mul = None if not mul else torch.from_numpy(
            mul_vals if mul_vals is not None
            else rng.uniform(-2.0, 2.0, C).astype(np.float32)).cuda()
        self.add = None if not add else torch.from_numpy(
            add_vals if add_vals is not None
            else rng.standard_normal(C).astype(np.float32)).cuda()
        self.scale = None if out_scale is None else torch.tensor([out_scale], device="cuda")
        self.amax = torch.full((1,), 123.0, device="cuda") if amax else None
        p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
        self.st = _lib.Epilogue(p(self.mul), p(self.add), p(self.scale), p(self.amax),
                                1 if relu else 0, _lib.DTYPES[out])
        self.relu, self.out = relu, out

    def host(self):
        return (None if self.mul is None else self.mul.cpu().numpy(),
                None if self.add is None else self.add.cpu().numpy())


def linear_ex(x, wd, wdt, ws, D_out, ep=None, bias=None):
    N, D_in = x.shape
    xd = torch.from_numpy(x).cuda()
    out = ep.out if ep is not None else "f32"
    y = torch.empty((N, D_out), dtype=TORCH_OUT[out], device="cuda")
    bd = None if bias is None else torch.from_numpy(bias).cuda()
    _lib.check(_lib.load().novaq_linear_forward_ex(
        xd.data_ptr(), O.F32, None, N, D_in, wd.data_ptr(), _lib.DTYPES[wdt],
        None if ws is None else ws.data_ptr(), None if bd is None else bd.data_ptr(), D_out,
        None if ep is None else ctypes.byref(ep.st), y.data_ptr(), stream()), "linear_ex")
    torch.cuda.synchronize()
    return to_host(y).reshape(N, D_out)


def conv_ex(x, wd, wdt, ws, wshape, stride, pad, mode="zeros", ep=None, bias=None):
    N, C, H, W = x.shape
    C_out, _, KH, KW = wshape
    OH, OW = (H + 2 * pad[0] - KH) // stride[0] + 1, (W + 2 * pad[1] - KW) // stride[1] + 1
    xd = torch.from_numpy(x).cuda()
    out = ep.out if ep is not None else "f32"
    y = torch.empty((N, C_out, OH, OW), dtype=TORCH_OUT[out], device="cuda")
    bd = None if bias is None else torch.from_numpy(bias).cuda()
    _lib.check(_lib.load().novaq_conv2d_forward_ex(
        xd.data_ptr(), O.F32, None, N, C, H, W, wd.data_ptr(), _lib.DTYPES[wdt],
        None if ws is None else ws.data_ptr(), C_out, KH, KW, stride[0], stride[1], pad[0],
        pad[1], _lib.PAD_MODES[mode], None if bd is None else bd.data_ptr(),
        None if ep is None else ctypes.byref(ep.st), y.data_ptr(), stream()), "conv2d_ex")
    torch.cuda.synchronize()
    return to_host(y).reshape(N, C_out, OH, OW)


def check_all_outputs(run, y0_bits, C, rng, axis=1):
    """Epilogue fp32 bit-exact vs the oracle on the unfused output, amax exact,
    and every narrower store equal to the oracle cast of the fp32 values."""
    y0 = y0_bits.view(np.float32)
    ep = Epi(C, rng)
    y1 = run(ep).view(np.float32)
    mul, add = ep.host()
    want = R.epilogue_f32(y0, mul, add, True, axis=axis)
    assert np.array_equal(y1.view(np.uint32), want.view(np.uint32)), \
        f"{np.count_nonzero(y1.view(np.uint32) != want.view(np.uint32))} epilogue mismatches"
    am = float(ep.amax.cpu()[0])
    assert am == float(np.abs(want).max())
    flat = want.reshape(-1)
    for out in ("bf16", "f16"):
        got = run(Epi(C, rng, out=out, mul_vals=mul, add_vals=add, amax=False)).reshape(-1)
        assert np.array_equal(got, O.cast(flat, O.F32, OUT[out])), out
    for out in ("e4m3", "e5m2"):
        s = O.scale_from_amax(np.float32(am), OUT[out])
        got = run(Epi(C, rng, out=out, out_scale=s, mul_vals=mul, add_vals=add,
                      amax=False)).reshape(-1)
        assert np.array_equal(got, O.cast(flat, O.F32, OUT[out], scale=s)), out


def rounding_classes(rng):
    """fp32 values covering every bf16 rounding case: random bf16 values of
    every exponent (subnormal to the largest finite) plus 0, 1, just below /
    at / just above the tie and the largest offset below the next value,
    with both parities of the kept bit; and the specials (signed zeros and
    infinities, NaNs with high / low / full payloads, subnormals at and
    around the tie, the largest finite that rounds to infinity)."""
    hi = rng.integers(0, 1 << 16, 400, dtype=np.uint32)
    base = hi << 16
    offs = np.array([0, 1, 0x7FFF, 0x8000, 0x8001, 0xFFFF], np.uint32)
    vals = (base[:, None] + offs[None, :]).reshape(-1)
    specials = np.array([0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7F800001,
                         0x7FC00000, 0x7FFFFFFF, 0xFF800001, 0xFFC00001, 0x7F80FFFF,
                         0x7FBFFFFF, 0x00000001, 0x00007FFF, 0x00008000, 0x00008001,
                         0x00018000, 0x007FFFFF, 0x807FFFFF, 0x7F7FFFFF, 0x7F7F7FFF,
                         0x7F7F8000, 0xFF7F8000], np.uint32)
    v = np.concatenate([vals, specials])
    v = np.concatenate([v, np.zeros((-v.size) % 64, np.uint32)])
    return v.view(np.float32)


@pytest.mark.parametrize("hw", [4, 3])
def test_bf16_stores_round_every_class(hw):
    """bf16 stores of the convolution's epilogue (staged through LDS when
    rows pack into 8-byte pieces, hw = 4; the lanes' own stores otherwise)
    equal the oracle's cast for every rounding class: with x = 0 each output
    channel is its bias, so the bias vector feeds the encoder chosen values."""
    print(f"bf16 store rounding hw={hw}", flush=True)
    rng = np.random.default_rng(17)
    bias = rounding_classes(rng)
    C_out, C = bias.size, 8
    x = np.zeros((2, C, hw, hw), np.float32)
    w = rng.standard_normal((C_out, C, 1, 1)).astype(np.float32)
    wd, ws, _ = quantized_codes(w, "e4m3", rng)
    y0 = conv_ex(x, wd, "e4m3", ws, w.shape, (1, 1), (0, 0), "zeros", None, bias)
    want = R.epilogue_f32(y0.view(np.float32), None, None, False, axis=1)
    ep = Epi(C_out, rng, relu=False, out="bf16", amax=False, mul=False, add=False)
    got = conv_ex(x, wd, "e4m3", ws, w.shape, (1, 1), (0, 0), "zeros", ep, bias).reshape(-1)
    assert np.array_equal(got, O.cast(want.reshape(-1), O.F32, O.BF16))


LINEAR_CASES = [
    ("e4m3", 256, 512, 256),   # linear_pingpong_kernel
    ("e2m1", 128, 256, 512),   # linear_wide_kernel, FP4
    ("bf16", 128, 128, 256),   # linear_pipe_kernel
    ("f16", 128, 64, 128),     # linear_pipe_kernel, 128-wide tiles
    ("e5m2", 33, 70, 46),      # linear_kernel (ragged)
    ("f32", 64, 96, 40),       # linear_kernel (fp32 weights)
]


@pytest.mark.parametrize("wdt,N,D_in,D_out", LINEAR_CASES)
def test_linear_epilogue_bit_exact(wdt, N, D_in, D_out):
    print(f"linear epilogue {wdt} {N}x{D_in}x{D_out}", flush=True)
    rng = np.random.default_rng(N + D_in + D_out)
    x = rng.standard_normal((N, D_in)).astype(np.float32)
    w = (rng.standard_normal((D_out, D_in)) * np.sqrt(2.0 / D_in)).astype(np.float32)
    bias = rng.standard_normal(D_out).astype(np.float32)
    wd, ws, _ = quantized_codes(w, wdt, rng)
    y0 = linear_ex(x, wd, wdt, ws, D_out, None, bias)
    check_all_outputs(lambda ep: linear_ex(x, wd, wdt, ws, D_out, ep, bias), y0, D_out, rng)


CONV_CASES = [
    # wdt, (N, C, H, W), C_out, (KH, KW), stride, pad, mode
    ("e2m1", (3, 8, 12, 12), 16, (3, 3), (1, 1), (1, 1), "zeros"),     # band, K9
    ("e2m1", (2, 32, 28, 28), 64, (3, 3), (1, 1), (1, 1), "zeros"),   # band, config [5] conv2's bands
    ("e4m3", (2, 5, 10, 11), 20, (5, 5), (1, 1), (2, 2), "reflect"),   # band, generic regroup
    ("bf16", (2, 4, 9, 9), 70, (3, 3), (2, 2), (1, 1), "replicate"),  # band, 2 co blocks
    ("e5m2", (2, 65, 7, 7), 24, (3, 3), (1, 1), (1, 1), "circular"),  # conv2d_kernel (C > 64)
    ("f32", (1, 5, 6, 301), 5, (1, 3), (1, 1), (0, 1), "zeros"),      # conv2d_kernel (OW > 256)
    ("e2m1", (3, 1, 28, 28), 32, (3, 3), (1, 1), (1, 1), "zeros"),    # small-C, vector stores
    ("e4m3", (2, 3, 7, 10), 9, (3, 5), (1, 1), (1, 2), "reflect"),    # small-C, OW % 4 != 0
    # small-C with two 8-channel groups per workgroup and a partial last group
    ("e2m1", (208, 2, 6, 6), 37, (3, 3), (1, 1), (1, 1), "zeros"),
    # one output channel, C no multiple of 8
    ("e4m3", (2, 32, 12, 16), 1, (3, 3), (1, 1), (1, 1), "reflect"),
    ("e2m1", (3, 37, 9, 8), 1, (2, 5), (1, 1), (1, 2), "zeros"),
]


@pytest.mark.parametrize("wdt,xs,C_out,k,stride,pad,mode", CONV_CASES)
def test_conv2d_epilogue_bit_exact(wdt, xs, C_out, k, stride, pad, mode):
    print(f"conv epilogue {wdt} {xs} -> {C_out} k={k} s={stride} p={pad} {mode}", flush=True)
    rng = np.random.default_rng(sum(xs) + C_out)
    x = rng.standard_normal(xs).astype(np.float32)
    wshape = (C_out, xs[1]) + k
    w = (rng.standard_normal(wshape) * np.sqrt(2.0 / (xs[1] * k[0] * k[1]))).astype(np.float32)
    bias = rng.standard_normal(C_out).astype(np.float32)
    wd, ws, _ = quantized_codes(w, wdt, rng)
    y0 = conv_ex(x, wd, wdt, ws, wshape, stride, pad, mode, None, bias)
    check_all_outputs(lambda ep: conv_ex(x, wd, wdt, ws, wshape, stride, pad, mode, ep, bias),
                      y0, C_out, rng)


def test_relu_special_values():
    """ReLU keeps the reference's rules: -0 for negative values, NaN for NaN
    and -Inf, +Inf kept; the amax ignores NaN and takes Inf."""
    rng = np.random.default_rng(11)
    N, D_in, D_out = 64, 64, 8
    x = rng.standard_normal((N, D_in)).astype(np.float32)
    w = rng.standard_normal((D_out, D_in)).astype(np.float32) * 0.1
    wd, ws, _ = quantized_codes(w, "f32", rng)
    add = np.array([np.inf, -np.inf, np.nan, -1e30, 1e30, 0.0, -0.0, -5.0], np.float32)
    y0 = linear_ex(x, wd, "f32", ws, D_out).view(np.float32)
    ep = Epi(D_out, rng, mul=False, add_vals=add)
    y1 = linear_ex(x, wd, "f32", ws, D_out, ep).view(np.float32)
    want = R.epilogue_f32(y0, None, add, True, axis=1)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(y1), nan)
    assert np.array_equal(y1[~nan].view(np.uint32), want[~nan].view(np.uint32))
    assert np.signbit(y1[:, 3]).all() and (y1[:, 3] == 0).all()  # -1e30 -> -0
    assert np.isnan(y1[:, 1]).all()                               # -inf * 0
    assert float(ep.amax.cpu()[0]) == np.inf


def bn_params(C, rng):
    return (rng.uniform(0.5, 1.5, C), rng.standard_normal(C) * 0.1, rng.standard_normal(C) * 0.2,
            rng.uniform(0.5, 2.0, C))


@pytest.mark.parametrize("wdt", ["e2m1", "e4m3"])
def test_conv_bn_relu_matches_reference_path(wdt):
    """Conv2d -> BatchNorm2d (eval) -> ReLU of novann main.py's first block on
    an MNIST-shaped batch, fused, against the reference's formulas in fp64."""
    rng = np.random.default_rng(21)
    x = rng.uniform(0, 1, (64, 1, 28, 28)).astype(np.float32)
    w = (rng.standard_normal((16, 1, 3, 3)) * np.sqrt(2.0 / 9)).astype(np.float32)
    q = QuantizedParameters.from_float(w, wdt)
    wdeq = q.dequantize().cpu().numpy().astype(np.float64).reshape(w.shape)
    g, b, m, v = bn_params(16, rng)
    y = F.conv2d(torch.from_numpy(x).cuda(), q, 3, 1, 1,
                 epilogue=F.Epilogue.batchnorm(g, b, m, v, 1e-5, relu=True))
    ref = R.relu(R.batchnorm_eval(R.conv2d(x.astype(np.float64), wdeq, (1, 1), (1, 1)), g, b, m, v))
    got = y.cpu().numpy()
    assert np.abs(got - ref).max() / np.abs(ref).max() <= TOL


def test_linear_bn_relu_bf16_store_matches_reference_path():
    """Linear -> BatchNorm1d (eval) -> ReLU with a bf16 output (main.py's
    classifier block), against the reference's formulas in fp64."""
    rng = np.random.default_rng(22)
    x = rng.standard_normal((256, 512)).astype(np.float32)
    w = (rng.standard_normal((256, 512)) * np.sqrt(2.0 / 512)).astype(np.float32)
    q = QuantizedParameters.from_float(w, "e4m3")
    wdeq = q.dequantize().cpu().numpy().astype(np.float64).reshape(w.shape)
    g, b, m, v = bn_params(256, rng)
    y = F.linear(torch.from_numpy(x).cuda(), q,
                 epilogue=F.Epilogue.batchnorm(g, b, m, v, 1e-5, relu=True, out_dtype="bf16"))
    assert y.dtype == torch.bfloat16 and y.shape == (256, 256)
    ref = R.relu(R.batchnorm_eval(R.linear(x.astype(np.float64), wdeq), g, b, m, v))
    got = y.float().cpu().numpy()
    assert np.abs(got - ref).max() / np.abs(ref).max() <= TOL


def test_fp8_store_returns_quantized_with_its_scale():
    rng = np.random.default_rng(23)
    x = rng.standard_normal((128, 256)).astype(np.float32)
    w = (rng.standard_normal((256, 256)) * 0.05).astype(np.float32)
    q = QuantizedParameters.from_float(w, "e4m3")
    amax = torch.zeros(1, device="cuda")
    y32 = F.linear(torch.from_numpy(x).cuda(), q, epilogue=F.Epilogue(relu=True, out_amax=amax))
    scale = torch.tensor([float(amax.cpu()[0]) / 448.0], device="cuda")
    y8 = F.linear(torch.from_numpy(x).cuda(), q,
                  epilogue=F.Epilogue(relu=True, out_dtype="e4m3", out_scale=scale))
    assert y8.dtype == "e4m3" and y8.shape == (128, 256)
    want = O.cast(y32.cpu().numpy().reshape(-1), O.F32, O.E4M3, scale=float(scale.cpu()[0]))
    assert np.array_equal(to_host(y8.data), want)


def test_epilogue_rejects_bad_arguments():
    lib = _lib.load()
    x = torch.zeros((4, 8), device="cuda")
    w = torch.zeros((8, 8), device="cuda")
    y = torch.zeros((4, 8), device="cuda")
    bad = _lib.Epilogue(None, None, None, None, 0, _lib.DTYPES["e2m1"])
    assert lib.novaq_linear_forward_ex(x.data_ptr(), O.F32, None, 4, 8, w.data_ptr(), O.F32,
                                       None, None, 8, ctypes.byref(bad), y.data_ptr(),
                                       stream()) == _lib.EDTYPE


# --- inputs stored by an epilogue: x in bf16 / f16 / E4M3 / E5M2 ------------

def x_codes(x, xt):
    """Device codes of x in xt, its scale (FP8; None otherwise) and the
    unscaled fp32 decode of the codes."""
    c = OUT[xt]
    if xt in ("e4m3", "e5m2"):
        s = O.scale_from_amax(O.amax(x), c)
        codes = O.cast(x.reshape(-1), O.F32, c, scale=s)
        return to_dev(codes, c), s, O.cast(codes, c, O.F32, n=x.size).reshape(x.shape)
    codes = O.cast(x.reshape(-1), O.F32, c)
    return to_dev(codes, c), None, O.cast(codes, c, O.F32).reshape(x.shape)


def combined_scale(ws, sx):
    """Device scale s_w * s_x rounded as the kernels form it (fp32)."""
    sw = 1.0 if ws is None else float(ws.cpu()[0])
    if sx is None:
        return ws
    return torch.tensor([np.float32(sw) * np.float32(sx)], dtype=torch.float32, device="cuda")


def linear_x(xd, xt, sx, N, D_in, wd, wdt, ws, D_out, bias):
    y = torch.empty((N, D_out), dtype=torch.float32, device="cuda")
    sxd = None if sx is None else torch.tensor([sx], dtype=torch.float32, device="cuda")
    bd = torch.from_numpy(bias).cuda()
    _lib.check(_lib.load().novaq_linear_forward_ex(
        xd.data_ptr(), OUT[xt], None if sxd is None else sxd.data_ptr(), N, D_in, wd.data_ptr(),
        _lib.DTYPES[wdt], None if ws is None else ws.data_ptr(), bd.data_ptr(), D_out, None,
        y.data_ptr(), stream()), "linear_ex")
    torch.cuda.synchronize()
    return to_host(y)


@pytest.mark.parametrize("xt", ["bf16", "f16", "e4m3", "e5m2"])
@pytest.mark.parametrize("wdt,N,D_in,D_out", LINEAR_CASES)
def test_linear_reads_stored_activations(xt, wdt, N, D_in, D_out):
    """A product on x stored as xt equals the fp32-input product on the
    decoded x with the scale folded into the weight scale: bit for bit for
    bf16 / f16 x (the same operands and order).  FP8 x on the FP8 product path
    multiplies its codes directly: the same exact products, summed by the
    FP8 MFMA (whose sums are not rounded as fp32 additions are: ~1e-5
    normwise at these sizes), so within 1e-4."""
    print(f"linear x={xt} {wdt} {N}x{D_in}x{D_out}", flush=True)
    rng = np.random.default_rng(N * 3 + D_in + D_out)
    x = rng.standard_normal((N, D_in)).astype(np.float32)
    w = (rng.standard_normal((D_out, D_in)) * np.sqrt(2.0 / D_in)).astype(np.float32)
    bias = rng.standard_normal(D_out).astype(np.float32)
    wd, ws, _ = quantized_codes(w, wdt, rng)
    xd, sx, xdec = x_codes(x, xt)
    got = linear_x(xd, xt, sx, N, D_in, wd, wdt, ws, D_out, bias)
    want = linear_x(torch.from_numpy(np.ascontiguousarray(xdec)).cuda(), "f32", None, N, D_in,
                    wd, wdt, combined_scale(ws, sx), D_out, bias)
    fp8_path = (xt in ("e4m3", "e5m2") and wdt in ("e4m3", "e5m2", "e2m1") and N % 128 == 0
                and D_out % 256 == 0 and D_in % 128 == 0)
    if fp8_path:
        g, r = got.view(np.float32).astype(np.float64), want.view(np.float32).astype(np.float64)
        err = np.abs(g - r).max() / np.abs(r).max()
        assert err <= 1e-4, err
    else:
        assert np.array_equal(got, want)


def conv_x(xd, xt, sx, xs, wd, wdt, ws, wshape, stride, pad, mode, bias):
    N, C, H, W = xs
    C_out, _, KH, KW = wshape
    OH, OW = (H + 2 * pad[0] - KH) // stride[0] + 1, (W + 2 * pad[1] - KW) // stride[1] + 1
    y = torch.empty((N, C_out, OH, OW), dtype=torch.float32, device="cuda")
    sxd = None if sx is None else torch.tensor([sx], dtype=torch.float32, device="cuda")
    bd = torch.from_numpy(bias).cuda()
    _lib.check(_lib.load().novaq_conv2d_forward_ex(
        xd.data_ptr(), OUT[xt], None if sxd is None else sxd.data_ptr(), N, C, H, W,
        wd.data_ptr(), _lib.DTYPES[wdt], None if ws is None else ws.data_ptr(), C_out, KH, KW,
        stride[0], stride[1], pad[0], pad[1], _lib.PAD_MODES[mode], bd.data_ptr(), None,
        y.data_ptr(), stream()), "conv2d_ex")
    torch.cuda.synchronize()
    return to_host(y)


@pytest.mark.parametrize("xt", ["bf16", "f16", "e4m3", "e5m2"])
@pytest.mark.parametrize("wdt,xs,C_out,k,stride,pad,mode", CONV_CASES)
def test_conv2d_reads_stored_activations(xt, wdt, xs, C_out, k, stride, pad, mode):
    print(f"conv x={xt} {wdt} {xs} -> {C_out} k={k} s={stride} p={pad} {mode}", flush=True)
    rng = np.random.default_rng(sum(xs) * 3 + C_out)
    x = rng.standard_normal(xs).astype(np.float32)
    wshape = (C_out, xs[1]) + k
    w = (rng.standard_normal(wshape) * np.sqrt(2.0 / (xs[1] * k[0] * k[1]))).astype(np.float32)
    bias = rng.standard_normal(C_out).astype(np.float32)
    wd, ws, _ = quantized_codes(w, wdt, rng)
    xd, sx, xdec = x_codes(x, xt)
    got = conv_x(xd, xt, sx, xs, wd, wdt, ws, wshape, stride, pad, mode, bias)
    want = conv_x(torch.from_numpy(np.ascontiguousarray(xdec)).cuda(), "f32", None, xs, wd, wdt,
                  combined_scale(ws, sx), wshape, stride, pad, mode, bias)
    assert np.array_equal(got, want)


def test_main_py_blocks_chained_through_narrow_activations():
    """novann main.py:24-38 (conv+BN+ReLU, conv s2+BN+ReLU, conv+BN+ReLU) on
    an MNIST-shaped batch: block 1 stores bf16, block 2 reads it and stores
    E4M3 (scale from a calibration pass's amax), block 3 reads that.  Each
    block's output is within 1e-2 of the reference formulas (fp64) applied
    to the activation it actually read."""
    rng = np.random.default_rng(31)
    N = 64
    x = rng.uniform(0, 1, (N, 1, 28, 28)).astype(np.float32)
    specs = [(1, 16, 1), (16, 32, 2), (32, 64, 1)]
    layers = []
    for cin, cout, st in specs:
        w = (rng.standard_normal((cout, cin, 3, 3)) * np.sqrt(2.0 / (cin * 9))).astype(np.float32)
        q = QuantizedParameters.from_float(w, "e2m1")
        wdeq = q.dequantize().cpu().numpy().astype(np.float64).reshape(w.shape)
        layers.append((q, wdeq, st, bn_params(cout, rng)))

    def ref_block(a, i):
        q, wdeq, st, (g, b, m, v) = layers[i]
        return R.relu(R.batchnorm_eval(R.conv2d(a, wdeq, (st, st), (1, 1)), g, b, m, v))

    def gpu_block(a, i, **kw):
        q, _, st, (g, b, m, v) = layers[i]
        return F.conv2d(a, q, 3, st, 1, epilogue=F.Epilogue.batchnorm(g, b, m, v, 1e-5,
                                                                      relu=True, **kw))

    y1 = gpu_block(torch.from_numpy(x).cuda(), 0, out_dtype="bf16")
    assert y1.dtype == torch.bfloat16
    r1 = ref_block(x.astype(np.float64), 0)
    a1 = y1.float().cpu().numpy()
    assert np.abs(a1 - r1).max() / np.abs(r1).max() <= TOL
    # block 2 on the bf16 activation: calibrate its amax in fp32, then store E4M3
    amax = torch.zeros(1, device="cuda")
    gpu_block(y1, 1, out_amax=amax)
    scale = torch.tensor([float(amax.cpu()[0]) / 448.0], device="cuda")
    y2 = gpu_block(y1, 1, out_dtype="e4m3", out_scale=scale)
    r2 = ref_block(a1.astype(np.float64), 1)
    a2 = F_dequant(y2)
    # E4M3 storage rounds each value to 3 mantissa bits: up to 2^-4 of it
    assert np.abs(a2 - r2).max() / np.abs(r2).max() <= 2.0 ** -4 + TOL
    # block 3 reads the E4M3 activation with its scale
    y3 = gpu_block(y2, 2)
    r3 = ref_block(a2.astype(np.float64), 2)
    a3 = y3.cpu().numpy()
    assert np.abs(a3 - r3).max() / np.abs(r3).max() <= TOL


def F_dequant(q):
    from novann_amd import quant
    return quant.dequantize(q).cpu().numpy()


def test_fused_layers_from_the_module_api():
    """novann main.py:24-46's blocks built from this package's layers and
    fused (conv+BN+ReLU x2 with bf16 activations, then a Linear+BN1d+ReLU on
    a pooled vector), against the reference formulas in fp64."""
    from novann_amd import module as M
    rng = np.random.default_rng(41)
    conv1 = M.Conv2d(1, 16, 3, padding=1, bias=False, weight_dtype="e2m1")
    conv2 = M.Conv2d(16, 32, 3, padding=1, stride=2, bias=False, weight_dtype="e2m1")
    bns = [M.BatchNorm2d(16), M.BatchNorm2d(32)]
    for bn in bns:
        g, b, m, v = bn_params(bn.num_features, rng)
        bn.gamma.data = g.reshape(bn.gamma.data.shape)
        bn.beta.data = b.reshape(bn.beta.data.shape)
        bn.running_mean = m.reshape(bn.running_mean.shape)
        bn.running_var = v.reshape(bn.running_var.shape)
    block1 = M.fuse(conv1, bns[0], M.ReLU(), out_dtype="bf16")
    block2 = M.fuse(conv2, bns[1], M.ReLU())
    x = rng.uniform(0, 1, (32, 1, 28, 28)).astype(np.float32)
    y1 = block1(torch.from_numpy(x).cuda())
    y2 = block2(y1)
    assert y1.dtype == torch.bfloat16 and tuple(y2.shape) == (32, 32, 14, 14)

    def ref(a, conv, bn):
        wdeq = conv.weight.dequantize().cpu().numpy().astype(np.float64).reshape(conv.weight.shape)
        return R.relu(R.batchnorm_eval(R.conv2d(a, wdeq, (conv.sh, conv.sw), (conv.ph, conv.pw)),
                                       bn.gamma.data, bn.beta.data, bn.running_mean,
                                       bn.running_var, bn.eps))
    a1 = y1.float().cpu().numpy()
    r1 = ref(x.astype(np.float64), conv1, bns[0])
    assert np.abs(a1 - r1).max() / np.abs(r1).max() <= TOL
    r2 = ref(a1.astype(np.float64), conv2, bns[1])
    got = y2.cpu().numpy()
    assert np.abs(got - r2).max() / np.abs(r2).max() <= TOL
    # classifier block: Linear(32 -> 16, no bias) + BatchNorm1d + ReLU on pooled features
    lin = M.Linear(32, 16, bias=False, weight_dtype="e4m3")
    bn1 = M.BatchNorm1d(16)
    g, b, m, v = bn_params(16, rng)
    bn1.gamma.data, bn1.beta.data = g.reshape(1, 16), b.reshape(1, 16)
    bn1.running_mean, bn1.running_var = m.reshape(1, 16), v.reshape(1, 16)
    feat = got.mean(axis=(2, 3)).astype(np.float32)
    out = M.fuse(lin, bn1, M.ReLU())(feat)
    wdeq = lin.weight.dequantize().cpu().numpy().astype(np.float64).reshape(16, 32)
    r3 = R.relu(R.batchnorm_eval(R.linear(feat.astype(np.float64), wdeq), g, b, m, v))
    assert isinstance(out, np.ndarray) and out.shape == (32, 16)
    assert np.abs(out - r3).max() / np.abs(r3).max() <= TOL
