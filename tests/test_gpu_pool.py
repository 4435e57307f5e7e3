"""MaxPool2d and GlobalAvgPool2d on the GPU (through the C ABI and the layers)
vs the restatement of novann.functional.max_pool2d / avg_pool2d
(functional.py:450-559): bit-exact (the window max is one of the inputs, and
the mean is evaluated in numpy's pairwise float32 order); a NaN result is
compared as NaN (numpy's own loops differ on its payload)."""
import numpy as np
import pytest
import torch

import oracle as O
from oracle import functional_ref as R
from novann_amd import _lib
from novann_amd import functional as F
from novann_amd import module as M
from novann_amd import quant
from tests.gpu_util import to_dev, to_host

pytestmark = pytest.mark.gpu

CODE = {"f32": O.F32, "f16": O.F16, "bf16": O.BF16, "e4m3": O.E4M3, "e5m2": O.E5M2}
STORE = {"f32": np.uint32, "f16": np.uint16, "bf16": np.uint16, "e4m3": np.uint8,
         "e5m2": np.uint8}


def same_bits_or_nan(got, want):
    g, w = got.view(np.float32), want.view(np.float32)
    nan = np.isnan(w)
    assert np.array_equal(np.isnan(g), nan)
    assert np.array_equal(g[~nan].view(np.uint32), w[~nan].view(np.uint32))


def relu_like(rng, shape):
    """Post-ReLU activations: many -0 (negative inputs) and a few +0 and NaN."""
    x = rng.standard_normal(shape).astype(np.float32)
    x = R.relu(x)
    flat = x.reshape(-1)
    flat[rng.integers(0, flat.size, flat.size // 50)] = 0.0
    flat[rng.integers(0, flat.size, 3)] = np.nan
    return x


GEOMS = [
    ((4, 3, 10, 10), (2, 2), (2, 2), (0, 0), "zeros"),      # reference test shape
    ((2, 4, 5, 5), (3, 3), (1, 1), (1, 1), "zeros"),        # reference padding test
    ((2, 3, 9, 11), (3, 2), (2, 1), (2, 1), "reflect"),
    ((1, 5, 7, 6), (2, 3), (1, 2), (1, 0), "replicate"),
    ((3, 2, 8, 8), (3, 3), (2, 2), (1, 2), "circular"),
    ((128, 32, 14, 14), (2, 2), (2, 2), (0, 0), "zeros"),   # main.py:35 (block 2 output)
    ((2, 3, 8, 12), (2, 2), (2, 2), (0, 0), "zeros"),       # 2-wide path, vector loads
    ((2, 2, 9, 16), (3, 2), (1, 2), (1, 0), "reflect"),     # 2-wide path, padded rows
    ((1, 2, 6, 7), (2, 2), (2, 2), (0, 0), "zeros"),        # 2-wide path, odd OW
]


@pytest.mark.parametrize("xs,k,s,p,mode", GEOMS)
def test_max_pool2d_f32_bit_exact(xs, k, s, p, mode):
    print(f"max_pool2d {xs} k={k} s={s} p={p} {mode}", flush=True)
    rng = np.random.default_rng(sum(xs))
    x = relu_like(rng, xs)
    got = F.max_pool2d(x, k, s, p, mode)
    assert isinstance(got, np.ndarray) and got.dtype == np.float32
    same_bits_or_nan(got, R.max_pool2d(x, k, s, p, mode))


@pytest.mark.parametrize("xt,off_x,off_y", [("f32", 1, 0), ("f32", 2, 1), ("bf16", 1, 1),
                                             ("e4m3", 3, 1)])
def test_max_pool2d_element_offset_views(xt, off_x, off_y):
    """x and y as views starting some elements into larger buffers (W % 4 == 0,
    OW even: the shape that reads 4 elements and stores pairs at once)."""
    print(f"max_pool2d views {xt} +{off_x} +{off_y}", flush=True)
    rng = np.random.default_rng(off_x * 10 + off_y)
    shape, oshape = (2, 3, 8, 12), (2, 3, 4, 6)
    n, no = int(np.prod(shape)), int(np.prod(oshape))
    v = relu_like(rng, (n + off_x,))
    codes = v.view(np.uint32) if xt == "f32" else O.cast(v, O.F32, CODE[xt])
    xbuf = to_dev(codes, CODE[xt])
    ybuf = torch.empty(no + off_y, dtype=xbuf.dtype, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = _lib.load().novaq_max_pool2d(xbuf[off_x:].data_ptr(), CODE[xt], *shape, 2, 2, 2, 2,
                                      0, 0, 0, ybuf[off_y:].data_ptr(), stream)
    assert rc == _lib.OK
    torch.cuda.synchronize()
    got = O.cast(to_host(ybuf[off_y:]), CODE[xt], O.F32).reshape(oshape)
    dec = O.cast(codes[off_x:], CODE[xt], O.F32, n=n).reshape(shape)
    same_bits_or_nan(got, R.max_pool2d(dec, 2, 2, 0, "zeros"))


@pytest.mark.parametrize("ksp", [(3, 2, 1), (2, 2, 0)])
@pytest.mark.parametrize("xt", ["bf16", "f16", "e4m3", "e5m2"])
def test_max_pool2d_narrow_codes(xt, ksp):
    """Pooling codes equals encoding the pooled decoded values (the max is
    one of the inputs); FP8 keeps its scale."""
    rng = np.random.default_rng(3)
    xs = (4, 6, 12, 12)
    x = relu_like(rng, xs)
    x[np.isnan(x)] = 1.0
    scale = 0.01 if xt in ("e4m3", "e5m2") else None
    codes = O.cast(x.reshape(-1), O.F32, CODE[xt], **({"scale": scale} if scale else {}))
    dec = O.cast(codes, CODE[xt], O.F32).reshape(xs)
    xd = to_dev(codes, CODE[xt]).view(xs)
    if scale:
        xd = quant.Quantized(xd, xs, xt, torch.tensor([scale], dtype=torch.float32,
                                                       device="cuda"))
    k, st, pd = ksp
    y = F.max_pool2d(xd, k, st, pd, "zeros")
    want = R.max_pool2d(dec, k, st, pd, "zeros")
    ycodes = to_host(y.data if scale else y).reshape(-1)
    assert np.array_equal(O.cast(ycodes, CODE[xt], O.F32).view(np.uint32),
                          want.reshape(-1).view(np.uint32))
    if scale:
        assert y.shape == want.shape and float(y.scale.cpu()[0]) == np.float32(scale)


# (2, 3, 89, 89), (1, 2, 90, 90), (1, 3, 1, 8191), (1, 1, 87, 89): planes whose
# numpy pairwise tree has 65 leaves; (2, 2, 64, 128): one whole 8192 block;
# 7 x 7, 14 x 14, 20 x 20 and 28 x 28: complete trees of 1, 2, 4 and 8 leaves
# (leaf sums added by shuffles)
@pytest.mark.parametrize("xs", [(2, 3, 4, 5), (4, 3, 10, 12), (128, 64, 7, 7), (3, 2, 1, 7),
                                (2, 2, 14, 14), (1, 3, 28, 28), (8, 64, 28, 28), (3, 5, 20, 20),
                                (2, 2, 37, 41), (1, 1, 128, 129),
                                (2, 3, 89, 89), (1, 2, 90, 90), (1, 3, 1, 8191), (1, 1, 87, 89),
                                (2, 2, 64, 128)])
def test_avg_pool2d_bit_exact(xs):
    print(f"avg_pool2d {xs}", flush=True)
    rng = np.random.default_rng(sum(xs))
    x = (rng.standard_normal(xs) * np.exp2(rng.integers(-8, 8, xs))).astype(np.float32)
    got = F.avg_pool2d(x)
    want = R.avg_pool2d(x)
    assert got.shape == (xs[0], xs[1], 1, 1)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


# plane sizes for every load width the GAP kernels pick (hw odd, 2 mod 4,
# 4 mod 8, 0 mod 8), trees 0 to 7 levels deep, leaves at unequal depths (250,
# 1000, 5000), a remainder in the last leaf (196, 52), planes whose tree is too
# deep for one wave's lanes (6400, 8192 for 4-byte x; odd sizes above 1000
# for all: the one-wave-per-plane kernel, in 2 to 16 passes) and planes of
# several numpy blocks (8193 on: whole blocks, then a short one)
GAP_HW = [1, 2, 3, 4, 6, 8, 12, 16, 49, 50, 52, 64, 100, 129, 196, 250, 256, 392, 784, 1000,
          1001, 1024, 2048, 3136, 4096, 5000, 6400, 7689, 7921, 8192, 8193, 9001, 12544, 16384,
          24577, 50176]


@pytest.mark.parametrize("xt", ["f32", "bf16", "f16", "e4m3", "e5m2"])
def test_avg_pool2d_plane_sizes(xt):
    """np.mean of the decoded (and, E4M3, scaled) planes bit for bit over
    GAP_HW, 38 planes each (several planes per wave and a partial last wave);
    plane 0 is all -0.0, whose mean numpy makes +0.0."""
    rng = np.random.default_rng(len(xt))
    for hw in GAP_HW:
        print(f"avg_pool2d {xt} hw={hw}", flush=True)
        shape = (2, 19, 1, hw)
        x = (rng.standard_normal(shape) * np.exp2(rng.integers(-6, 6, shape))).astype(np.float32)
        x[0, 0] = -0.0
        if xt == "f32":
            got = F.avg_pool2d(torch.from_numpy(x).cuda()).cpu().numpy()
            want = R.avg_pool2d(x)
        else:
            scale = 0.75 if xt == "e4m3" else None
            codes = O.cast(x.reshape(-1), O.F32, CODE[xt], scale=scale)
            dev = to_dev(codes, CODE[xt])
            arg = (quant.Quantized(dev, shape, xt, torch.tensor([scale], device="cuda"))
                   if scale else dev.view(shape))
            got = F.avg_pool2d(arg).cpu().numpy()
            dec = O.cast(codes, CODE[xt], O.F32, n=x.size, scale=scale).reshape(shape)
            want = R.avg_pool2d(dec)
        assert np.array_equal(got.reshape(-1).view(np.uint32), want.reshape(-1).view(np.uint32)), \
            (xt, hw)


def test_avg_pool2d_known_answer_and_narrow_input():
    """test_gap2d.py:20-27's constant input; bf16 and scaled E4M3 inputs equal
    np.mean of the dequantized arrays."""
    x = np.ones((2, 3, 4, 5), np.float32) * 3.0
    assert np.array_equal(F.avg_pool2d(x), np.full((2, 3, 1, 1), 3.0, np.float32))
    rng = np.random.default_rng(4)
    y = rng.standard_normal((8, 16, 7, 7)).astype(np.float32)
    b = O.cast(y.reshape(-1), O.F32, O.BF16)
    got = F.avg_pool2d(to_dev(b, O.BF16).view(8, 16, 7, 7))
    want = R.avg_pool2d(O.cast(b, O.BF16, O.F32).reshape(y.shape))
    assert np.array_equal(got.cpu().numpy().view(np.uint32), want.view(np.uint32))
    s = O.scale_from_amax(O.amax(y), O.E4M3)
    q = O.cast(y.reshape(-1), O.F32, O.E4M3, scale=s)
    qa = quant.Quantized(to_dev(q, O.E4M3), y.shape, "e4m3",
                         torch.tensor([s], dtype=torch.float32, device="cuda"))
    got = F.avg_pool2d(qa)
    deq = O.cast(q, O.E4M3, O.F32, n=y.size, scale=s).reshape(y.shape)
    assert np.array_equal(got.cpu().numpy().view(np.uint32), R.avg_pool2d(deq).view(np.uint32))


@pytest.mark.parametrize("xt,off", [("f32", 1), ("f32", 3), ("bf16", 2), ("e4m3", 5)])
def test_avg_pool2d_offset_views(xt, off):
    """x as a view some elements into a larger buffer: the C ABI refuses it
    (NOVAQ_EALIGN: the plane loads are 4-element vectors), the host layer
    copies it to an aligned buffer and returns the same bits as the aligned
    call."""
    print(f"avg_pool2d view {xt} +{off}", flush=True)
    rng = np.random.default_rng(off)
    shape = (3, 5, 6, 7)
    n = int(np.prod(shape))
    v = rng.standard_normal(n + off).astype(np.float32)
    codes = v.view(np.uint32) if xt == "f32" else O.cast(v, O.F32, CODE[xt])
    buf = to_dev(codes, CODE[xt])
    view = buf[off:off + n]
    y = torch.empty(shape[:2], device="cuda")
    rc = _lib.load().novaq_global_avg_pool2d(view.data_ptr(), CODE[xt], None, *shape,
                                             y.data_ptr(), torch.cuda.current_stream().cuda_stream)
    assert rc == _lib.EALIGN
    scale = torch.ones(1, device="cuda")
    arg = quant.Quantized(view, shape, xt, scale) if xt == "e4m3" else view.view(shape)
    got = F.avg_pool2d(arg).cpu().numpy()
    dec = O.cast(codes[off:], CODE[xt], O.F32, n=n).reshape(shape)
    assert np.array_equal(got.view(np.uint32), R.avg_pool2d(dec).view(np.uint32))


def test_layers_like_reference():
    """test_maxpooling2d.py:10-27 and test_gap2d.py:10-17 on the layers."""
    rng = np.random.RandomState(8)
    x = rng.randn(4, 3, 10, 10).astype(np.float32)
    assert M.MaxPool2d(kernel_size=2, stride=2, padding=0)(x).shape == (4, 3, 5, 5)
    assert M.MaxPool2d(kernel_size=3, stride=1, padding=1)(x[:2, :, :5, :5]).shape == (2, 3, 5, 5)
    assert M.MaxPool2d(2)(x).shape == (4, 3, 5, 5)  # stride defaults to the kernel size
    assert M.GlobalAvgPool2d()(rng.randn(4, 3, 10, 12).astype(np.float32)).shape == (4, 3, 1, 1)


def test_main_py_pool_path_with_fused_bf16_activations():
    """main.py:30-42: conv(s2)+BN+ReLU stored bf16 -> MaxPool2d(2, 2) on the
    bf16 codes -> conv+BN+ReLU -> GlobalAvgPool2d, each stage equal to the
    reference's functions applied to what it actually read."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((32, 16, 28, 28)).astype(np.float32)
    c2 = M.Conv2d(16, 32, 3, stride=2, padding=1, bias=False, weight_dtype="e2m1")
    c3 = M.Conv2d(32, 64, 3, padding=1, bias=False, weight_dtype="e2m1")
    b2, b3 = M.BatchNorm2d(32), M.BatchNorm2d(64)
    a = M.fuse(c2, b2, M.ReLU(), out_dtype="bf16")(torch.from_numpy(x).cuda())
    p = M.MaxPool2d(2, 2)(a)
    assert p.dtype == torch.bfloat16 and tuple(p.shape) == (32, 32, 7, 7)
    a_host = a.float().cpu().numpy()
    same_bits_or_nan(p.float().cpu().numpy(), R.max_pool2d(a_host, 2, 2))
    h = M.fuse(c3, b3, M.ReLU())(p)
    g = M.GlobalAvgPool2d()(h)
    assert np.array_equal(g.cpu().numpy().view(np.uint32),
                          R.avg_pool2d(h.cpu().numpy()).view(np.uint32))
