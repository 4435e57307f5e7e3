"""MaxPool2d and GlobalAvgPool2d backward on the GPU (through the C ABI and the
layers) vs the restatement of MaxPool2d.backward
(layers/pooling/maxpool/maxpool2d.py:79-129) and GlobalAvgPool2d.backward
(layers/pooling/gap/global_avg_pool2d.py:35-57): bit for bit, a NaN compared
as NaN.  The inputs carry ties (-0 / +0 and repeated values, so grads split
two to four ways), NaN windows, and +-inf / NaN grads."""
import numpy as np
import pytest
import torch

import oracle as O
from oracle import functional_ref as R
from novann_amd import _lib
from novann_amd import functional as F
from novann_amd import module as M
from novann_amd import quant
from tests.gpu_util import to_dev

pytestmark = pytest.mark.gpu

CODE = {"f32": O.F32, "f16": O.F16, "bf16": O.BF16, "e4m3": O.E4M3, "e5m2": O.E5M2}


def same_bits_or_nan(got, want):
    g, w = np.asarray(got, np.float32), np.asarray(want, np.float32)
    assert g.shape == w.shape
    nan = np.isnan(w)
    assert np.array_equal(np.isnan(g), nan)
    assert np.array_equal(g[~nan].view(np.uint32), w[~nan].view(np.uint32))


def tied(rng, shape):
    """Post-ReLU-like values on a coarse grid: many -0 / +0 and repeated
    values (ties), and a few NaN."""
    x = rng.choice(np.array([-0.0, 0.0, 0.0, 0.5, 1.0, 1.0, 2.0, -1.5], np.float32), shape)
    flat = x.reshape(-1)
    flat[rng.integers(0, flat.size, 3)] = np.nan
    return x


def grads(rng, shape):
    g = rng.standard_normal(shape).astype(np.float32)
    flat = g.reshape(-1)
    flat[rng.integers(0, flat.size, 2)] = np.inf
    flat[rng.integers(0, flat.size, 2)] = -np.inf
    flat[rng.integers(0, flat.size, 2)] = np.nan
    return g


GEOMS = [
    ((2, 3, 6, 6), (2, 2), (2, 2), (0, 0), "zeros"),        # the reference's gradient check
    ((256, 64, 28, 28), (2, 2), (2, 2), (0, 0), "zeros"),   # config [5]-sized activations
    ((2, 4, 5, 5), (3, 3), (1, 1), (1, 1), "zeros"),        # overlapping windows
    ((2, 3, 9, 11), (3, 2), (2, 1), (2, 1), "reflect"),
    ((1, 5, 7, 6), (2, 3), (1, 2), (1, 0), "replicate"),
    ((3, 2, 8, 8), (3, 3), (2, 2), (1, 2), "circular"),
    ((2, 3, 7, 9), (2, 2), (2, 2), (0, 0), "zeros"),        # odd H, W: uncovered last row/col
    ((2, 2, 6, 10), (2, 2), (2, 2), (1, 1), "zeros"),       # 2x2 with padding: general kernel
    ((1, 2, 5, 4), (5, 4), (1, 1), (0, 0), "zeros"),        # one window over the plane
]


@pytest.mark.parametrize("xs,k,s,p,mode", GEOMS, ids=lambda v: str(v).replace(" ", ""))
def test_max_pool2d_backward_f32_bit_exact(xs, k, s, p, mode):
    print(f"max_pool2d_backward {xs} k={k} s={s} p={p} {mode}", flush=True)
    rng = np.random.default_rng(sum(xs) + sum(k))
    x = tied(rng, xs)
    OH = (xs[2] + 2 * p[0] - k[0]) // s[0] + 1
    OW = (xs[3] + 2 * p[1] - k[1]) // s[1] + 1
    g = grads(rng, (xs[0], xs[1], OH, OW))
    got = F.max_pool2d_backward(g, x, k, s, p, mode)
    assert isinstance(got, np.ndarray) and got.dtype == np.float32
    same_bits_or_nan(got, R.max_pool2d_backward(g, x, k, s, p, mode))


@pytest.mark.parametrize("ksp", [(2, 2, 0), (3, 1, 1)])
@pytest.mark.parametrize("xt", ["bf16", "f16", "e4m3", "e5m2"])
def test_max_pool2d_backward_narrow_inputs(xt, ksp):
    """x as a fused epilogue stores it: windows compared on the stored codes'
    values (FP8 with a positive scale: the same order and ties)."""
    print(f"max_pool2d_backward {xt} {ksp}", flush=True)
    rng = np.random.default_rng(4)
    xs = (4, 6, 12, 12)
    x = tied(rng, xs)
    x[np.isnan(x)] = 1.0
    scale = 0.01 if xt in ("e4m3", "e5m2") else None
    codes = O.cast(x.reshape(-1), O.F32, CODE[xt], **({"scale": scale} if scale else {}))
    dec = O.cast(codes, CODE[xt], O.F32).reshape(xs)
    xd = to_dev(codes, CODE[xt]).view(xs)
    if scale:
        xd = quant.Quantized(xd, xs, xt, torch.tensor([scale], dtype=torch.float32,
                                                       device="cuda"))
    k, st, pd = ksp
    OH = (12 + 2 * pd - k) // st + 1
    g = grads(rng, (4, 6, OH, OH))
    got = F.max_pool2d_backward(torch.from_numpy(g).cuda(), xd, k, st, pd)
    assert got.dtype == torch.float32 and tuple(got.shape) == xs
    same_bits_or_nan(got.cpu().numpy(), R.max_pool2d_backward(g, dec, k, st, pd))


@pytest.mark.parametrize("xs", [(2, 3, 6, 6), (1, 2, 4, 5), (3, 5, 7, 7), (2, 3, 1, 3),
                                (256, 64, 28, 28), (128, 64, 7, 7)])
def test_global_avg_pool2d_backward_bit_exact(xs):
    """H*W a multiple of 4 (16-byte stores) and not; the reference's uniform
    1/(4*5) gradient (test_gap2d.py:54-70)."""
    print(f"avg_pool2d_backward {xs}", flush=True)
    rng = np.random.default_rng(sum(xs))
    g = grads(rng, (xs[0], xs[1], 1, 1))
    got = F.avg_pool2d_backward(g, xs)
    assert isinstance(got, np.ndarray) and got.shape == xs
    same_bits_or_nan(got, R.global_avg_pool2d_backward(g, xs))
    ones = F.avg_pool2d_backward(np.ones((1, 2, 1, 1), np.float32), (1, 2, 4, 5))
    assert np.all(ones == np.float32(0.05))


def test_layers_forward_backward_like_reference():
    """The reference's layer gradient checks (test_maxpooling2d.py:30-50,
    test_gap2d.py:30-51) as bit-exact comparisons with the restatement, and
    the cache released by MaxPool2d.backward (maxpool2d.py:123)."""
    rng = np.random.RandomState(8)
    x = (rng.randn(2, 3, 6, 6) * 0.1).astype(np.float32)
    mp = M.MaxPool2d(kernel_size=2, stride=2, padding=0)
    y = mp(x)
    G = (rng.randn(*y.shape) * 0.1).astype(np.float32)
    same_bits_or_nan(mp.backward(G), R.max_pool2d_backward(G, x, 2, 2))
    with pytest.raises(RuntimeError):
        mp.backward(G)
    gap = M.GlobalAvgPool2d()
    out = gap(x)
    G2 = (rng.randn(*out.shape) * 0.1).astype(np.float32)
    same_bits_or_nan(gap.backward(G2), R.global_avg_pool2d_backward(G2, x.shape))


def test_c_abi_refusals():
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    g = torch.zeros(64, device="cuda")
    x = torch.zeros(256, device="cuda")
    gi = torch.full((256,), np.nan, device="cuda")
    args = (1, 1, 16, 16, 2, 2, 2, 2, 0, 0)
    assert lib.novaq_max_pool2d_backward(g.data_ptr(), x.data_ptr(), _lib.E2M1, *args, 0,
                                         gi.data_ptr(), st) == _lib.EDTYPE
    assert lib.novaq_max_pool2d_backward(g.data_ptr(), x.data_ptr(), _lib.F32, *args, 9,
                                         gi.data_ptr(), st) == _lib.EPADMODE
    assert lib.novaq_max_pool2d_backward(g.data_ptr() + 2, x.data_ptr(), _lib.F32, *args, 0,
                                         gi.data_ptr(), st) == _lib.EALIGN
    assert lib.novaq_max_pool2d_backward(g.data_ptr(), x.data_ptr(), _lib.F32, 1, 1, 1, 1, 2, 2,
                                         1, 1, 0, 0, 0, gi.data_ptr(), st) == _lib.ESHAPE
    assert lib.novaq_global_avg_pool2d_backward(g.data_ptr(), 1, 1, 16, 16, gi.data_ptr() + 1,
                                                st) == _lib.EALIGN
    assert lib.novaq_global_avg_pool2d_backward(g.data_ptr(), 1, 0, 16, 16, gi.data_ptr(),
                                                st) == _lib.EINVAL
    torch.cuda.synchronize()
    assert torch.isnan(gi).all()  # nothing launched


@pytest.mark.parametrize("xt,off_x,off_g,off_gi", [("f32", 1, 0, 0), ("f32", 0, 1, 2),
                                                    ("f32", 3, 1, 1), ("bf16", 1, 0, 3),
                                                    ("e4m3", 3, 1, 0)])
def test_max_pool2d_backward_element_offset_views(xt, off_x, off_g, off_gi):
    """x, grad and grad_input as views some elements into larger buffers on a
    2x2 stride-2 map: buffers the vector path cannot take run the general
    kernel, with the same bits."""
    print(f"max_pool2d_backward views {xt} +{off_x} +{off_g} +{off_gi}", flush=True)
    rng = np.random.default_rng(off_x * 100 + off_g * 10 + off_gi)
    shape, oshape = (2, 3, 8, 12), (2, 3, 4, 6)
    n, no = int(np.prod(shape)), int(np.prod(oshape))
    v = tied(rng, (n + off_x,))
    v[np.isnan(v)] = 0.5
    codes = v.view(np.uint32) if xt == "f32" else O.cast(v, O.F32, CODE[xt])
    dec = (v if xt == "f32" else O.cast(codes, CODE[xt], O.F32))[off_x:].reshape(shape)
    xbuf = to_dev(codes, CODE[xt])
    g = grads(rng, (no + off_g,))
    gbuf = torch.from_numpy(g).cuda()
    gibuf = torch.full((n + off_gi,), np.nan, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = _lib.load().novaq_max_pool2d_backward(gbuf[off_g:].data_ptr(), xbuf[off_x:].data_ptr(),
                                               CODE[xt], *shape, 2, 2, 2, 2, 0, 0, 0,
                                               gibuf[off_gi:].data_ptr(), stream)
    assert rc == _lib.OK
    got = gibuf[off_gi:].cpu().numpy().reshape(shape)
    same_bits_or_nan(got, R.max_pool2d_backward(g[off_g:].reshape(oshape), dec, 2, 2))
