"""Pins the oracle's products (CPU only): the C fp64 loops against numpy's
fp64 matmul and the numpy im2col restatement of NovaNN's conv2d, and both
against torch CPU conv2d; the padding index rules against numpy.pad."""
import numpy as np
import pytest
import torch

import oracle as O
from oracle import functional_ref as R


def test_linear_f64_matches_numpy():
    rng = np.random.default_rng(0)
    x = rng.standard_normal((33, 70)).astype(np.float32)
    w = rng.standard_normal((21, 70)).astype(np.float32)
    b = rng.standard_normal(21).astype(np.float32)
    y = O.linear_f64(x, w, b)
    r = x.astype(np.float64) @ w.astype(np.float64).T + b
    assert np.allclose(y, r, rtol=1e-6, atol=1e-6)
    # the reference's own fp32 arithmetic (x @ W.T then += b) agrees to fp32 rounding
    assert np.allclose(R.linear(x, w, b.reshape(1, -1)), r, rtol=1e-4, atol=1e-4)


def test_linear_golden(golden):
    g = golden["products"]
    codes, s = g["lin_codes"], float(g["lin_scale"][0])
    w = O.cast(codes.reshape(-1), O.E4M3, O.F32, scale=s).reshape(codes.shape)
    y = O.linear_f64(g["lin_x"], w, g["lin_bias"])
    assert np.allclose(y, g["lin_y"], rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("mode,tmode", [("zeros", "constant"), ("reflect", "reflect"),
                                        ("replicate", "replicate"),
                                        ("circular", "circular")])
@pytest.mark.parametrize("case", [(2, 3, 9, 7, 4, 3, 3, 1, 1, 1, 1), (1, 2, 12, 10, 3, 5, 3, 2, 1, 2, 1),
                                  (2, 4, 6, 6, 2, 1, 1, 1, 1, 0, 0)])
def test_conv2d_f64_vs_im2col_and_torch(mode, tmode, case):
    N, C, H, W, Co, KH, KW, sh, sw, ph, pw = case
    rng = np.random.default_rng(sum(case))
    x = rng.standard_normal((N, C, H, W)).astype(np.float32)
    w = rng.standard_normal((Co, C, KH, KW)).astype(np.float32)
    b = rng.standard_normal(Co).astype(np.float32)
    y = O.conv2d_f64(x, w, (sh, sw), (ph, pw), mode, b)
    r = R.conv2d(x.astype(np.float64), w.astype(np.float64), (sh, sw), (ph, pw), mode,
                 b.astype(np.float64))
    assert np.allclose(y, r, rtol=1e-5, atol=1e-5)
    xt = torch.nn.functional.pad(torch.from_numpy(x).double(), (pw, pw, ph, ph), mode=tmode)
    t = torch.nn.functional.conv2d(xt, torch.from_numpy(w).double(), torch.from_numpy(b).double(),
                                   stride=(sh, sw)).numpy()
    assert np.allclose(y, t, rtol=1e-5, atol=1e-5)


def test_conv2d_golden(golden):
    g = golden["products"]
    n = 5 * 3 * 3 * 3
    w = O.cast(g["conv_packed"], O.E2M1, O.F32, n=n, scale=float(g["conv_scale"][0]))
    for mode in ("zeros", "reflect", "replicate", "circular"):
        y = O.conv2d_f64(g["conv_x"], w.reshape(5, 3, 3, 3), (2, 1), (2, 1), mode, g["conv_bias"])
        assert np.allclose(y, g[f"conv_y_{mode}"], rtol=1e-5, atol=1e-5), mode


def test_pad_index_matches_numpy_pad_any_width():
    for n in range(1, 7):
        x = np.arange(n)
        for p in range(0, 15):
            for mode, np_mode in [("reflect", "reflect"), ("replicate", "edge"),
                                  ("circular", "wrap")]:
                ref = np.pad(x, (p, p), mode=np_mode)
                mine = np.array([x[O.pad_index(i - p, n, mode)] for i in range(n + 2 * p)])
                assert np.array_equal(ref, mine), (n, p, mode)
    assert O.pad_index(-1, 5, "zeros") == -1


def test_conv2d_rejects_bad_mode():
    with pytest.raises(ValueError):
        R.im2col(np.zeros((1, 1, 4, 4)), 3, 3, padding_mode="mirror")


@pytest.mark.parametrize("mode", ["zeros", "reflect", "replicate", "circular"])
@pytest.mark.parametrize("case", [(2, 3, 5, 4, 3, 2, 1, 1, 1, 1), (1, 2, 7, 6, 2, 3, 2, 1, 2, 0),
                                  (3, 1, 4, 4, 1, 1, 1, 2, 0, 0)])
def test_im2col_and_windows_match_index_loops(mode, case):
    """The column matrix conv2d(extras=True) returns and max_pool2d's window
    view, against their definitions written as index loops over np.pad:
    col[(c, kh, kw), (n, oh, ow)] = xp[n, c, oh*sh + kh, ow*sw + kw] with rows
    and columns numbered row-major (a transposed or mis-strided view fails)."""
    N, C, H, W, KH, KW, sh, sw, ph, pw = case
    x = np.arange(N * C * H * W, dtype=np.float32).reshape(N, C, H, W) * 0.5 - 3.0
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)), mode=R.NP_PAD[mode])
    col, OH, OW = R.im2col(x, KH, KW, (sh, sw), (ph, pw), mode)
    win, OH2, OW2, pshape = R.pool_windows(x, (KH, KW), (sh, sw), (ph, pw), mode)
    assert (OH2, OW2) == (OH, OW) and pshape == xp.shape
    assert col.shape == (C * KH * KW, N * OH * OW) and win.shape == (N, C, OH, OW, KH, KW)
    for c in range(C):
        for kh in range(KH):
            for kw in range(KW):
                for n in range(N):
                    for oh in range(OH):
                        for ow in range(OW):
                            v = xp[n, c, oh * sh + kh, ow * sw + kw]
                            assert col[(c * KH + kh) * KW + kw, (n * OH + oh) * OW + ow] == v
                            assert win[n, c, oh, ow, kh, kw] == v
