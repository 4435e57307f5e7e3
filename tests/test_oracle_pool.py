"""CPU pins of the pooling restatements (oracle/functional_ref.py): brute-force
window loops, torch's max_pool2d, exact means, and the reference's own
known-answer test (tests/layers/pooling/gap/test_gap2d.py:20-27)."""
import math

import numpy as np
import pytest
import torch

from oracle import functional_ref as R


def brute_max(x, k, s, p, mode):
    """Window max by loops: largest value, a later equal one replacing it,
    NaN once seen."""
    xp = np.pad(x, ((0, 0), (0, 0), (p[0], p[0]), (p[1], p[1])), mode=R.NP_PAD[mode])
    N, C, Hp, Wp = xp.shape
    OH, OW = (Hp - k[0]) // s[0] + 1, (Wp - k[1]) // s[1] + 1
    out = np.empty((N, C, OH, OW), np.float32)
    for n in range(N):
        for c in range(C):
            for i in range(OH):
                for j in range(OW):
                    acc = None
                    for a in range(k[0]):
                        for b in range(k[1]):
                            v = xp[n, c, i * s[0] + a, j * s[1] + b]
                            if acc is None or (not np.isnan(acc) and (v >= acc or np.isnan(v))):
                                acc = v
                    out[n, c, i, j] = acc
    return out


@pytest.mark.parametrize("k,s,p,mode", [((2, 2), (2, 2), (0, 0), "zeros"),
                                        ((3, 3), (1, 1), (1, 1), "zeros"),
                                        ((3, 2), (2, 1), (2, 1), "reflect"),
                                        ((2, 3), (1, 2), (1, 0), "replicate"),
                                        ((3, 3), (2, 2), (1, 2), "circular")])
def test_max_pool2d_matches_brute_force(k, s, p, mode):
    rng = np.random.default_rng(sum(k) + sum(s))
    x = rng.choice(np.array([-0.0, 0.0, -1.0, 1.0, 2.0, -3.0], np.float32), (2, 3, 7, 8))
    x[0, 0, 0, 0] = np.nan
    got = R.max_pool2d(x, k, s, p, mode)
    want = brute_max(x, k, s, p, mode)
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


def test_max_pool2d_matches_torch_without_padding():
    rng = np.random.default_rng(1)
    x = rng.standard_normal((4, 3, 10, 10)).astype(np.float32)
    want = torch.nn.functional.max_pool2d(torch.from_numpy(x), 2, 2).numpy()
    assert np.array_equal(R.max_pool2d(x, 2, 2), want)
    assert R.max_pool2d(x, 2, 2).shape == (4, 3, 5, 5)  # test_maxpooling2d.py:10-17
    assert R.max_pool2d(x[:2, :, :5, :5], 3, 1, 1).shape == (2, 3, 5, 5)  # :20-27


def test_zero_padding_pads_zeros_not_minus_infinity():
    """The reference pads with 0 (np.pad constant): an all-negative window
    touching the border gives 0 (torch would give the negative maximum)."""
    x = -np.ones((1, 1, 3, 3), np.float32)
    want = np.zeros((1, 1, 3, 3), np.float32)
    want[0, 0, 1, 1] = -1.0  # the one window inside the input
    assert np.array_equal(R.max_pool2d(x, 3, 1, 1), want)


def test_avg_pool2d_exact_means_and_known_answer():
    x = np.ones((2, 3, 4, 5), np.float32) * 3.0
    assert np.allclose(R.avg_pool2d(x), 3.0) and R.avg_pool2d(x).shape == (2, 3, 1, 1)
    rng = np.random.default_rng(2)
    y = rng.standard_normal((3, 4, 7, 7)).astype(np.float32)
    got = R.avg_pool2d(y).reshape(3, 4)
    for n in range(3):
        for c in range(4):
            exact = math.fsum(float(v) for v in y[n, c].ravel()) / 49
            assert abs(got[n, c] - exact) <= 4 * np.spacing(np.float32(abs(exact))) + 1e-7


def brute_max_backward(g, x, k, s, p, mode):
    """MaxPool2d's input gradient by per-element loops (gathered, not
    scattered): for each input element, the windows holding it in (oh, ow)
    order, each recomputing its max (NaN once seen), the count of elements
    equal to it (1 when none), and adding (element == max) * (grad / count),
    every step rounded to float32."""
    f32 = np.float32
    xp = np.pad(x, ((0, 0), (0, 0), (p[0], p[0]), (p[1], p[1])), mode=R.NP_PAD[mode])
    N, C, H, W = x.shape
    Hp, Wp = xp.shape[2:]
    OH, OW = (Hp - k[0]) // s[0] + 1, (Wp - k[1]) // s[1] + 1
    out = np.empty_like(x)
    for n in range(N):
        for c in range(C):
            for h in range(H):
                for w in range(W):
                    hp, wp = h + p[0], w + p[1]
                    acc = f32(0.0)
                    for i in range(OH):
                        if not i * s[0] <= hp < i * s[0] + k[0]:
                            continue
                        for j in range(OW):
                            if not j * s[1] <= wp < j * s[1] + k[1]:
                                continue
                            vals = [float(xp[n, c, i * s[0] + a, j * s[1] + b])
                                    for a in range(k[0]) for b in range(k[1])]
                            mx = math.nan if any(math.isnan(v) for v in vals) else max(vals)
                            cnt = sum(v == mx for v in vals) or 1
                            q = f32(g[n, c, i, j]) / f32(cnt)
                            m = f32(1.0) if float(xp[n, c, hp, wp]) == mx else f32(0.0)
                            acc = f32(acc + f32(m * q))
                    out[n, c, h, w] = acc
    return out


def same_bits_or_nan(got, want):
    nan = np.isnan(want)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))


@pytest.mark.parametrize("k,s,p,mode", [((2, 2), (2, 2), (0, 0), "zeros"),
                                        ((3, 3), (1, 1), (1, 1), "zeros"),
                                        ((3, 2), (2, 1), (2, 1), "reflect"),
                                        ((2, 3), (1, 2), (1, 0), "replicate"),
                                        ((3, 3), (2, 2), (1, 2), "circular")])
def test_max_pool2d_backward_matches_brute_force(k, s, p, mode):
    """Ties (several -0 / +0 / 1.0 maxima: the grad split three or more ways),
    a NaN window, +-inf and NaN grads, overlapping windows and every padding
    mode, bit for bit."""
    rng = np.random.default_rng(7 + sum(k) + sum(s))
    x = rng.choice(np.array([-0.0, 0.0, -1.0, 1.0, 2.0, -3.0], np.float32), (2, 3, 7, 8))
    x[0, 0, 0, 0] = np.nan
    OH = (7 + 2 * p[0] - k[0]) // s[0] + 1
    OW = (8 + 2 * p[1] - k[1]) // s[1] + 1
    g = rng.standard_normal((2, 3, OH, OW)).astype(np.float32)
    g[1, 2, 0, 0] = np.inf
    g[1, 1, -1, -1] = -np.inf
    g[0, 2, 0, 1] = np.nan
    got = R.max_pool2d_backward(g, x, k, s, p, mode)
    assert got.shape == x.shape and got.dtype == np.float32
    same_bits_or_nan(got, brute_max_backward(g, x, k, s, p, mode))


def test_max_pool2d_backward_ties_split_and_padding_dropped():
    """Closed forms: three equal maxima get grad / 3 each, a unique maximum the
    whole grad; a padded zero that is a window's maximum takes the grad and
    the cropped result does not hold it."""
    x = np.array([[[[1.0, 1.0], [1.0, 0.5]]]], np.float32)
    got = R.max_pool2d_backward(np.array([[[[3.0]]]], np.float32), x, 2, 2)
    assert np.array_equal(got, np.array([[[[1.0, 1.0], [1.0, 0.0]]]], np.float32))
    got = R.max_pool2d_backward(np.array([[[[0.3]]]], np.float32), x, 2, 2)
    assert got[0, 0, 0, 0] == np.float32(0.3) / np.float32(3.0)
    neg = -np.ones((1, 1, 2, 2), np.float32)
    got = R.max_pool2d_backward(np.ones((1, 1, 3, 3), np.float32), neg, 2, 1, 1)
    # of the nine 2x2 windows of the zero-padded 4x4, eight hold a padded 0
    # above the -1s (their grad lands on the padding); the middle one holds
    # the four -1s and splits its grad four ways
    assert np.array_equal(got, np.full((1, 1, 2, 2), 0.25, np.float32))


@pytest.mark.parametrize("k,s,p", [((2, 2), (2, 2), (0, 0)), ((3, 3), (1, 1), (1, 1)),
                                   ((3, 2), (2, 1), (1, 0))])
def test_max_pool2d_backward_finite_differences(k, s, p):
    """The derivative of sum(G * max_pool2d(x)) (the reference's own gradient
    check, tests/layers/pooling/maxpool/test_maxpooling2d.py:30-50): positive
    inputs without ties, so the zero padding is never a maximum."""
    rng = np.random.RandomState(8)
    x = (rng.rand(2, 3, 6, 6).astype(np.float64) + 0.5)
    G = rng.randn(*R.max_pool2d(x.astype(np.float32), k, s, p).shape)
    eps = 1e-5
    num = np.zeros_like(x)
    for idx in np.ndindex(x.shape):
        xp, xm = x.copy(), x.copy()
        xp[idx] += eps
        xm[idx] -= eps
        num[idx] = ((G * R.pool_windows(xp, k, s, p)[0].max(axis=(4, 5))).sum() -
                    (G * R.pool_windows(xm, k, s, p)[0].max(axis=(4, 5))).sum()) / (2 * eps)
    got = R.max_pool2d_backward(G.astype(np.float32), x.astype(np.float32), k, s, p)
    assert np.abs(got - num).max() < 5e-3


def test_global_avg_pool2d_backward_known_answers():
    """The reference's uniform-gradient test (test_gap2d.py:54-70: 1/(4*5)),
    its gradient check (:30-51), and each element the correctly rounded
    float32 product of grad and float32(1 / (H*W))."""
    got = R.global_avg_pool2d_backward(np.ones((1, 2, 1, 1), np.float32), (1, 2, 4, 5))
    assert got.shape == (1, 2, 4, 5) and np.allclose(got, 0.05)
    rng = np.random.default_rng(3)
    for H, W in [(6, 6), (7, 7), (3, 11), (28, 28)]:
        g = rng.standard_normal((2, 3, 1, 1)).astype(np.float32)
        got = R.global_avg_pool2d_backward(g, (2, 3, H, W))
        f = float(np.float32(1.0 / (H * W)))
        for n in range(2):
            for c in range(3):
                want = np.float32(float(g[n, c, 0, 0]) * f)  # exact in double, one rounding
                assert np.all(got[n, c].view(np.uint32) == want.view(np.uint32))
        # d/dx of sum(g * mean(x)) = g / (H*W)
        assert np.allclose(got, g / (H * W), rtol=1e-6, atol=0)
