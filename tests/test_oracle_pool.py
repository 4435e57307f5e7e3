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
