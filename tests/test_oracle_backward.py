"""The numpy restatement of Linear.backward (novann/layers/linear/linear.py:85-108)
pinned by central finite differences of the restated forward in fp64 -- the
check the reference's own test applies to its layer
(tests/layers/linear/test_linear.py:31-64), here with an fp64 step so the
agreement is tight.  Shapes with D_in != D_out and a square one, so a
transposed operand cannot pass."""
import numpy as np
import pytest

from oracle import functional_ref as R


def loss(x, w, b, g):
    return float(np.sum(R.linear(x, w, b) * g))


def numeric(f, a, h=1e-6):
    out = np.zeros_like(a)
    it = np.nditer(a, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        old = a[i]
        a[i] = old + h
        up = f()
        a[i] = old - h
        dn = f()
        a[i] = old
        out[i] = (up - dn) / (2 * h)
    return out


@pytest.mark.parametrize("N,D_in,D_out", [(3, 5, 4), (4, 4, 4), (2, 7, 3)])
def test_linear_backward_matches_finite_differences(N, D_in, D_out):
    rng = np.random.default_rng(N * 100 + D_in * 10 + D_out)
    x = rng.standard_normal((N, D_in))
    w = rng.standard_normal((D_out, D_in))
    b = rng.standard_normal((1, D_out))
    g = rng.standard_normal((N, D_out))
    gi, gw, gb = R.linear_backward(g, x, w)
    f = lambda: loss(x, w, b, g)  # noqa: E731
    assert gi.shape == x.shape and gw.shape == w.shape and gb.shape == b.shape
    np.testing.assert_allclose(gw, numeric(f, w), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gi, numeric(f, x), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gb, numeric(f, b), rtol=1e-6, atol=1e-7)
    # without a bias term there is no bias gradient
    assert R.linear_backward(g, x, w, bias=False)[2] is None


def test_planted_transpose_mistake_is_caught():
    """grad @ w.T (a transposed operand) fails the same check."""
    rng = np.random.default_rng(1)
    x, w, b, g = (rng.standard_normal(s) for s in ((4, 4), (4, 4), (1, 4), (4, 4)))
    f = lambda: loss(x, w, b, g)  # noqa: E731
    assert not np.allclose(g @ w.T, numeric(f, x), rtol=1e-6, atol=1e-7)
