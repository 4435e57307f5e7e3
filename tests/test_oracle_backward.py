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


def conv_loss(x, w, b, g, stride, padding, mode):
    return float(np.sum(R.conv2d(x, w, stride, padding, mode, b) * g))


@pytest.mark.parametrize("case", [
    # (N, C, H, W, C_out, KH, KW, sh, sw, ph, pw)
    (2, 3, 5, 6, 4, 3, 3, 1, 1, 1, 1),
    (1, 2, 7, 7, 3, 3, 2, 2, 1, 0, 1),
    (2, 1, 6, 5, 2, 2, 3, 1, 2, 2, 1),
])
def test_conv2d_backward_zeros_padding_matches_finite_differences(case):
    N, C, H, W, C_out, KH, KW, sh, sw, ph, pw = case
    rng = np.random.default_rng(sum(case))
    x = rng.standard_normal((N, C, H, W))
    w = rng.standard_normal((C_out, C, KH, KW))
    b = rng.standard_normal(C_out)
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    g = rng.standard_normal((N, C_out, OH, OW))
    gi, gw, gb = R.conv2d_backward(g, x, w, (sh, sw), (ph, pw), "zeros")
    f = lambda: conv_loss(x, w, b, g, (sh, sw), (ph, pw), "zeros")  # noqa: E731
    assert gi.shape == x.shape and gw.shape == w.shape and gb.shape == (C_out, 1)
    np.testing.assert_allclose(gw, numeric(f, w), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gi, numeric(f, x), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gb.reshape(-1), numeric(f, b), rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("mode", ["reflect", "replicate", "circular"])
def test_conv2d_backward_other_modes(mode):
    """grad_weight and grad_bias are the true gradients in every mode (the
    column matrix holds the mode's padding); grad_input is the cropped col2im,
    i.e. the zero-padding gradient, whatever the mode (conv2d.py:143-146)."""
    rng = np.random.default_rng(len(mode))
    x = rng.standard_normal((2, 2, 5, 6))
    w = rng.standard_normal((3, 2, 3, 3))
    b = rng.standard_normal(3)
    g = rng.standard_normal((2, 3, 5, 6))
    gi, gw, gb = R.conv2d_backward(g, x, w, (1, 1), (1, 1), mode)
    f = lambda: conv_loss(x, w, b, g, (1, 1), (1, 1), mode)  # noqa: E731
    np.testing.assert_allclose(gw, numeric(f, w), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(gb.reshape(-1), numeric(f, b), rtol=1e-6, atol=1e-7)
    gi0, _, _ = R.conv2d_backward(g, x, w, (1, 1), (1, 1), "zeros")
    np.testing.assert_allclose(gi, gi0, rtol=0, atol=0)
    # and that differs from the true gradient of the padded forward
    assert not np.allclose(gi, numeric(f, x), rtol=1e-6, atol=1e-7)


def test_col2im_is_the_adjoint_of_im2col():
    """<im2col(x), c> == <x, col2im(c)> for zero padding (the scatter is the
    transpose of the gather), with strides and uneven padding."""
    rng = np.random.default_rng(5)
    x = rng.standard_normal((2, 3, 7, 8))
    col, OH, OW = R.im2col(x, 3, 2, (2, 1), (1, 2), "zeros")
    c = rng.standard_normal(col.shape)
    lhs = float(np.sum(col * c))
    rhs = float(np.sum(x * R.col2im(c, x.shape, 3, 2, (2, 1), (1, 2))))
    assert abs(lhs - rhs) <= 1e-9 * max(1.0, abs(lhs))
