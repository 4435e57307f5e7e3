"""CPU checks of the epilogue restatements (ReLU, eval BatchNorm) and of the
host-side BatchNorm fold, against independent implementations and
properties."""
import numpy as np
import pytest
import torch

from oracle import functional_ref as R
from novann_amd.functional import Epilogue


def test_relu_values_and_sign_rules():
    """ReLU as the reference computes it: max(x, 0) in value, the sign of
    negative inputs kept on the zero they become, NaN for NaN and -Inf."""
    rng = np.random.default_rng(0)
    x = rng.standard_normal(1000).astype(np.float32)
    x[:6] = [0.0, -0.0, np.inf, -np.inf, np.nan, -1e-45]
    y = R.relu(x)
    fin = np.isfinite(x)
    np.testing.assert_array_equal(y[fin], np.maximum(x[fin], 0.0))
    assert np.array_equal(np.signbit(y[fin]), np.signbit(x[fin]) & (x[fin] <= 0))
    assert y[2] == np.inf and np.isnan(y[3]) and np.isnan(y[4])
    # torch.relu agrees in value (it returns +0 for negative inputs)
    t = torch.relu(torch.from_numpy(x[fin])).numpy()
    np.testing.assert_array_equal(np.abs(y[fin]), t)


def test_relu_mistake_is_caught():
    """A plain max(x, 0) (the common restatement) differs in the sign of zero."""
    x = np.array([-1.0, -0.0, 2.0], np.float32)
    assert not np.array_equal(np.signbit(R.relu(x)), np.signbit(np.maximum(x, 0.0)))


@pytest.mark.parametrize("shape,axis", [((4, 3, 5, 6), 1), ((7, 9), 1)])
def test_batchnorm_eval_matches_torch(shape, axis):
    rng = np.random.default_rng(len(shape))
    x = rng.standard_normal(shape)
    C = shape[axis]
    g, b = rng.standard_normal(C), rng.standard_normal(C)
    m, v = rng.standard_normal(C), rng.uniform(0.1, 3.0, C)
    want = torch.nn.functional.batch_norm(
        torch.from_numpy(x), torch.from_numpy(m), torch.from_numpy(v), torch.from_numpy(g),
        torch.from_numpy(b), training=False, eps=1e-5).numpy()
    np.testing.assert_allclose(R.batchnorm_eval(x, g, b, m, v, 1e-5, axis), want, rtol=1e-12,
                               atol=1e-12)


def test_batchnorm_fold_equals_the_unfolded_form():
    """Epilogue.batchnorm's (mul, add) applied as v * mul + add agrees with
    the reference's formula to fp32 rounding."""
    rng = np.random.default_rng(3)
    C = 16
    x = rng.standard_normal((8, C, 5, 5)).astype(np.float32)
    g, b = rng.standard_normal(C), rng.standard_normal(C)
    m, v = rng.standard_normal(C), rng.uniform(0.01, 4.0, C)
    ep = Epilogue.batchnorm(g.reshape(1, C, 1, 1), b.reshape(1, C, 1, 1),
                            m.reshape(1, C, 1, 1), v.reshape(1, C, 1, 1), eps=1e-5)
    got = R.epilogue_f32(x, ep.channel_mul, ep.channel_add)
    want = R.batchnorm_eval(x, g, b, m, v, 1e-5)
    np.testing.assert_allclose(got, want, rtol=2e-6, atol=2e-6 * np.abs(want).max())


def test_epilogue_f32_order():
    """mul before add, relu last; each step an fp32 operation."""
    y = np.array([[1.0, -2.0], [3.0, 0.5]], np.float32)
    got = R.epilogue_f32(y, [2.0, 3.0], [-1.0, 1.0], True, axis=1)
    np.testing.assert_array_equal(got, np.array([[1.0, -0.0], [5.0, 2.5]], np.float32))
    assert np.signbit(got[0, 1])
