"""The module / layer contract and the default weights of the layers, on the
host (no GPU: every layer here is fp32, so nothing is quantized).

The initialisers follow novann/core/init.py and the layers' defaults
novann/core/config.py:24-40 with linear.py:47-68 and conv2d.py:55-72.  What
pins them:
  - the distribution tests of the reference's own tests/initializers/
    test_init.py:21-115 (same shapes, nonlinearity and bounds);
  - closed forms: gains, fans of 2-5 dimensional shapes, the std / bound each
    formula gives, checked on large draws;
  - the generator stream: after np.random.seed(s), a layer's weight is the
    next draw of numpy's global legacy generator, which RandomState(s) replays
    through its own methods (standard_normal / normal / uniform); two layers
    built in a row take consecutive draws, as the reference's layers do.
"""
import numpy as np
import pytest

from novann_amd import init as I
from novann_amd import module as M

SHAPES = [(200, 784), (3, 128, 128), (128, 3, 3, 3), (128, 3, 3, 3, 3)]


def test_gains_and_fans():
    assert I.calculate_gain("linear") == I.calculate_gain("sigmoid") == 1.0
    assert I.calculate_gain("tanh") == 5.0 / 3.0
    assert I.calculate_gain("relu") == np.sqrt(2.0)
    assert I.calculate_gain("leakyrelu") == np.sqrt(2.0 / (1 + 0.01 ** 2))
    assert I.calculate_gain("leakyrelu", 0.2) == np.sqrt(2.0 / 1.04)
    with pytest.raises(ValueError):
        I.calculate_gain("gelu")
    assert I.fans((200, 784)) == (784, 200)
    assert I.fans((3, 128, 128)) == (128 * 128, 3 * 128)
    assert I.fans((128, 3, 3, 3)) == (27, 128 * 9)
    assert I.fans((128, 3, 3, 3, 3)) == (81, 128 * 27)
    with pytest.raises(ValueError):
        I.fans((5,))
    with pytest.raises(ValueError):
        I.fans((1, 2, 3, 4, 5, 6))
    with pytest.raises(ValueError):
        I.shape_validation((4, 4), "fan_avg")


def test_reference_distribution_tests():
    """tests/initializers/test_init.py:21-115 of the reference, same checks."""
    g = I.calculate_gain("leakyrelu")
    for shape in SHAPES:
        fan_in, fan_out = I.shape_validation(shape, "both")
        w = I.kaiming_normal_(shape, nonlinearity="leakyrelu")
        assert abs(w.mean()) < 0.1 and abs(w.std() - g / np.sqrt(fan_in)) < 0.1
        w = I.kaiming_uniform_(shape, nonlinearity="leakyrelu")
        lim = g * np.sqrt(3.0 / fan_in)
        assert np.all(w <= lim) and np.all(w >= -lim)
        w = I.xavier_normal_(shape, g)
        assert abs(w.mean()) < 0.1 and abs(w.var() - g * np.sqrt(2 / (fan_in + fan_out))) < 0.1
        w = I.xavier_uniform_(shape, g)
        lim = g * np.sqrt(6 / (fan_in + fan_out))
        assert np.all(w <= lim) and np.all(w >= -lim)
        assert abs(I.random_init_(shape, g).mean()) < 0.1
        with pytest.raises(ValueError):
            I.kaiming_normal_(shape, nonlinearity="gelu")
        with pytest.raises(ValueError):
            I.kaiming_uniform_(shape, nonlinearity="gelu")


def test_formulas_on_large_draws():
    np.random.seed(1)
    w = I.kaiming_normal_((2048, 512))
    assert w.dtype == np.float32 and abs(w.std() / np.sqrt(2.0 / 512) - 1) < 0.01
    w = I.kaiming_uniform_((2048, 512))
    b = np.sqrt(2.0) * np.sqrt(3.0 / 512)
    assert w.max() <= b and w.min() >= -b and w.max() > 0.999 * b
    assert abs(w.std() / (b / np.sqrt(3.0)) - 1) < 0.01   # uniform(-b, b): std b / sqrt 3
    w = I.random_init_((2048, 512))
    assert w.dtype == np.float32 and abs(w.std() / 0.001 - 1) < 0.01
    w = I.xavier_normal_((2048, 512), 2.0)
    assert abs(w.std() / (2.0 * np.sqrt(2.0 / 2560)) - 1) < 0.01


def test_seeded_linear_weights_are_the_reference_draws():
    np.random.seed(7)
    a = M.Linear(64, 32)
    b = M.Linear(16, 8, bias=False)
    rs = np.random.RandomState(7)
    want_a = rs.standard_normal((32, 64)).astype(np.float32) * np.float32(0.001)
    want_b = rs.standard_normal((8, 16)).astype(np.float32) * np.float32(0.001)
    assert a.weight.data.dtype == np.float32
    assert np.array_equal(a.weight.data.view(np.uint32), want_a.view(np.uint32))
    assert np.array_equal(b.weight.data.view(np.uint32), want_b.view(np.uint32))
    assert a.bias.data.shape == (1, 32) and not a.bias.data.any() and b.bias is None
    assert a.weight.name == "linear weight" and a.bias.name == "linear bias"


def test_seeded_conv2d_weights_are_the_reference_draws():
    np.random.seed(11)
    c1 = M.Conv2d(1, 32, 3, padding=1)
    c2 = M.Conv2d(32, 64, (3, 3), padding=1)
    rs = np.random.RandomState(11)
    for c, cin, cout in ((c1, 1, 32), (c2, 32, 64)):
        bound = np.sqrt(2.0) * np.sqrt(3.0 / (cin * 9))
        want = rs.uniform(-bound, bound, (cout, cin, 3, 3)).astype(np.float32)
        assert np.array_equal(c.weight.data.view(np.uint32), want.view(np.uint32))
        assert c.bias.data.shape == (cout, 1) and c.bias.data.dtype == np.float32


def test_init_argument_and_reset_parameters():
    np.random.seed(3)
    lin = M.Linear(8, 4, init=I.DEFAULT_NORMAL_INIT_MAP["relu"])
    rs = np.random.RandomState(3)
    want = rs.normal(0.0, np.sqrt(2.0) / np.sqrt(8), (4, 8)).astype(np.float32)
    assert np.array_equal(lin.weight.data, want)
    lin.reset_parameters(lambda shape: np.full(shape, 0.5))
    assert lin.weight.data.dtype == np.float32 and np.all(lin.weight.data == 0.5)
    np.random.seed(3)
    lin.reset_parameters()   # back to the layer's own init function
    assert np.array_equal(lin.weight.data, want)
    conv = M.Conv2d(2, 3, 3, init=lambda shape: np.ones(shape))
    assert conv.weight.data.dtype == np.float32 and np.all(conv.weight.data == 1.0)


def test_module_contract():
    lin = M.Linear(4, 3)
    assert isinstance(lin, M.Layer) and isinstance(lin, M.Module)
    assert lin._training
    lin.eval()
    assert not lin._training
    lin.train()
    assert lin._training
    assert lin.parameters() == [lin.weight, lin.bias]
    assert lin.weight.grad is not None and lin.weight.grad.shape == (3, 4)
    lin.zero_grad()
    assert lin.weight.grad is None and lin.bias.grad is None
    conv = M.Conv2d(2, 3, 3, bias=False)
    assert conv.parameters() == [conv.weight]
    assert M.Module().parameters() == []
    with pytest.raises(TypeError):
        M.Layer()            # abstract forward / backward
    bn = M.BatchNorm2d(3)
    assert bn.parameters() == [bn.gamma, bn.beta] and bn._training
    assert repr(lin) == "Linear(in_features=4, out_features=3, bias=True)"
    # the reference's positional order: (in, out, bias, init)
    f = lambda shape: np.zeros(shape)  # noqa: E731
    assert M.Linear(4, 3, True, f).init_fn is f
    assert M.Conv2d(1, 2, 3, 1, 0, True, "zeros", f).init_fn is f
    # stride None means the kernel size (conv2d.py:41)
    assert (M.Conv2d(1, 1, (2, 3), stride=None).sh, M.Conv2d(1, 1, (2, 3), stride=None).sw) == (2, 3)


def test_forward_coerces_numpy_input_to_float32():
    x = np.ones((2, 3), np.float64)
    assert M._as_f32(x).dtype == np.float32
    x32 = np.ones((2, 3), np.float32)
    assert M._as_f32(x32) is x32          # copy=False keeps float32 arrays as they are
