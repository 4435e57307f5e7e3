"""CPU pins of the AdamW restatement (oracle/optim_ref.py): torch's Adam and
AdamW (independent implementations), the first step's closed form, and the
float32 evaluation the reference's arrays imply."""
import numpy as np
import pytest
import torch

from oracle import optim_ref as OR


def run_oracle(w0, grads, **hp):
    w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
    for t, g in enumerate(grads, 1):
        w, m, v = OR.adamw_step(w, g, m, v, t, **hp)
    return w


def run_torch(w0, grads, cls, **kw):
    p = torch.nn.Parameter(torch.from_numpy(w0.astype(np.float64)))
    opt = cls([p], **kw)
    for g in grads:
        p.grad = torch.from_numpy(g.astype(np.float64))
        opt.step()
    return p.detach().numpy()


@pytest.mark.parametrize("lr,b1,b2", [(1e-3, 0.9, 0.999), (3e-2, 0.8, 0.99)])
def test_adam_part_matches_torch_adam(lr, b1, b2):
    rng = np.random.default_rng(0)
    w0 = rng.standard_normal(500).astype(np.float32)
    grads = [rng.standard_normal(500).astype(np.float32) for _ in range(20)]
    got = run_oracle(w0, grads, lr=lr, b1=b1, b2=b2, eps=1e-8, wd=0.0)
    want = run_torch(w0, grads, torch.optim.Adam, lr=lr, betas=(b1, b2), eps=1e-8)
    np.testing.assert_allclose(got, want, rtol=0, atol=20 * lr * 1e-5 + 1e-6)


def test_weight_decay_matches_torch_adamw_up_to_the_order():
    """The reference decays after the Adam update (w -= lr*wd*w on the updated
    w); torch decays before it.  The two differ by lr*wd*(Adam update) per
    step, at most lr^2 * wd per step and element."""
    rng = np.random.default_rng(1)
    lr, wd, steps = 1e-2, 0.1, 10
    w0 = rng.standard_normal(300).astype(np.float32)
    grads = [rng.standard_normal(300).astype(np.float32) for _ in range(steps)]
    got = run_oracle(w0, grads, lr=lr, wd=wd)
    want = run_torch(w0, grads, torch.optim.AdamW, lr=lr, weight_decay=wd, eps=1e-8)
    assert np.abs(got - want).max() <= steps * lr * lr * wd * 1.01 + 1e-5
    # and the decay is there: without it the result moves by about lr*wd*|w| per step
    nodecay = run_oracle(w0, grads, lr=lr, wd=0.0)
    assert np.abs(nodecay - want).max() > 10 * np.abs(got - want).max()


def test_first_step_closed_form():
    """From zero moments, step 1 moves each weight by lr * g / (|g| + eps)
    (m_hat = g, v_hat = g^2 up to float32 rounding); BatchNorm parameters
    (decay=False) skip the decay."""
    rng = np.random.default_rng(2)
    w0 = rng.standard_normal(1000).astype(np.float32)
    g = rng.standard_normal(1000).astype(np.float32)
    lr = 1e-3
    w1, m1, v1 = OR.adamw_step(w0, g, np.zeros_like(w0), np.zeros_like(w0), 1, lr, wd=0.5,
                               decay=False)
    # (w1 is rounded to float32 at |w0|: an ulp of w0 is the resolution)
    want = lr * g.astype(np.float64) / (np.abs(g) + 1e-8)
    assert np.all(np.abs((w0.astype(np.float64) - w1) - want)
                  <= np.spacing(np.abs(w0)) + 1e-5 * np.abs(want))
    np.testing.assert_allclose(m1, 0.1 * g, rtol=1e-6)
    np.testing.assert_allclose(v1, 0.001 * g * g, rtol=1e-5)


def test_float32_evaluation():
    """Every intermediate is float32 (the reference's arrays are float32 and
    its hyper-parameters Python floats): the result differs from a float64
    evaluation of the same formula."""
    rng = np.random.default_rng(3)
    w0 = rng.standard_normal(4096).astype(np.float32)
    g = rng.standard_normal(4096).astype(np.float32)
    w32, _, _ = OR.adamw_step(w0, g, np.zeros_like(w0), np.zeros_like(w0), 3, 1e-3, wd=0.01)
    w0d, gd = w0.astype(np.float64), g.astype(np.float64)
    m = 0.1 * gd
    v = 0.001 * gd * gd
    w64 = w0d - 1e-3 * (m / (1 - 0.9 ** 3)) / (np.sqrt(v / (1 - 0.999 ** 3)) + 1e-8)
    w64 -= 1e-3 * 0.01 * w64
    assert not np.array_equal(w32, w64.astype(np.float32))
    np.testing.assert_allclose(w32, w64, rtol=1e-6, atol=1e-7)


def run_oracle64(w0, grads, **hp):
    w, m, v = w0.copy(), np.zeros_like(w0), np.zeros_like(w0)
    for t, g in enumerate(grads, 1):
        w, m, v = OR.adamw_step_f64(w, g, m, v, t, **hp)
    return w, m, v


@pytest.mark.parametrize("gdt", [np.float64, np.float32])
def test_float64_parameters_match_torch_adam(gdt):
    """float64 parameters (BatchNorm's gamma / beta) step in float64: torch's
    Adam in float64 agrees to float64 rounding for a float64 gradient; a
    float32 gradient's products are float32 roundings (relative 2^-24) in
    numpy, which stays well within float32 distance of torch."""
    rng = np.random.default_rng(4)
    w0 = rng.standard_normal(400)
    grads = [rng.standard_normal(400).astype(gdt) for _ in range(15)]
    got, m, v = run_oracle64(w0, grads, lr=1e-2, b1=0.9, b2=0.999, eps=1e-8, wd=0.0)
    assert got.dtype == m.dtype == v.dtype == np.float64
    want = run_torch(w0, grads, torch.optim.Adam, lr=1e-2, betas=(0.9, 0.999), eps=1e-8)
    tol = 1e-12 if gdt == np.float64 else 1e-6
    np.testing.assert_allclose(got, want, rtol=0, atol=tol)


def test_float64_parameter_with_float32_gradient_rounds_the_products():
    """With a float32 gradient numpy rounds (1 - b1) * g and (1 - b2) * g**2 to
    float32 (a Python scalar keeps a float32 array float32) before the float64
    sums: the moments then differ from those of the widened gradient."""
    rng = np.random.default_rng(5)
    w0 = rng.standard_normal(2000)
    g32 = rng.standard_normal(2000).astype(np.float32)
    _, m32, v32 = OR.adamw_step_f64(w0, g32, np.zeros(2000), np.zeros(2000), 1, 1e-3)
    _, m64, v64 = OR.adamw_step_f64(w0, g32.astype(np.float64), np.zeros(2000), np.zeros(2000),
                                    1, 1e-3)
    assert not np.array_equal(m32, m64) and not np.array_equal(v32, v64)
    np.testing.assert_allclose(m32, m64, rtol=2 ** -23)
    # m = b1 * 0 + f32(0.1 * g): each moment is a float32 value
    assert np.array_equal(m32, m32.astype(np.float32).astype(np.float64))
