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
