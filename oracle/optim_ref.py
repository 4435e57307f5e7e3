"""numpy restatement of NovaNN's AdamW step -- TEST INFRASTRUCTURE ONLY.

Restates ``AdamW.step`` (novann/optim/adamw.py:41-65) for one float32
parameter, in the reference's order of operations.  The reference's
parameters and moment buffers are float32 arrays (linear.py:59-65,
conv2d.py:65-69, ``np.zeros_like`` at adamw.py:36-37) and its
hyper-parameters Python floats, so numpy evaluates every step as a float32
operation with the Python scalar rounded to float32 (``1 - b1`` and
``b1 ** t`` are formed in double first, as Python does):

  m = f(b1) * m + f(1 - b1) * g
  v = f(b2) * v + f(1 - b2) * (g * g)
  m_hat = m / f(1 - b1**t);  v_hat = v / f(1 - b2**t)
  w = w - (f(lr) * m_hat) / (sqrt(v_hat) + f(eps))
  w = w - f(lr * wd) * w          (when wd > 0 and the parameter is not a
                                   BatchNorm gamma / beta)

f() is the float32 rounding of a Python float.
"""
from __future__ import annotations

import numpy as np


def adamw_step(w, g, m, v, t: int, lr: float, b1: float = 0.9, b2: float = 0.999,
               eps: float = 1e-8, wd: float = 0.0, decay: bool = True):
    """One AdamW step at step count t (1-based) on float32 arrays; returns
    new (w, m, v) (the inputs are not modified)."""
    w = np.asarray(w, np.float32).copy()
    g = np.asarray(g, np.float32)
    m = b1 * np.asarray(m, np.float32) + (1 - b1) * g
    v = b2 * np.asarray(v, np.float32) + (1 - b2) * (g ** 2)
    m_hat = m / (1 - b1 ** t)
    v_hat = v / (1 - b2 ** t)
    w -= lr * m_hat / (np.sqrt(v_hat) + eps)
    if wd > 0 and decay:
        w -= lr * wd * w
    assert w.dtype == m.dtype == v.dtype == np.float32
    return w, m, v


def adamw_step_f64(w, g, m, v, t: int, lr: float, b1: float = 0.9, b2: float = 0.999,
                   eps: float = 1e-8, wd: float = 0.0, decay: bool = True):
    """The same statements on a float64 parameter with float64 moments (the
    reference's BatchNorm gamma / beta are float64 arrays, batchnorm2d.py:
    33-55, and ``np.zeros_like`` gives their moments that dtype).  ``g`` keeps
    its own dtype: numpy forms ``(1 - b1) * g`` and ``g ** 2`` in float32 for a
    float32 gradient (a Python float does not widen an array) and widens only
    when adding them to the float64 moments.  Returns new (w, m, v)."""
    w = np.array(w, dtype=np.float64)
    m = b1 * np.asarray(m, np.float64) + (1 - b1) * g
    v = b2 * np.asarray(v, np.float64) + (1 - b2) * (g ** 2)
    m_hat = m / (1 - b1 ** t)
    v_hat = v / (1 - b2 ** t)
    w -= lr * m_hat / (np.sqrt(v_hat) + eps)
    if wd > 0 and decay:
        w -= lr * wd * w
    assert w.dtype == m.dtype == v.dtype == np.float64
    return w, m, v
