"""numpy restatement of NovaNN's forward operators -- TEST INFRASTRUCTURE ONLY.

Restates, with this build's own code, the arithmetic of
  - ``novann.functional.linear``  (novann/functional.py:147-163):
    ``out = input @ weight.T`` then ``out += bias`` (in place, fp32);
  - ``Linear.backward`` (novann/layers/linear/linear.py:85-108):
    grad_weight = grad.T @ x, grad_bias = grad summed over the batch
    (keepdims), grad_input = grad @ weight;
  - ``Conv2d.backward`` and ``Conv2d._col2im``
    (novann/layers/convolutional/conv2d.py:117-148, 179-207): grad_weight =
    grad (C_out, N*OH*OW) @ col.T, grad_bias = row sums, grad_col = w_col.T @
    grad scattered with np.add.at into a zero-padded (N, C, H_p, W_p) buffer
    whose border is then cropped;
  - ``novann.functional.relu`` (novann/functional.py:8-22): ``x * (x > 0)``;
  - ``novann.functional.max_pool2d`` (:450-534): np.pad, an as_strided
    (N, C, OH, OW, KH, KW) window view (returned with extras=True),
    ``max(axis=(4, 5))``; and
    ``avg_pool2d`` (:548-559): ``np.mean(x, axis=(2, 3), keepdims=True)``;
  - ``MaxPool2d.backward`` (layers/pooling/maxpool/maxpool2d.py:79-129): the
    window mask of the max, grad split over ties, shares scattered in window
    order into the padded shape and cropped; ``GlobalAvgPool2d.backward``
    (layers/pooling/gap/global_avg_pool2d.py:35-57): grad * (1 / (H*W));
  - eval-mode ``BatchNorm2d`` / ``BatchNorm1d`` (batchnorm2d.py:98-102,
    batchnorm1d.py:138-149): ``gamma * (x - mean) / sqrt(var + eps) + beta``
    per channel, in fp64 as the reference's float64 running statistics make it;
  - ``novann.functional.conv2d``  (novann/functional.py:275-385):
    pad with numpy.pad (constant / reflect / edge / wrap, :325-344), take
    (N, C, OH, OW, KH, KW) windows with ``as_strided`` (:358-364), reorder
    to a (C*KH*KW, N*OH*OW) column matrix (:367), one GEMM with the
    (C_out, C*KH*KW) weight (:374-377), bias (:378-379), and return the
    (N, C_out, OH, OW) view (:382).
The window ordering and the output layout have to match the reference's
exactly (they decide which products are summed), so they are the same here.
Used as the fp32 CPU baseline (the reference's own numpy arithmetic) and as a
second checker next to the C oracle's fp64 loops.
"""
from __future__ import annotations

import numpy as np
from numpy.lib.stride_tricks import as_strided

NP_PAD = {"zeros": "constant", "reflect": "reflect", "replicate": "edge",
          "circular": "wrap"}


def linear(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None) -> np.ndarray:
    out = x @ w.T
    if bias is not None:
        out += bias.reshape(1, -1)
    return out


def linear_backward(grad: np.ndarray, x: np.ndarray, w: np.ndarray, bias: bool = True):
    """(grad_input, grad_weight, grad_bias) of ``linear`` for grad = dL/dy,
    in the order Linear.backward forms them (linear.py:100-107)."""
    grad_weight = grad.T @ x
    grad_bias = np.sum(grad, axis=0, keepdims=True) if bias else None
    grad_input = grad @ w
    return grad_input, grad_weight, grad_bias


def _pair(v):
    if isinstance(v, int):
        return (v, v)
    return tuple(v)


def im2col(x: np.ndarray, KH: int, KW: int, stride=(1, 1), padding=(0, 0),
           padding_mode: str = "zeros"):
    """(C*KH*KW, N*OH*OW) column matrix and (OH, OW)."""
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    if padding_mode not in NP_PAD:
        raise ValueError(f"padding_mode Only accept {tuple(NP_PAD)} not '{padding_mode}'")
    N, C, H, W = x.shape
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)), mode=NP_PAD[padding_mode])
    OH = (H + 2 * ph - KH) // sh + 1
    OW = (W + 2 * pw - KW) // sw + 1
    s0, s1, s2, s3 = xp.strides
    win = as_strided(xp, shape=(N, C, OH, OW, KH, KW),
                     strides=(s0, s1, s2 * sh, s3 * sw, s2, s3))
    col = win.transpose(1, 4, 5, 0, 2, 3).reshape(C * KH * KW, N * OH * OW)
    return col, OH, OW


def conv2d(x: np.ndarray, w: np.ndarray, stride=(1, 1), padding=(0, 0),
           padding_mode: str = "zeros", bias: np.ndarray | None = None) -> np.ndarray:
    C_out, C, KH, KW = w.shape
    N = x.shape[0]
    col, OH, OW = im2col(x, KH, KW, stride, padding, padding_mode)
    out = w.reshape(C_out, -1) @ col
    if bias is not None:
        out += bias.reshape(C_out, 1)
    return out.reshape(C_out, N, OH, OW).transpose(1, 0, 2, 3)


def col2im(col: np.ndarray, x_shape, KH: int, KW: int, stride=(1, 1), padding=(0, 0)):
    """Scatter-add a (C*KH*KW, N*OH*OW) column gradient into a zero-padded
    (N, C, H+2ph, W+2pw) image and crop the border (conv2d.py:117-148).  Rows
    are (c, kh, kw), columns (n, oh, ow), as ``im2col`` lays them out."""
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    N, C, H, W = x_shape
    OH = (H + 2 * ph - KH) // sh + 1
    OW = (W + 2 * pw - KW) // sw + 1
    cols = col.reshape(C, KH, KW, N, OH, OW)
    out = np.zeros((N, C, H + 2 * ph, W + 2 * pw), dtype=col.dtype)
    for kh in range(KH):
        for kw in range(KW):
            # window position (kh, kw) of output pixel (oh, ow) lands on padded
            # row oh*sh + kh, column ow*sw + kw; within one (kh, kw) the targets
            # are distinct, so a sliced += accumulates exactly as np.add.at
            out[:, :, kh:kh + sh * (OH - 1) + 1:sh, kw:kw + sw * (OW - 1) + 1:sw] += \
                cols[:, kh, kw].transpose(1, 0, 2, 3)
    return out[:, :, ph:ph + H, pw:pw + W]


def conv2d_backward(grad: np.ndarray, x: np.ndarray, w: np.ndarray, stride=(1, 1),
                    padding=(0, 0), padding_mode: str = "zeros", bias: bool = True):
    """(grad_input, grad_weight, grad_bias) in the order Conv2d.backward forms
    them (conv2d.py:194-207); grad_bias has the reference's (C_out, 1) shape."""
    C_out, C, KH, KW = w.shape
    col, OH, OW = im2col(x, KH, KW, stride, padding, padding_mode)
    g = grad.transpose(1, 0, 2, 3).reshape(C_out, -1)
    grad_weight = (g @ col.T).reshape(w.shape)
    grad_bias = np.sum(g, axis=1).reshape(-1, 1) if bias else None
    grad_col = w.reshape(C_out, -1).T @ g
    grad_input = col2im(grad_col, x.shape, KH, KW, stride, padding)
    return grad_input, grad_weight, grad_bias


def relu(x: np.ndarray) -> np.ndarray:
    """functional.py:19-20: the mask as x's dtype, then a multiply (negative
    values give -0, NaN stays NaN, -Inf gives NaN)."""
    with np.errstate(invalid="ignore"):  # -Inf * 0 is NaN, as in the reference
        return x * (x > 0).astype(x.dtype, copy=False)


def batchnorm_eval(x: np.ndarray, gamma, beta, running_mean, running_var, eps: float = 1e-5,
                   axis: int = 1) -> np.ndarray:
    """Eval-mode batch norm over channel axis ``axis`` in fp64
    (batchnorm2d.py:98-102; batchnorm1d.py:138-149 with axis 1 of a 2-D x)."""
    shape = [1] * x.ndim
    shape[axis] = -1
    r = lambda a: np.asarray(a, dtype=np.float64).reshape(shape)  # noqa: E731
    x_hat = (x.astype(np.float64) - r(running_mean)) / np.sqrt(r(running_var) + eps)
    return r(gamma) * x_hat + r(beta)


def epilogue_f32(y: np.ndarray, mul=None, add=None, do_relu: bool = False,
                 axis: int = 1) -> np.ndarray:
    """The fused epilogue's fp32 steps on an fp32 product output y (each one
    rounded fp32 operation, in the kernels' order): y * mul[c], + add[c],
    then relu."""
    shape = [1] * y.ndim
    shape[axis] = -1
    v = np.asarray(y, dtype=np.float32)
    if mul is not None:
        v = v * np.asarray(mul, np.float32).reshape(shape)
    if add is not None:
        v = v + np.asarray(add, np.float32).reshape(shape)
    if do_relu:
        v = relu(v)
    return v


def pool_windows(x: np.ndarray, kernel_size, stride, padding=(0, 0),
                 padding_mode: str = "zeros"):
    """(windows, OH, OW, padded_shape): the (N, C, OH, OW, KH, KW) strided view
    of the padded input that max_pool2d(..., extras=True) returns
    (functional.py:516-534)."""
    KH, KW = _pair(kernel_size)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    N, C, H, W = x.shape
    xp = np.pad(x, ((0, 0), (0, 0), (ph, ph), (pw, pw)), mode=NP_PAD[padding_mode])
    OH = (H + 2 * ph - KH) // sh + 1
    OW = (W + 2 * pw - KW) // sw + 1
    s0, s1, s2, s3 = xp.strides
    win = as_strided(xp, shape=(N, C, OH, OW, KH, KW),
                     strides=(s0, s1, s2 * sh, s3 * sw, s2, s3))
    return win, OH, OW, xp.shape


def max_pool2d(x: np.ndarray, kernel_size, stride, padding=(0, 0),
               padding_mode: str = "zeros") -> np.ndarray:
    """The reference's window view and max (functional.py:493-532)."""
    return pool_windows(x, kernel_size, stride, padding, padding_mode)[0].max(axis=(4, 5))


def avg_pool2d(x: np.ndarray) -> np.ndarray:
    """functional.py:559."""
    return np.mean(x, axis=(2, 3), keepdims=True)


def max_pool2d_backward(grad: np.ndarray, x: np.ndarray, kernel_size, stride,
                        padding=(0, 0), padding_mode: str = "zeros") -> np.ndarray:
    """MaxPool2d.backward (layers/pooling/maxpool/maxpool2d.py:79-129): over
    the forward's window view of the padded input, mask = (window == its max)
    (all 0 when the max is NaN), count = the mask's sum (1 where 0), each
    window's share = mask * (grad / count) in float32; the shares are added
    into a zero buffer of the padded shape in (oh, ow) order (:114-124) and
    the padding is cropped (:126-129)."""
    KH, KW = _pair(kernel_size)
    sh, sw = _pair(stride)
    ph, pw = _pair(padding)
    N, C, H, W = x.shape
    win, OH, OW, pshape = pool_windows(np.asarray(x, np.float32), kernel_size, stride,
                                       padding, padding_mode)
    g = np.asarray(grad, np.float32).reshape(N, C, OH, OW)
    mx = win.max(axis=(4, 5), keepdims=True)
    mask = (win == mx).astype(np.float32)
    count = mask.sum(axis=(4, 5), keepdims=True)
    count[count == 0] = 1.0
    share = mask * (g[:, :, :, :, np.newaxis, np.newaxis] / count)
    gp = np.zeros(pshape, np.float32)
    for i in range(OH):
        for j in range(OW):
            gp[:, :, i * sh:i * sh + KH, j * sw:j * sw + KW] += share[:, :, i, j]
    return gp[:, :, ph:ph + H, pw:pw + W]


def global_avg_pool2d_backward(grad: np.ndarray, x_shape) -> np.ndarray:
    """GlobalAvgPool2d.backward (layers/pooling/gap/global_avg_pool2d.py:35-57):
    ``ones * (grad * (1.0 / (H * W)))`` in float32 (the Python float factor
    becomes float32 before the product)."""
    N, C, H, W = x_shape
    g = np.asarray(grad, np.float32).reshape(N, C, 1, 1)
    return np.ones((N, C, H, W), np.float32) * (g * (1.0 / (H * W)))
