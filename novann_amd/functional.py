"""Drop-in ``linear`` / ``conv2d`` with NovaNN's operator signatures.

Mirrors novann/functional.py:147-163 (``linear``) and :275-385 (``conv2d``):
same argument names, order and meaning, same output shapes, and the same
``ValueError`` cases.  Arguments may be numpy arrays (copied to the device,
result copied back as an ndarray, as the reference returns) or device
tensors (result stays on the device).  The weight is a ``Parameters``
(fp32 ``.data``) or a ``QuantizedParameters`` (E4M3 / E5M2 / E2M1 codes plus a
per-tensor scale).  The work runs in libnovaq.so on the GPU; there is no CPU
path.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import Any, Optional, Tuple, Union

import numpy as np
import torch

from . import _lib
from ._lib import DTYPES, PAD_MODES, check
from .module import Parameters, QuantizedParameters

IntPair = Union[int, Tuple[int, int], str]


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("novann_amd needs a HIP device (no CPU fallback)")
    return torch.device("cuda", torch.cuda.current_device())


def _to_device_f32(a, what: str) -> Tuple[torch.Tensor, bool]:
    """(contiguous fp32 device tensor, True if the caller passed numpy)."""
    if isinstance(a, np.ndarray):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(_device()), True
    if isinstance(a, torch.Tensor):
        if not a.is_cuda:
            a = a.to(_device())
        return _aligned(a.to(torch.float32).contiguous()), False
    raise TypeError(f"{what} must be a numpy array or a torch tensor")


def _aligned(t: torch.Tensor) -> torch.Tensor:
    """The kernels read 16-byte vectors: a view that does not start on a
    16-byte boundary (a slice of a larger tensor) is copied, not refused."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


_X_DTYPES = {torch.float16: "f16", torch.bfloat16: "bf16", torch.float8_e4m3fn: "e4m3",
             torch.float8_e5m2: "e5m2"}


def _x_arg(a, what: str):
    """(device tensor, dtype name, scale tensor or None, logical shape, was_numpy)
    for a product input: fp32 (numpy or tensors of other float types are
    converted), a bf16 / f16 / FP8 device tensor as stored, or a
    quant.Quantized E4M3 / E5M2 activation (codes + its scale)."""
    from . import quant
    if isinstance(a, quant.Quantized):
        if a.dtype not in ("e4m3", "e5m2"):
            raise TypeError(f"{what}: a quantized input must be e4m3 or e5m2, got {a.dtype}")
        a.check(what)
        return _aligned(a.data.contiguous()), a.dtype, a.scale, tuple(a.shape), False
    if isinstance(a, torch.Tensor) and a.is_cuda and a.dtype in _X_DTYPES:
        return _aligned(a.contiguous()), _X_DTYPES[a.dtype], None, tuple(a.shape), False
    t, was_numpy = _to_device_f32(a, what)
    return t, "f32", None, tuple(t.shape), was_numpy


def _weight_args(weight, dev: torch.device):
    """(codes tensor, dtype code, scale tensor or None) for a weight."""
    if isinstance(weight, QuantizedParameters):
        from . import quant
        n = 1
        for d in weight.stored_shape:
            n *= int(d)
        quant._require_holds(weight.codes, weight.dtype, n, "weight codes")
        return _aligned(weight.codes.to(dev).contiguous()), DTYPES[weight.dtype], weight.scale.to(dev)
    data = weight.data if isinstance(weight, Parameters) else weight
    w, _ = _to_device_f32(data, "weight")
    return w, DTYPES["f32"], None


def _bias_arg(bias, dev: torch.device) -> Optional[torch.Tensor]:
    if bias is None:
        return None
    data = bias.data if isinstance(bias, Parameters) else bias
    b, _ = _to_device_f32(data, "bias")
    return _aligned(b.reshape(-1).contiguous())


def _stream(dev: torch.device) -> int:
    return torch.cuda.current_stream(dev).cuda_stream


OUT_STORAGE = {"f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16,
               "e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2}


@dataclass
class Epilogue:
    """Fused epilogue of ``linear`` / ``conv2d`` (struct novaq_epilogue).

    Per output channel c: v = v * channel_mul[c] + channel_add[c] (each step
    only when given), then ReLU as novann's ``v * (v > 0)``
    (novann/functional.py:8-22) when ``relu``, then the store in
    ``out_dtype``: 'f32', 'f16' / 'bf16' (round to nearest even) or
    'e4m3' / 'e5m2' as encode(v / s) with ``out_scale`` s (a one-element fp32
    device tensor, default 1).  ``out_amax`` (a one-element fp32 device
    tensor) receives max |v| before the cast.  channel_mul / channel_add are
    arrays or tensors of C_out values."""
    channel_mul: Any = None
    channel_add: Any = None
    relu: bool = False
    out_dtype: str = "f32"
    out_scale: Optional[torch.Tensor] = None
    out_amax: Optional[torch.Tensor] = None

    @classmethod
    def batchnorm(cls, gamma, beta, running_mean, running_var, eps: float = 1e-5,
                  **kw) -> "Epilogue":
        """Eval-mode BatchNorm (batchnorm2d.py:98-102, batchnorm1d.py:138-149)
        gamma * (v - mean) / sqrt(var + eps) + beta, folded in fp64 into
        channel_mul = gamma / sqrt(var + eps), channel_add = beta - mean *
        channel_mul, rounded to fp32."""
        def flat(a):
            a = a.data if isinstance(a, Parameters) else a
            if isinstance(a, torch.Tensor):
                a = a.detach().cpu().numpy()
            return np.asarray(a, dtype=np.float64).reshape(-1)
        g, b, m, v = flat(gamma), flat(beta), flat(running_mean), flat(running_var)
        mul = g / np.sqrt(v + eps)
        return cls(channel_mul=mul.astype(np.float32), channel_add=(b - m * mul).astype(np.float32),
                   **kw)


def _epilogue_args(ep: Optional[Epilogue], channels: int, dev: torch.device):
    """(ctypes struct or None, output storage dtype, tensors to keep alive)."""
    if ep is None:
        return None, torch.float32, []
    if ep.out_dtype not in OUT_STORAGE:
        raise TypeError(f"epilogue out_dtype must be one of {tuple(OUT_STORAGE)}")
    keep = []

    def chan(a, what):
        if a is None:
            return None
        t, _ = _to_device_f32(a, what)
        t = t.reshape(-1).contiguous()
        if t.numel() != channels:
            raise ValueError(f"epilogue {what} has {t.numel()} values, expected {channels}")
        keep.append(t)
        return t.data_ptr()

    def scalar(t, what):
        if t is None:
            return None
        if not isinstance(t, torch.Tensor) or not t.is_cuda or t.dtype != torch.float32:
            raise TypeError(f"epilogue {what} must be a float32 device tensor")
        return t.data_ptr()

    st = _lib.Epilogue(chan(ep.channel_mul, "channel_mul"), chan(ep.channel_add, "channel_add"),
                       scalar(ep.out_scale, "out_scale"), scalar(ep.out_amax, "out_amax"),
                       1 if ep.relu else 0, DTYPES[ep.out_dtype])
    return st, OUT_STORAGE[ep.out_dtype], keep


def _finish(y: torch.Tensor, ep: Optional[Epilogue], was_numpy: bool):
    """The caller-facing output: ndarray for numpy callers with f32 / f16
    output; FP8 outputs as quant.Quantized (codes + the scale they carry)."""
    from . import quant
    if ep is not None and ep.out_dtype in ("e4m3", "e5m2"):
        scale = ep.out_scale if ep.out_scale is not None else torch.ones(
            1, dtype=torch.float32, device=y.device)
        return quant.Quantized(data=y.reshape(-1), shape=tuple(y.shape), dtype=ep.out_dtype,
                               scale=scale, amax=ep.out_amax)
    if was_numpy and y.dtype in (torch.float32, torch.float16):
        return y.cpu().numpy()
    return y


def linear(input, weight, bias: Optional[Parameters] = None, *,
           epilogue: Optional[Epilogue] = None):
    """y = input @ W^T + b  (novann/functional.py:147-163).

    input (N, D_in); weight (D_out, D_in) as Parameters or
    QuantizedParameters; bias (1, D_out) Parameters or None.  Returns
    (N, D_out) fp32: an ndarray when input was an ndarray.  ``epilogue``
    (keyword only, not in the reference) fuses what follows the layer (eval
    BatchNorm1d, ReLU, a cast of y) into the product; see Epilogue."""
    x, xdt, xs, xshape, was_numpy = _x_arg(input, "input")
    if len(xshape) != 2:
        raise ValueError(f"linear expects a 2-D input, got shape {xshape}")
    wshape = weight.shape if isinstance(weight, QuantizedParameters) else tuple(
        (weight.data if isinstance(weight, Parameters) else weight).shape)
    if len(wshape) != 2 or wshape[1] != xshape[1]:
        raise ValueError(f"matmul: input {xshape} does not match weight {wshape}")
    N, D_in = xshape
    D_out = wshape[0]
    w, wdt, ws = _weight_args(weight, x.device)
    b = _bias_arg(bias, x.device)
    if b is not None and b.numel() != D_out:
        raise ValueError(f"bias has {b.numel()} values, expected {D_out}")
    if epilogue is not None or xdt != "f32":
        st, ydt, keep = _epilogue_args(epilogue, D_out, x.device)
        y = torch.empty((N, D_out), dtype=ydt, device=x.device)
        check(_lib.load().novaq_linear_forward_ex(
            x.data_ptr(), DTYPES[xdt], None if xs is None else xs.data_ptr(), N, D_in,
            w.data_ptr(), wdt,
            None if ws is None else ws.data_ptr(), None if b is None else b.data_ptr(), D_out,
            None if st is None else ctypes.byref(st), y.data_ptr(), _stream(x.device)), "linear")
        return _finish(y, epilogue, was_numpy)
    y = torch.empty((N, D_out), dtype=torch.float32, device=x.device)
    check(_lib.load().novaq_linear_forward(
        x.data_ptr(), N, D_in, w.data_ptr(), wdt, None if ws is None else ws.data_ptr(),
        None if b is None else b.data_ptr(), D_out, y.data_ptr(), _stream(x.device)),
        "linear")
    return y.cpu().numpy() if was_numpy else y


def linear_backward(grad, input, weight, bias: bool = True):
    """Gradients of ``linear(input, weight, bias)`` for ``grad`` = dL/dy.

    Restates Linear.backward (novann/layers/linear/linear.py:85-108) on the
    GPU: returns ``(grad_input, grad_weight, grad_bias)`` with
    grad_input = grad @ W (N, D_in), grad_weight = grad.T @ input
    (D_out, D_in) and grad_bias = grad summed over the batch (1, D_out), or
    None when ``bias`` is false.  A quantized weight enters as s * decode(codes)
    (its gradient is the gradient of that dequantized matrix).  ndarrays in ->
    ndarrays out."""
    g, was_numpy = _to_device_f32(grad, "grad")
    x, _ = _to_device_f32(input, "input")
    if g.dim() != 2 or x.dim() != 2 or g.shape[0] != x.shape[0]:
        raise ValueError(f"grad {tuple(g.shape)} does not match input {tuple(x.shape)}")
    N, D_out = g.shape
    D_in = x.shape[1]
    wshape = weight.shape if isinstance(weight, QuantizedParameters) else tuple(
        (weight.data if isinstance(weight, Parameters) else weight).shape)
    if tuple(wshape) != (D_out, D_in):
        raise ValueError(f"weight {tuple(wshape)} does not match grad {tuple(g.shape)} and "
                         f"input {tuple(x.shape)}")
    w, wdt, ws = _weight_args(weight, x.device)
    if wdt == DTYPES["e2m1"] and (D_in % 2 or D_out % 2):
        # nibble-packed codes transpose only with even sides: decode them to
        # bf16 (exact for every E2M1 value, no scale) and multiply those same
        # values, the scale applied after accumulation as for the codes
        from . import quant
        rows = quant.cast(w, "bf16", src_dtype="e2m1", n=D_out * weight.padded_cols)
        w, wdt = rows.view(D_out, weight.padded_cols)[:, :D_in].contiguous(), DTYPES["bf16"]
    lib = _lib.load()
    gi = torch.empty((N, D_in), dtype=torch.float32, device=x.device)
    gw = torch.empty((D_out, D_in), dtype=torch.float32, device=x.device)
    gb = torch.empty((1, D_out), dtype=torch.float32, device=x.device) if bias else None
    nbytes = lib.novaq_linear_backward_workspace(N, D_in, D_out, wdt)
    # FP8 weights at whole-tile shapes need no workspace (the query returns 0)
    work = torch.empty(nbytes, dtype=torch.uint8, device=x.device) if nbytes else None
    check(lib.novaq_linear_backward(
        g.data_ptr(), x.data_ptr(), N, D_in, w.data_ptr(), wdt,
        None if ws is None else ws.data_ptr(), D_out, gi.data_ptr(), gw.data_ptr(),
        None if gb is None else gb.data_ptr(), None if work is None else work.data_ptr(),
        nbytes, _stream(x.device)), "linear backward")
    if was_numpy:
        return (gi.cpu().numpy(), gw.cpu().numpy(), None if gb is None else gb.cpu().numpy())
    return gi, gw, gb


def _pair(v: IntPair) -> Tuple[int, int]:
    """int -> (v, v); 'valid' -> (0, 0); 'same' and other strings raise
    ValueError (novann/functional.py:302-313)."""
    if isinstance(v, (int, np.integer)):
        return (int(v), int(v))
    if isinstance(v, str):
        if v == "valid":
            return (0, 0)
        if v == "same":
            raise ValueError("The 'same' value is not currently supported")
        raise ValueError(f"Unsupported value '{v}'")
    return tuple(int(e) for e in v)


def conv2d(input, weight, kernel_size: IntPair, stride: IntPair = 1, padding: IntPair = 0,
           *, bias: Optional[Parameters] = None, padding_mode: str = "zeros",
           extras: bool = False, epilogue: Optional[Epilogue] = None):
    """2-D cross-correlation (novann/functional.py:275-385).

    input (N, C, H, W); weight (C_out, C, KH, KW); returns (N, C_out, OH, OW)
    fp32 with OH = (H + 2ph - KH)//sh + 1.  The product uses implicit im2col
    (no column matrix).  ``extras=True`` returns ``(out, col, w_col)`` as the
    reference does (:383-384) for callers that cache them (Conv2d.forward,
    novann/layers/convolutional/conv2d.py:162-175): ``col`` is the
    (C*KH*KW, N*OH*OW) fp32 column matrix (rows (c, kh, kw), columns
    (n, oh, ow), the padding mode resolved), written by its own gather kernel;
    ``w_col`` is the weight as a (C_out, C*KH*KW) fp32 matrix -- a view of an
    fp32 weight's data, as ``weight.data.reshape(C_out, -1)`` is in the
    reference, or s * decode(codes) for a quantized weight.  numpy in -> numpy
    out.  ``epilogue`` (not in the reference) fuses eval BatchNorm2d, ReLU and a
    cast of y into the convolution; see Epilogue."""
    KH, KW = _pair(kernel_size)
    ph, pw = _pair(padding)
    sh, sw = _pair(stride)
    modes = tuple(PAD_MODES)
    if padding_mode not in PAD_MODES:
        raise ValueError(f"padding_mode Only accept {modes} not '{padding_mode}'")
    x, xdt, xs, xshape, was_numpy = _x_arg(input, "input")
    if len(xshape) != 4:
        raise ValueError(f"conv2d expects (N, C, H, W), got {xshape}")
    N, C, H, W = xshape
    wshape = weight.shape if isinstance(weight, QuantizedParameters) else tuple(
        (weight.data if isinstance(weight, Parameters) else weight).shape)
    if len(wshape) != 4 or wshape[1] != C or (wshape[2], wshape[3]) != (KH, KW):
        raise ValueError(f"weight shape {wshape} does not match input channels {C} and "
                         f"kernel {(KH, KW)}")
    C_out = wshape[0]
    OH = (H + 2 * ph - KH) // sh + 1
    OW = (W + 2 * pw - KW) // sw + 1
    if OH <= 0 or OW <= 0:
        raise ValueError(f"output size {(OH, OW)} is empty")
    w, wdt, ws = _weight_args(weight, x.device)
    b = _bias_arg(bias, x.device)
    if b is not None and b.numel() != C_out:
        raise ValueError(f"bias has {b.numel()} values, expected {C_out}")
    if epilogue is not None or xdt != "f32":
        st, ydt, keep = _epilogue_args(epilogue, C_out, x.device)
        y = torch.empty((N, C_out, OH, OW), dtype=ydt, device=x.device)
        check(_lib.load().novaq_conv2d_forward_ex(
            x.data_ptr(), DTYPES[xdt], None if xs is None else xs.data_ptr(), N, C, H, W,
            w.data_ptr(), wdt, None if ws is None else ws.data_ptr(), C_out, KH, KW, sh, sw, ph,
            pw, PAD_MODES[padding_mode], None if b is None else b.data_ptr(),
            None if st is None else ctypes.byref(st), y.data_ptr(), _stream(x.device)),
            "conv2d")
        out = _finish(y, epilogue, was_numpy)
    else:
        y = torch.empty((N, C_out, OH, OW), dtype=torch.float32, device=x.device)
        check(_lib.load().novaq_conv2d_forward(
            x.data_ptr(), N, C, H, W, w.data_ptr(), wdt, None if ws is None else ws.data_ptr(),
            C_out, KH, KW, sh, sw, ph, pw, PAD_MODES[padding_mode],
            None if b is None else b.data_ptr(), y.data_ptr(), _stream(x.device)), "conv2d")
        out = y.cpu().numpy() if was_numpy else y
    if not extras:
        return out
    col = im2col(x, (KH, KW), (sh, sw), (ph, pw), padding_mode, _xdtype=xdt, _xscale=xs,
                 _shape=xshape)
    return out, (col.cpu().numpy() if was_numpy else col), _w_col(weight, C_out, was_numpy)


def _w_col(weight, C_out: int, was_numpy: bool):
    """conv2d's (C_out, C*KH*KW) weight matrix (functional.py:374): a view of
    an fp32 weight's data, the dequantized weight for quantized codes."""
    if isinstance(weight, QuantizedParameters):
        w = weight.dequantize().reshape(C_out, -1)
        return w.cpu().numpy() if was_numpy else w
    data = weight.data if isinstance(weight, Parameters) else weight
    if isinstance(data, torch.Tensor):
        w = data.reshape(C_out, -1)
        return w.detach().cpu().numpy() if was_numpy else w
    return np.asarray(data).reshape(C_out, -1)


def im2col(input, kernel_size: IntPair, stride: IntPair = 1, padding: IntPair = 0,
           padding_mode: str = "zeros", *, _xdtype=None, _xscale=None, _shape=None):
    """The column matrix of conv2d (novann/functional.py:346-368) as a
    (C*KH*KW, N*OH*OW) fp32 device tensor: col[(c, kh, kw), (n, oh, ow)] =
    the input padded with numpy.pad's rules at [n, c, oh*sh + kh, ow*sw + kw].
    Narrow inputs are decoded (FP8 times its scale)."""
    KH, KW = _pair(kernel_size)
    ph, pw = _pair(padding)
    sh, sw = _pair(stride)
    if padding_mode not in PAD_MODES:
        raise ValueError(f"padding_mode Only accept {tuple(PAD_MODES)} not '{padding_mode}'")
    if _xdtype is None:
        x, xdt, xs, xshape, _ = _x_arg(input, "input")
    else:
        x, xdt, xs, xshape = input, _xdtype, _xscale, _shape
    if len(xshape) != 4:
        raise ValueError(f"im2col expects (N, C, H, W), got {xshape}")
    N, C, H, W = xshape
    OH = (H + 2 * ph - KH) // sh + 1
    OW = (W + 2 * pw - KW) // sw + 1
    if OH <= 0 or OW <= 0:
        raise ValueError(f"output size {(OH, OW)} is empty")
    col = torch.empty((C * KH * KW, N * OH * OW), dtype=torch.float32, device=x.device)
    check(_lib.load().novaq_im2col(x.data_ptr(), DTYPES[xdt], None if xs is None else xs.data_ptr(),
                                   N, C, H, W, KH, KW, sh, sw, ph, pw, PAD_MODES[padding_mode],
                                   col.data_ptr(), _stream(x.device)), "im2col")
    return col


def conv2d_backward(grad, input, weight, kernel_size: IntPair, stride: IntPair = 1,
                    padding: IntPair = 0, *, bias: bool = True, padding_mode: str = "zeros"):
    """Gradients of ``conv2d(input, weight, ...)`` for ``grad`` = dL/dy.

    Restates Conv2d.backward with its _col2im
    (novann/layers/convolutional/conv2d.py:117-148, 179-207) on the GPU:
    returns ``(grad_input, grad_weight, grad_bias)``; grad_weight has the
    weight's shape, grad_bias the reference's (C_out, 1) (None when ``bias``
    is false), grad_input the input's shape (accumulated into a zero-padded
    image whose border is cropped, as the reference does, in every padding
    mode).  ndarrays in -> ndarrays out."""
    KH, KW = _pair(kernel_size)
    ph, pw = _pair(padding)
    sh, sw = _pair(stride)
    if padding_mode not in PAD_MODES:
        raise ValueError(f"padding_mode Only accept {tuple(PAD_MODES)} not '{padding_mode}'")
    g, was_numpy = _to_device_f32(grad, "grad")
    x, _ = _to_device_f32(input, "input")
    if x.dim() != 4 or g.dim() != 4:
        raise ValueError(f"conv2d_backward expects 4-D grad and input, got {tuple(g.shape)} "
                         f"and {tuple(x.shape)}")
    N, C, H, W = x.shape
    wshape = weight.shape if isinstance(weight, QuantizedParameters) else tuple(
        (weight.data if isinstance(weight, Parameters) else weight).shape)
    C_out = wshape[0]
    OH, OW = (H + 2 * ph - KH) // sh + 1, (W + 2 * pw - KW) // sw + 1
    if tuple(wshape) != (C_out, C, KH, KW) or tuple(g.shape) != (N, C_out, OH, OW):
        raise ValueError(f"grad {tuple(g.shape)}, input {tuple(x.shape)} and weight "
                         f"{tuple(wshape)} do not match")
    w, wdt, ws = _weight_args(weight, x.device)
    lib = _lib.load()
    gi = torch.empty((N, C, H, W), dtype=torch.float32, device=x.device)
    gw = torch.empty((C_out, C, KH, KW), dtype=torch.float32, device=x.device)
    gb = torch.empty((C_out, 1), dtype=torch.float32, device=x.device) if bias else None
    nbytes = lib.novaq_conv2d_backward_workspace(N, C, C_out, KH, KW, wdt)
    work = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    check(lib.novaq_conv2d_backward(
        g.data_ptr(), x.data_ptr(), N, C, H, W, w.data_ptr(), wdt,
        None if ws is None else ws.data_ptr(), C_out, KH, KW, sh, sw, ph, pw,
        PAD_MODES[padding_mode], gi.data_ptr(), gw.data_ptr(),
        None if gb is None else gb.data_ptr(), work.data_ptr(), nbytes, _stream(x.device)),
        "conv2d backward")
    if was_numpy:
        return (gi.cpu().numpy(), gw.cpu().numpy(), None if gb is None else gb.cpu().numpy())
    return gi, gw, gb


def _narrow_out(y: torch.Tensor, xdt: str, xs, was_numpy: bool, shape):
    """A pooled result in the input's storage: ndarray for numpy callers,
    quant.Quantized (same scale) for FP8 inputs, the device tensor otherwise."""
    from . import quant
    if xdt in ("e4m3", "e5m2"):
        scale = xs if xs is not None else torch.ones(1, dtype=torch.float32, device=y.device)
        return quant.Quantized(data=y.reshape(-1), shape=tuple(shape), dtype=xdt, scale=scale)
    return y.cpu().numpy() if was_numpy else y


def max_pool2d(input, kernel_size: IntPair, stride: IntPair, padding: IntPair = 0,
               padding_mode: str = "zeros", extras: bool = False):
    """2-D max pooling (novann/functional.py:450-532): the input padded with
    numpy.pad's rules (zeros pads 0), the max of each window.  Returns
    (N, C, OH, OW) in the input's storage (fp32 ndarray for numpy input; bf16
    / f16 tensors and FP8 Quantized activations pool without decoding: the
    result is one of the input values).  ``extras=True`` returns
    ``(out, windows, OH, OW, padded_shape)`` as the reference does (:533-534)
    for MaxPool2d.forward's cache (layers/pooling/maxpool/maxpool2d.py:63-75):
    ``windows`` is the (N, C, OH, OW, KH, KW) strided view of the padded input
    (padded on the device in the input's storage, FP8 as codes), an ndarray
    for numpy input."""
    KH, KW = _pair(kernel_size)
    ph, pw = _pair(padding)
    sh, sw = _pair(stride)
    if padding_mode not in PAD_MODES:
        raise ValueError(f"padding_mode Only accept {tuple(PAD_MODES)} not '{padding_mode}'")
    x, xdt, xs, xshape, was_numpy = _x_arg(input, "input")
    if len(xshape) != 4:
        raise ValueError(f"max_pool2d expects (N, C, H, W), got {xshape}")
    N, C, H, W = xshape
    OH = (H + 2 * ph - KH) // sh + 1
    OW = (W + 2 * pw - KW) // sw + 1
    if OH <= 0 or OW <= 0:
        raise ValueError(f"output size {(OH, OW)} is empty")
    y = torch.empty(N * C * OH * OW, dtype=x.dtype, device=x.device)
    check(_lib.load().novaq_max_pool2d(x.data_ptr(), DTYPES[xdt], N, C, H, W, KH, KW, sh, sw,
                                       ph, pw, PAD_MODES[padding_mode], y.data_ptr(),
                                       _stream(x.device)), "max_pool2d")
    out = _narrow_out(y.view(N, C, OH, OW), xdt, xs, was_numpy, (N, C, OH, OW))
    if not extras:
        return out
    Hp, Wp = H + 2 * ph, W + 2 * pw
    xp = torch.empty((N, C, Hp, Wp), dtype=x.dtype, device=x.device)
    check(_lib.load().novaq_pad2d(x.data_ptr(), DTYPES[xdt], N, C, H, W, ph, pw,
                                  PAD_MODES[padding_mode], xp.data_ptr(), _stream(x.device)),
          "max_pool2d padding")
    shape = (N, C, OH, OW, KH, KW)
    if was_numpy:
        from numpy.lib.stride_tricks import as_strided
        xp_h = xp.cpu().numpy()
        s0, s1, s2, s3 = xp_h.strides
        windows = as_strided(xp_h, shape=shape, strides=(s0, s1, s2 * sh, s3 * sw, s2, s3))
    else:
        s0, s1, s2, s3 = xp.stride()
        windows = xp.as_strided(shape, (s0, s1, s2 * sh, s3 * sw, s2, s3))
    return out, windows, OH, OW, (N, C, Hp, Wp)


def max_pool2d_backward(grad, input, kernel_size: IntPair, stride: IntPair,
                        padding: IntPair = 0, padding_mode: str = "zeros"):
    """MaxPool2d's input gradient (novann/layers/pooling/maxpool/maxpool2d.py:
    79-129) for grad (N, C, OH, OW) and the forward's input (as max_pool2d
    takes it: fp32, bf16 / f16 or an FP8 Quantized activation, whose windows
    compare as stored): each window's grad split over the elements equal to
    its maximum, the windows' shares added per element in window order, the
    padding's shares dropped.  Returns (N, C, H, W) fp32, an ndarray for a
    numpy grad; bit for bit the reference's result."""
    KH, KW = _pair(kernel_size)
    ph, pw = _pair(padding)
    sh, sw = _pair(stride)
    if padding_mode not in PAD_MODES:
        raise ValueError(f"padding_mode Only accept {tuple(PAD_MODES)} not '{padding_mode}'")
    x, xdt, _, xshape, _ = _x_arg(input, "input")
    if len(xshape) != 4:
        raise ValueError(f"max_pool2d_backward expects an (N, C, H, W) input, got {xshape}")
    N, C, H, W = xshape
    OH = (H + 2 * ph - KH) // sh + 1
    OW = (W + 2 * pw - KW) // sw + 1
    g, was_numpy = _to_device_f32(grad, "grad")
    if tuple(g.shape) != (N, C, OH, OW):
        raise ValueError(f"grad shape {tuple(g.shape)} is not the output's {(N, C, OH, OW)}")
    gi = torch.empty((N, C, H, W), dtype=torch.float32, device=x.device)
    check(_lib.load().novaq_max_pool2d_backward(g.data_ptr(), x.data_ptr(), DTYPES[xdt], N, C, H,
                                                W, KH, KW, sh, sw, ph, pw,
                                                PAD_MODES[padding_mode], gi.data_ptr(),
                                                _stream(x.device)), "max_pool2d_backward")
    return gi.cpu().numpy() if was_numpy else gi


def avg_pool2d_backward(grad, input_shape):
    """GlobalAvgPool2d's input gradient (novann/layers/pooling/gap/
    global_avg_pool2d.py:35-57): grad (N, C, 1, 1) spread over the (N, C, H, W)
    input shape as grad * float32(1 / (H*W)).  Returns fp32, an ndarray for a
    numpy grad."""
    N, C, H, W = input_shape
    g, was_numpy = _to_device_f32(grad, "grad")
    if g.numel() != N * C:
        raise ValueError(f"grad has {g.numel()} elements, not N*C = {N * C}")
    gi = torch.empty((N, C, H, W), dtype=torch.float32, device=g.device)
    check(_lib.load().novaq_global_avg_pool2d_backward(g.data_ptr(), N, C, H, W, gi.data_ptr(),
                                                       _stream(g.device)), "avg_pool2d_backward")
    return gi.cpu().numpy() if was_numpy else gi


def avg_pool2d(input):
    """Global average over H and W (novann/functional.py:548-559): returns
    (N, C, 1, 1) fp32, equal bit for bit to the reference's np.mean on the
    same float32 values (narrow inputs are decoded, FP8 times its scale)."""
    x, xdt, xs, xshape, was_numpy = _x_arg(input, "input")
    if len(xshape) != 4:
        raise ValueError(f"avg_pool2d expects (N, C, H, W), got {xshape}")
    N, C, H, W = xshape
    y = torch.empty((N, C, 1, 1), dtype=torch.float32, device=x.device)
    check(_lib.load().novaq_global_avg_pool2d(x.data_ptr(), DTYPES[xdt],
                                              None if xs is None else xs.data_ptr(), N, C, H, W,
                                              y.data_ptr(), _stream(x.device)), "avg_pool2d")
    return y.cpu().numpy() if was_numpy else y
