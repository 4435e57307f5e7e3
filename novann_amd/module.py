"""Parameter containers, the module / layer contract, and layers with
NovaNN's interface.

``Parameters`` mirrors novann/module/module.py:6-38 (``.data``, ``.grad``,
``.name``), ``Module`` its train / eval / parameters / zero_grad contract
(module.py:41-85) and ``Layer`` the callable forward / backward base
(module/layer.py:6-59).  ``QuantizedParameters`` is the packed replacement of
``.data`` for quantized weights: device codes (E4M3 / E5M2 / E2M1) plus a
per-tensor scale.  ``Linear`` mirrors novann/layers/linear/linear.py:10-118
and ``Conv2d`` novann/layers/convolutional/conv2d.py:9-217: same constructor
arguments, ``reset_parameters`` with the reference's default initialisers
drawn from numpy's global generator (so a seeded construction gives the
reference's weights), parameter shapes, the float32 coercion of numpy inputs,
forward and backward; both call the GPU operators in ``functional``.
``BatchNorm2d`` / ``BatchNorm1d`` hold the reference's parameters and running
statistics (batchnorm2d.py:33-55, batchnorm1d.py:33-55) and ``ReLU`` stands
for novann's ReLU layer; on this path they run fused into the product before
them (``fuse``), in eval mode.
"""
from __future__ import annotations

from abc import ABC, abstractmethod
from typing import Optional

import numpy as np
import torch

from .init import DEFAULT_NORMAL_INIT_MAP, DEFAULT_UNIFORM_INIT_MAP


class Parameters:
    """Holds a parameter array and its gradient (module.py:6-38)."""

    def __init__(self, data) -> None:
        self.data = data
        self.grad = np.zeros_like(data) if isinstance(data, np.ndarray) else None
        self.name: Optional[str] = None

    @property
    def shape(self):
        return tuple(self.data.shape)

    def zero_grad(self, set_to_none: bool = True) -> None:
        if set_to_none:
            self.grad = None
        elif self.grad is None:
            self.grad = (torch.zeros_like(self.data) if isinstance(self.data, torch.Tensor)
                         else np.zeros_like(self.data))
        elif isinstance(self.grad, torch.Tensor):
            self.grad.zero_()
        else:
            self.grad.fill(0.0)


class QuantizedParameters:
    """Per-tensor quantized weight resident on the device: the packed
    replacement of ``Parameters.data`` (module.py:20-23).

    codes: flat device tensor of codes (E2M1: two per byte, element 2i in the
    low nibble, rows of the innermost dimension packed contiguously); shape:
    logical shape; dtype: 'e4m3' | 'e5m2' | 'e2m1'; scale: one fp32 device
    value s, the weight being s * decode(codes); amax: max |w| the scale was
    derived from.  For training, ``master`` holds the fp32 weights the
    optimizer steps (the codes are re-quantized from them after each step)
    and ``grad`` the gradient of the dequantized weight.

    A 2-D E2M1 weight (a Linear's (out, in)) with an odd number of columns
    keeps whole bytes per row: codes and master carry one zero column more
    (``padded_cols``), whose +0 codes the products never read; a zero column
    changes neither the amax nor, under AdamW (zero gradient), its value."""

    def __init__(self, codes: torch.Tensor, shape, dtype: str, scale: torch.Tensor,
                 amax: Optional[torch.Tensor] = None, name: Optional[str] = None,
                 master: Optional[torch.Tensor] = None):
        self.codes = codes
        self.shape = tuple(int(d) for d in shape)
        self.dtype = dtype
        self.scale = scale
        self.amax = amax
        self.name = name
        self.master = master
        self.grad = None

    @property
    def padded_cols(self) -> int:
        """Columns per stored row: the logical ones, plus one pad column for an
        odd-width 2-D E2M1 weight."""
        cols = self.shape[-1] if self.shape else 1
        pad = self.dtype == "e2m1" and len(self.shape) == 2 and cols % 2 == 1
        return cols + 1 if pad else cols

    @property
    def stored_shape(self) -> tuple:
        return self.shape[:-1] + (self.padded_cols,) if self.shape else self.shape

    @classmethod
    def from_float(cls, w, dtype: str, device=None,
                   keep_master: bool = False) -> "QuantizedParameters":
        """Quantize an fp32 array with per-tensor amax scaling on the GPU
        (keeping an fp32 device copy as ``master`` when asked)."""
        from . import quant
        if isinstance(w, Parameters):
            w = w.data
        if isinstance(w, np.ndarray):
            dev = device or torch.device("cuda", torch.cuda.current_device())
            w = torch.from_numpy(np.ascontiguousarray(w, dtype=np.float32)).to(dev)
        w = w.to(torch.float32).contiguous()
        shape = tuple(w.shape)
        if dtype == "e2m1" and w.dim() == 2 and w.shape[1] % 2 == 1:
            w = torch.nn.functional.pad(w, (0, 1))  # whole bytes per row
        q = quant.quantize(w, dtype)
        master = w.clone() if keep_master else None
        return cls(q.data, shape, dtype, q.scale, q.amax, master=master)

    def zero_grad(self, set_to_none: bool = True) -> None:
        if set_to_none or self.grad is None:
            self.grad = None
        elif isinstance(self.grad, torch.Tensor):
            self.grad.zero_()
        else:
            self.grad.fill(0.0)

    def dequantize(self) -> torch.Tensor:
        """s * decode(codes) as an fp32 device tensor of the logical shape."""
        from . import quant
        y = quant.dequantize(quant.Quantized(self.codes, self.stored_shape, self.dtype,
                                             self.scale), "f32")
        return y if self.stored_shape == self.shape else y[..., :self.shape[-1]].contiguous()


class Module:
    """Train / eval mode and parameter access (module.py:41-85): modules start
    in training mode; ``parameters()`` is empty unless a subclass owns some;
    ``zero_grad`` clears every parameter's gradient (``set_to_none`` as
    Parameters.zero_grad)."""

    def __init__(self) -> None:
        self._training = True

    def train(self) -> None:
        self._training = True

    def eval(self) -> None:
        self._training = False

    def parameters(self):
        return []

    def zero_grad(self) -> None:
        for p in self.parameters():
            p.zero_grad()


class Layer(Module, ABC):
    """A module called as ``layer(x)`` -> ``forward(x)``, with ``backward``
    (module/layer.py:6-59)."""

    def __call__(self, x):
        return self.forward(x)

    @abstractmethod
    def forward(self, x):
        raise NotImplementedError("Layer subclasses must implement forward method")

    @abstractmethod
    def backward(self, grad):
        raise NotImplementedError("Layer subclasses must implement backward method")


def _as_f32(x):
    """The reference's layer-entry coercion ``x.astype(np.float32, copy=False)``
    (linear.py:81, conv2d.py:159) for numpy inputs; device tensors and
    quantized activations are the products' own input formats and pass as
    they are, except float64, which becomes float32 as in numpy."""
    if isinstance(x, np.ndarray):
        return x.astype(np.float32, copy=False)
    if isinstance(x, torch.Tensor) and x.dtype == torch.float64:
        return x.float()
    return x


def _pair(v):
    if isinstance(v, int):
        return (v, v)
    if isinstance(v, str):
        if v == "valid":
            return (0, 0)
        if v == "same":
            raise ValueError("The 'same' value is not currently supported")
        raise ValueError(f"Unsupported value '{v}'")
    return tuple(v)


class Linear(Layer):
    """Linear with an fp32 or quantized weight (linear.py:10-118).

    weight (out_features, in_features); bias (1, out_features) zeros.
    ``reset_parameters`` draws the weight with ``initializer``, else ``init``,
    else DEFAULT_NORMAL_INIT_MAP["default"] (``random_init_``, linear.py:47-68),
    from numpy's global generator; ``weight_dtype`` ('e4m3' | 'e5m2' | 'e2m1')
    then stores it quantized (per-tensor amax scale, fp32 master kept for the
    optimizer).  The forward input, coerced to float32 as linear.py:81 does,
    is cached for ``backward``."""

    def __init__(self, in_features: int, out_features: int, bias: bool = True, init=None,
                 weight_dtype: Optional[str] = None) -> None:
        super().__init__()
        self.in_features, self.out_features = in_features, out_features
        self.use_bias = bias
        self.init_fn = init
        self.weight_dtype = weight_dtype
        self.weight = None
        self.bias = None
        self._cache_input = None
        self.reset_parameters()

    def reset_parameters(self, initializer=None) -> None:
        init = initializer or self.init_fn or DEFAULT_NORMAL_INIT_MAP["default"]
        w = init((self.out_features, self.in_features))
        self.weight = Parameters(np.asarray(w, dtype=np.float32))
        self.weight.name = "linear weight"
        if self.weight_dtype is not None:
            self.weight = QuantizedParameters.from_float(self.weight, self.weight_dtype,
                                                         keep_master=True)
            self.weight.name = "linear weight"
        self.bias = None
        if self.use_bias:
            self.bias = Parameters(np.zeros((1, self.out_features), dtype=np.float32))
            self.bias.name = "linear bias"

    def forward(self, x):
        from . import functional as F
        x = _as_f32(x)
        self._cache_input = x
        return F.linear(x, self.weight, self.bias)

    def backward(self, grad):
        """Sets weight.grad = grad.T @ x and bias.grad = grad summed over the
        batch, returns grad @ W (linear.py:85-108)."""
        from . import functional as F
        gi, gw, gb = F.linear_backward(_as_f32(grad), self._cache_input, self.weight,
                                       self.bias is not None)
        self.weight.grad = gw
        if self.bias is not None:
            self.bias.grad = gb
        return gi

    def parameters(self):
        return [self.weight] + ([self.bias] if self.bias is not None else [])

    def __repr__(self) -> str:
        return (f"Linear(in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.use_bias})")


class Conv2d(Layer):
    """Conv2d with an fp32 or quantized weight (conv2d.py:9-217).

    weight (out_channels, in_channels, KH, KW); bias (out_channels, 1) zeros;
    stride defaults to 1 (a None stride means kernel_size, conv2d.py:41).
    ``reset_parameters`` draws the weight with ``initializer``, else ``init``,
    else DEFAULT_UNIFORM_INIT_MAP["relu"] (Kaiming-uniform for ReLU,
    conv2d.py:55-72), from numpy's global generator; ``weight_dtype`` stores it
    quantized as in Linear.  The forward input, coerced to float32 as
    conv2d.py:159 does, is cached for ``backward`` (the reference caches its
    im2col matrix, conv2d.py:173-175; this path never builds one)."""

    def __init__(self, in_channels: int, out_channels: int, kernel_size, stride=1,
                 padding=0, bias: bool = True, padding_mode: str = "zeros", init=None,
                 weight_dtype: Optional[str] = None) -> None:
        super().__init__()
        self.in_channels, self.out_channels = in_channels, out_channels
        self.KH, self.KW = _pair(kernel_size)
        self.sh, self.sw = _pair(stride if stride is not None else kernel_size)
        self.ph, self.pw = _pair(padding)
        self.pm = padding_mode
        self.init_fn = init
        self.use_bias = bias
        self.weight_dtype = weight_dtype
        self.weight = None
        self.bias = None
        self._cache_input = None
        self.reset_parameters()

    def reset_parameters(self, initializer=None) -> None:
        init = initializer or self.init_fn or DEFAULT_UNIFORM_INIT_MAP["relu"]
        w = init((self.out_channels, self.in_channels, self.KH, self.KW))
        self.weight = Parameters(np.asarray(w, dtype=np.float32))
        self.weight.name = "conv2d weight"
        if self.weight_dtype is not None:
            self.weight = QuantizedParameters.from_float(self.weight, self.weight_dtype,
                                                         keep_master=True)
            self.weight.name = "conv2d weight"
        self.bias = None
        if self.use_bias:
            self.bias = Parameters(np.zeros((self.out_channels, 1), dtype=np.float32))
            self.bias.name = "conv2d bias"

    def forward(self, x):
        from . import functional as F
        x = _as_f32(x)
        self._cache_input = x
        return F.conv2d(x, self.weight, (self.KH, self.KW), (self.sh, self.sw),
                        (self.ph, self.pw), bias=self.bias, padding_mode=self.pm)

    def backward(self, grad):
        """Sets weight.grad and bias.grad, returns the input gradient
        (conv2d.py:179-207)."""
        from . import functional as F
        gi, gw, gb = F.conv2d_backward(_as_f32(grad), self._cache_input, self.weight,
                                       (self.KH, self.KW), (self.sh, self.sw),
                                       (self.ph, self.pw), bias=self.bias is not None,
                                       padding_mode=self.pm)
        self.weight.grad = gw
        if self.bias is not None:
            self.bias.grad = gb
        return gi

    def parameters(self):
        return [self.weight] + ([self.bias] if self.bias is not None else [])


class _BatchNorm(Module):
    """Parameters and running statistics of novann's BatchNorm layers, used
    as an eval-mode epilogue of the product before them."""

    _shape_tail: tuple = ()

    def __init__(self, num_features: int, momentum: float = 0.1, eps: float = 1e-5) -> None:
        super().__init__()
        self.num_features = int(num_features)
        self.momentum, self.eps = float(momentum), float(eps)
        shape = (1, self.num_features) + self._shape_tail
        self.gamma = Parameters(np.ones(shape))
        self.beta = Parameters(np.zeros(shape))
        self.gamma.name, self.beta.name = "gamma", "beta"
        self.running_mean = np.zeros(shape)
        self.running_var = np.ones(shape)

    def epilogue(self, relu: bool = False, **kw):
        """The fused epilogue gamma * (v - mean) / sqrt(var + eps) + beta
        (batchnorm2d.py:98-102), then ReLU when ``relu``."""
        from .functional import Epilogue
        return Epilogue.batchnorm(self.gamma.data, self.beta.data, self.running_mean,
                                  self.running_var, self.eps, relu=relu, **kw)

    def parameters(self):
        return [self.gamma, self.beta]


class BatchNorm2d(_BatchNorm):
    """novann BatchNorm2d's state (batchnorm2d.py:33-55): (1, C, 1, 1) arrays."""
    _shape_tail = (1, 1)


class BatchNorm1d(_BatchNorm):
    """novann BatchNorm1d's state (batchnorm1d.py:33-55): (1, C) arrays."""
    _shape_tail = ()


class ReLU(Module):
    """novann's ReLU layer (relu.py:8-48): x * (x > 0), fused into the
    product before it."""


class Fused(Module):
    """A Linear or Conv2d followed by an eval-mode BatchNorm and / or a ReLU,
    run as one product whose epilogue applies them (the layers that follow a
    product on novann's main path, main.py:24-46).  ``out_dtype`` 'bf16',
    'f16', 'e4m3' or 'e5m2' stores the activation narrow for the next product
    (FP8 with ``out_scale``, e.g. from a calibration pass's ``out_amax``)."""

    def __init__(self, layer, bn: Optional[_BatchNorm] = None, relu: bool = False,
                 out_dtype: str = "f32", out_scale=None) -> None:
        if not isinstance(layer, (Linear, Conv2d)):
            raise TypeError("fuse: the first layer must be a Linear or a Conv2d")
        want = BatchNorm2d if isinstance(layer, Conv2d) else BatchNorm1d
        if bn is not None and not isinstance(bn, want):
            raise TypeError(f"fuse: {type(layer).__name__} is followed by {want.__name__}")
        super().__init__()
        self.layer, self.bn, self.relu = layer, bn, relu
        self.out_dtype, self.out_scale = out_dtype, out_scale

    def parameters(self):
        return self.layer.parameters() + (self.bn.parameters() if self.bn is not None else [])

    def __call__(self, x, out_amax=None):
        return self.forward(x, out_amax)

    def forward(self, x, out_amax=None):
        from . import functional as F
        kw = dict(relu=self.relu, out_dtype=self.out_dtype, out_scale=self.out_scale,
                  out_amax=out_amax)
        ep = self.bn.epilogue(**kw) if self.bn is not None else F.Epilogue(**kw)
        L = self.layer
        if isinstance(L, Linear):
            return F.linear(x, L.weight, L.bias, epilogue=ep)
        return F.conv2d(x, L.weight, (L.KH, L.KW), (L.sh, L.sw), (L.ph, L.pw), bias=L.bias,
                        padding_mode=L.pm, epilogue=ep)


def fuse(*layers, out_dtype: str = "f32", out_scale=None) -> Fused:
    """Fuse [Linear | Conv2d] [BatchNorm1d | BatchNorm2d] [ReLU] into one layer."""
    if not layers:
        raise ValueError("fuse: no layers")
    head, rest = layers[0], list(layers[1:])
    bn = rest.pop(0) if rest and isinstance(rest[0], _BatchNorm) else None
    relu = bool(rest) and isinstance(rest[0], ReLU)
    if relu:
        rest.pop(0)
    if rest:
        raise ValueError(f"fuse: cannot fuse {type(rest[0]).__name__} after "
                         f"{type(head).__name__}")
    return Fused(head, bn, relu, out_dtype, out_scale)


class MaxPool2d(Module):
    """novann MaxPool2d (layers/pooling/maxpool/maxpool2d.py:8-132): kernel,
    stride (None = kernel size), padding, padding_mode; forward and backward
    on the GPU.  The forward input is cached for ``backward`` (the reference
    caches its window view, :63-75) and released by it (:123)."""

    def __init__(self, kernel_size, stride=None, padding=0, padding_mode: str = "zeros") -> None:
        super().__init__()
        self.KH, self.KW = _pair(kernel_size)
        self.sh, self.sw = _pair(stride if stride is not None else kernel_size)
        self.ph, self.pw = _pair(padding)
        self.pm = padding_mode
        self._cache_input = None

    def __call__(self, x):
        return self.forward(x)

    def forward(self, x):
        from . import functional as F
        self._cache_input = x
        return F.max_pool2d(x, (self.KH, self.KW), (self.sh, self.sw), (self.ph, self.pw),
                            padding_mode=self.pm)

    def backward(self, grad):
        """The input gradient (maxpool2d.py:79-129)."""
        from . import functional as F
        if self._cache_input is None:
            raise RuntimeError("MaxPool2d.backward called without a forward")
        gi = F.max_pool2d_backward(grad, self._cache_input, (self.KH, self.KW),
                                   (self.sh, self.sw), (self.ph, self.pw), padding_mode=self.pm)
        self._cache_input = None
        return gi


class GlobalAvgPool2d(Module):
    """novann GlobalAvgPool2d (layers/pooling/gap/global_avg_pool2d.py:7-57):
    (N, C, H, W) -> (N, C, 1, 1) means and their input gradient, on the GPU;
    the forward caches the input shape (:30)."""

    def __init__(self) -> None:
        super().__init__()
        self._x_shape = None

    def __call__(self, x):
        return self.forward(x)

    def forward(self, x):
        from . import functional as F
        self._x_shape = tuple(x.shape)
        return F.avg_pool2d(x)

    def backward(self, grad):
        """grad / (H*W) over each plane (global_avg_pool2d.py:35-57)."""
        from . import functional as F
        if self._x_shape is None:
            raise RuntimeError("GlobalAvgPool2d.backward called without a forward")
        return F.avg_pool2d_backward(grad, self._x_shape)
