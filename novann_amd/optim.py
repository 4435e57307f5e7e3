"""AdamW with NovaNN's interface (novann/optim/adamw.py:6-69), on the GPU.

Same constructor (parameters, lr, betas, weight_decay, epsilon), ``step`` and
``zero_grad``; BatchNorm gamma / beta (by name) are not decayed, as there.
Each step is the float32 update the reference computes on its float32 arrays,
bit for bit (libnovaq ``novaq_adamw_step``).  ``QuantizedParameters`` step
their fp32 ``master`` weights and re-quantize their codes and scale in the
same call (``novaq_adamw_requantize``).  ``Parameters`` holding numpy arrays
are uploaded at every step (so changes a caller makes to ``.data`` between
steps count, as with the reference), stepped on the device and written back
in place.  float64 arrays (the BatchNorm gamma / beta, float64 in the
reference too) keep float64 moments and step in float64 with numpy's
promotion of a float32 gradient (``novaq_adamw_step_f64``); any other numpy
array steps in float32 (the reference's float32 parameters).
"""
from __future__ import annotations

import ctypes
from typing import Iterable, List, Optional

import numpy as np
import torch

from . import _lib
from ._lib import DTYPES, check
from .module import Parameters, QuantizedParameters


def _device() -> torch.device:
    if not torch.cuda.is_available():
        raise RuntimeError("novann_amd needs a HIP device (no CPU fallback)")
    return torch.device("cuda", torch.cuda.current_device())


def _dev_f32(a, dev) -> torch.Tensor:
    if isinstance(a, np.ndarray):
        return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dev)
    return a.to(device=dev, dtype=torch.float32).contiguous()


def _is_f64(p) -> bool:
    d = getattr(p, "data", None)
    return isinstance(d, np.ndarray) and d.dtype == np.float64


def _dev_grad64(g, dev):
    """A float64 parameter's gradient on the device in the dtype numpy would
    compute with: float32 stays float32, anything else becomes float64."""
    if isinstance(g, torch.Tensor):
        g = g.detach().cpu().numpy()
    g = np.asarray(g)
    dt = np.float32 if g.dtype == np.float32 else np.float64
    return torch.from_numpy(np.ascontiguousarray(g, dtype=dt)).to(dev), dt == np.float32


class AdamW:
    """AdamW with decoupled weight decay (adamw.py:6-69)."""

    def __init__(self, parameters: Iterable, lr: float, betas=(0.9, 0.999),
                 weight_decay: float = 0, epsilon: float = 1e-8) -> None:
        self.params: List = list(parameters)
        self.lr, self.wd = float(lr), float(weight_decay)
        self.b1, self.b2 = float(betas[0]), float(betas[1])
        self.eps = float(epsilon)
        self.t = 0
        dev = _device()
        self._w: List[torch.Tensor] = []
        for p in self.params:
            if isinstance(p, QuantizedParameters):
                if p.master is None:
                    raise ValueError("AdamW: a QuantizedParameters needs fp32 master weights "
                                     "(QuantizedParameters.from_float(..., keep_master=True))")
                self._w.append(p.master)
            elif _is_f64(p):
                self._w.append(torch.from_numpy(np.ascontiguousarray(p.data)).to(dev))
            elif isinstance(p.data, np.ndarray):
                self._w.append(_dev_f32(p.data, dev))
            else:
                if p.data.dtype != torch.float32 or not p.data.is_contiguous():
                    raise TypeError("AdamW: device parameters must be contiguous float32")
                self._w.append(p.data)
        self.m_t = [torch.zeros_like(w) for w in self._w]
        self.v_t = [torch.zeros_like(w) for w in self._w]
        self._amax_scale: List[Optional[torch.Tensor]] = [
            torch.empty(2, dtype=torch.float32, device=dev)
            if isinstance(p, QuantizedParameters) else None for p in self.params]

    def step(self) -> None:
        """One optimization step (adamw.py:41-65)."""
        self.t += 1
        lib = _lib.load()
        for i, p in enumerate(self.params):
            if p.grad is None:
                continue
            w = self._w[i]
            if isinstance(getattr(p, "data", None), np.ndarray):
                # the caller may have changed .data since the last step
                w.copy_(torch.from_numpy(np.ascontiguousarray(p.data).reshape(w.shape).astype(
                    np.float64 if w.dtype == torch.float64 else np.float32, copy=False)))
            is_bn_param = getattr(p, "name", None) in ("gamma", "beta")
            hp = _lib.AdamW(self.lr, self.b1, self.b2, self.eps, self.wd, self.t,
                            0 if is_bn_param else 1)
            stream = torch.cuda.current_stream(w.device).cuda_stream
            if w.dtype == torch.float64:
                g, g32 = _dev_grad64(p.grad, w.device)
                if g.numel() != w.numel():
                    raise ValueError(f"AdamW: gradient of {g.numel()} values for a parameter "
                                     f"of {w.numel()}")
                check(lib.novaq_adamw_step_f64(
                    w.data_ptr(), g.data_ptr(), int(g32), self.m_t[i].data_ptr(),
                    self.v_t[i].data_ptr(), w.numel(), ctypes.byref(hp), stream), "adamw f64")
                p.data[...] = w.cpu().numpy().reshape(p.data.shape)
                continue
            g = _dev_f32(p.grad, w.device)
            if isinstance(p, QuantizedParameters) and p.stored_shape != p.shape:
                # the pad column of an odd-width E2M1 weight: zero gradient
                g = torch.nn.functional.pad(g.reshape(p.shape), (0, 1))
            g = g.reshape(w.shape)
            if isinstance(p, QuantizedParameters):
                st = self._amax_scale[i]
                check(lib.novaq_adamw_requantize(
                    w.data_ptr(), g.data_ptr(), self.m_t[i].data_ptr(), self.v_t[i].data_ptr(),
                    w.numel(), ctypes.byref(hp), p.codes.data_ptr(), DTYPES[p.dtype],
                    st.data_ptr(), stream), "adamw requantize")
                # the codes and scale the products read now follow the master
                # (the next step rewrites st after this step's readers, in
                # stream order)
                p.amax, p.scale = st[0:1], st[1:2]
            else:
                check(lib.novaq_adamw_step(
                    w.data_ptr(), g.data_ptr(), self.m_t[i].data_ptr(), self.v_t[i].data_ptr(),
                    w.numel(), ctypes.byref(hp), None, stream), "adamw step")
                if isinstance(p.data, np.ndarray):
                    p.data[...] = w.cpu().numpy().reshape(p.data.shape)

    def zero_grad(self, set_to_none: bool = False) -> None:
        """Clears the gradients of all optimized parameters (adamw.py:67-70)."""
        for p in self.params:
            p.zero_grad(set_to_none=set_to_none)
