"""AdamW with NovaNN's interface (novann/optim/adamw.py:6-69), on the GPU.

Same constructor (parameters, lr, betas, weight_decay, epsilon), ``step`` and
``zero_grad``; BatchNorm gamma / beta (by name) are not decayed, as there.
Each step is the float32 update the reference computes on its float32 arrays,
bit for bit (libnovaq ``novaq_adamw_step``).  ``QuantizedParameters`` step
their fp32 ``master`` weights and re-quantize their codes and scale in the
same call (``novaq_adamw_requantize``).  ``Parameters`` holding numpy arrays
are stepped on a device copy and written back in place, so a caller that
keeps the arrays sees them change as with the reference.
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
            g = _dev_f32(p.grad, w.device).reshape(w.shape)
            is_bn_param = getattr(p, "name", None) in ("gamma", "beta")
            hp = _lib.AdamW(self.lr, self.b1, self.b2, self.eps, self.wd, self.t,
                            0 if is_bn_param else 1)
            stream = torch.cuda.current_stream(w.device).cuda_stream
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
