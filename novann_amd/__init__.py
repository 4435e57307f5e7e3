"""novann_amd -- MI355X-native quantized-dtype hot path for NovaNN layers.

Casts fp32/fp16/bf16 <-> FP8 (E4M3, E5M2) and FP4 (E2M1, nibble-packed) with
per-tensor amax scaling, and the Linear / Conv2d forward products on
quantized weights, all as HIP kernels for gfx950 in ``libnovaq.so`` behind
the C ABI of ``include/novaq.h``.  This package is the host side: it mirrors
NovaNN's ``functional.linear`` / ``functional.conv2d`` and its ``Linear`` /
``Conv2d`` layers.
"""
from . import _lib
from ._lib import LIB_PATH, load

__version__ = "0.1.0"

__all__ = ["LIB_PATH", "load", "quant", "functional", "module"]


def __getattr__(name):
    # Lazy submodules: importing the package does not import torch.
    if name in ("quant", "functional", "module"):
        import importlib
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
