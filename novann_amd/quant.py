"""Cast, amax and per-tensor quantization on device tensors.

Thin host layer over the C ABI: torch provides the device memory and the
current HIP stream, libnovaq.so does the work.  Element storage:

  f32 -> torch.float32, f16 -> torch.float16, bf16 -> torch.bfloat16,
  e4m3 -> torch.float8_e4m3fn, e5m2 -> torch.float8_e5m2,
  e2m1 -> torch.uint8 holding ceil(n/2) bytes (element 2i in the low nibble).

The rounding / special-value rules are the ones in include/novaq.h.
NovaNN itself has no cast API; its only conversion is ``astype(np.float32)``
at layer entry (novann/layers/linear/linear.py:81).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch

from . import _lib
from ._lib import DTYPES, check

STORAGE = {
    "f32": torch.float32, "f16": torch.float16, "bf16": torch.bfloat16,
    "e4m3": torch.float8_e4m3fn, "e5m2": torch.float8_e5m2, "e2m1": torch.uint8,
}
QUANTIZED = ("e4m3", "e5m2", "e2m1")


def _dtype_code(name: str) -> int:
    try:
        return DTYPES[name]
    except KeyError:
        raise TypeError(f"unknown dtype '{name}', expected one of {tuple(DTYPES)}") from None


def storage_numel(dtype: str, n: int) -> int:
    """Number of storage elements holding n logical elements."""
    return (n + 1) // 2 if dtype == "e2m1" else n


_BITS = {"f32": 32, "f16": 16, "bf16": 16, "e4m3": 8, "e5m2": 8, "e2m1": 4}


def _require_holds(t: torch.Tensor, dtype: str, n: int, what: str) -> None:
    """ValueError unless t's storage holds n logical elements of dtype (the
    kernels would otherwise read or write past the end of the buffer)."""
    need = (n * _BITS[dtype] + 7) // 8
    have = t.numel() * t.element_size()
    if have < need:
        raise ValueError(f"{what} holds {have} bytes, {n} {dtype} elements need {need}")


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _require_device(t: torch.Tensor, what: str) -> None:
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise ValueError(f"{what} must be a CUDA (HIP) device tensor")
    if not t.is_contiguous():
        raise ValueError(f"{what} must be contiguous")


def _aligned16(t: torch.Tensor) -> torch.Tensor:
    """t itself when its data starts on a 16-byte boundary (what the kernels'
    vector accesses need), else an aligned copy: a view into a larger tensor
    works, at the cost of the copy."""
    return t if t.data_ptr() % 16 == 0 else t.clone()


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def dtype_of(t: torch.Tensor) -> str:
    for k, v in STORAGE.items():
        if t.dtype == v:
            return k
    raise TypeError(f"no novaq dtype is stored as {t.dtype}")


def cast(src: torch.Tensor, dst_dtype: str, *, src_dtype: Optional[str] = None,
         n: Optional[int] = None, scale: Optional[torch.Tensor] = None,
         out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Cast the n elements of ``src`` to ``dst_dtype``; returns a flat tensor.

    ``scale`` is a one-element fp32 device tensor s: quantizing encodes x/s
    (as x * (1/s)), dequantizing decodes q * s.  ``n`` defaults to the number
    of logical elements of src (2 per byte for e2m1)."""
    _require_device(src, "src")
    src_dtype = src_dtype or dtype_of(src)
    st, dt = _dtype_code(src_dtype), _dtype_code(dst_dtype)
    if n is None:
        n = src.numel() * 2 if src_dtype == "e2m1" else src.numel()
    n = int(n)
    if n < 0:
        raise ValueError(f"cast: negative element count {n}")
    _require_holds(src, src_dtype, n, "src")
    src = _aligned16(src)
    target = None
    if out is None:
        out = torch.empty(storage_numel(dst_dtype, n), dtype=STORAGE[dst_dtype],
                          device=src.device)
    else:
        _require_device(out, "out")
        if out.dtype != STORAGE[dst_dtype]:
            raise TypeError(f"out must be {STORAGE[dst_dtype]} for {dst_dtype}, got {out.dtype}")
        _require_holds(out, dst_dtype, n, "out")
        if out.data_ptr() % 16:
            # write into an aligned buffer, then copy into the caller's view
            target, out = out, torch.empty(storage_numel(dst_dtype, n),
                                           dtype=STORAGE[dst_dtype], device=src.device)
    if scale is not None:
        _require_device(scale, "scale")
        if scale.dtype != torch.float32:
            raise TypeError("scale must be float32")
    lib = _lib.load()
    check(lib.novaq_cast(src.data_ptr(), st, out.data_ptr(), dt, n, _ptr(scale),
                         _stream(src)), f"cast {src_dtype}->{dst_dtype}")
    if target is not None:
        target.reshape(-1)[:out.numel()].copy_(out)
        return target
    return out


def amax(x: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """NaN-ignoring max |x| as a one-element fp32 device tensor."""
    _require_device(x, "x")
    x = _aligned16(x)
    if out is None:
        out = torch.empty(1, dtype=torch.float32, device=x.device)
    check(_lib.load().novaq_amax(x.data_ptr(), _dtype_code(dtype_of(x)), x.numel(),
                                 out.data_ptr(), _stream(x)), "amax")
    return out


def scale_from_amax(a: torch.Tensor, dst_dtype: str) -> torch.Tensor:
    """s = amax / fmt_max (448 / 57344 / 6), or 1 if amax is 0 or not finite."""
    _require_device(a, "amax")
    out = torch.empty(1, dtype=torch.float32, device=a.device)
    check(_lib.load().novaq_scale_from_amax(a.data_ptr(), _dtype_code(dst_dtype),
                                            out.data_ptr(), _stream(a)), "scale_from_amax")
    return out


@dataclass
class Quantized:
    """Per-tensor quantized data: codes (flat storage), logical shape, dtype
    name and the device tensors amax and scale (one fp32 each)."""
    data: torch.Tensor
    shape: tuple
    dtype: str
    scale: torch.Tensor
    amax: Optional[torch.Tensor] = None

    @property
    def numel(self) -> int:
        n = 1
        for d in self.shape:
            n *= int(d)
        return n

    def check(self, what: str = "quantized tensor") -> None:
        """ValueError unless ``data`` holds the codes of prod(shape) elements."""
        if self.dtype not in QUANTIZED:
            raise TypeError(f"{what}: dtype must be one of {QUANTIZED}, got {self.dtype}")
        _require_device(self.data, f"{what} data")
        _require_holds(self.data, self.dtype, self.numel, f"{what} data")


def quantize(x: torch.Tensor, dst_dtype: str) -> Quantized:
    """amax -> s = amax / fmt_max -> encode(x * (1/s)), all on the device."""
    _require_device(x, "x")
    if dst_dtype not in QUANTIZED:
        raise TypeError(f"quantize target must be one of {QUANTIZED}")
    x = _aligned16(x)
    n = x.numel()
    data = torch.empty(storage_numel(dst_dtype, n), dtype=STORAGE[dst_dtype], device=x.device)
    st = torch.empty(2, dtype=torch.float32, device=x.device)
    check(_lib.load().novaq_quantize(x.data_ptr(), _dtype_code(dtype_of(x)), data.data_ptr(),
                                     _dtype_code(dst_dtype), n, st.data_ptr(), _stream(x)),
          f"quantize ->{dst_dtype}")
    return Quantized(data=data, shape=tuple(x.shape), dtype=dst_dtype, scale=st[1:2],
                     amax=st[0:1])


def dequantize(q: Quantized, dst_dtype: str = "f32") -> torch.Tensor:
    """decode(q) * s in the requested float type, reshaped to q.shape."""
    q.check()
    y = cast(q.data, dst_dtype, src_dtype=q.dtype, n=q.numel, scale=q.scale)
    return y.view(q.shape)


def pack_fp4(x: torch.Tensor, scale: Optional[torch.Tensor] = None) -> torch.Tensor:
    """fp32 -> E2M1, two elements per byte (element 2i in bits 3..0)."""
    if x.dtype != torch.float32:
        raise TypeError("pack_fp4 takes float32")
    return cast(x, "e2m1", scale=scale)


def unpack_fp4(packed: torch.Tensor, n: int, scale: Optional[torch.Tensor] = None
               ) -> torch.Tensor:
    """E2M1 bytes -> n fp32 values (times scale when given)."""
    return cast(packed, "f32", src_dtype="e2m1", n=n, scale=scale)
