"""Device <-> host helpers for the GPU tests (raw bit patterns, no rounding)."""
from __future__ import annotations

import numpy as np
import torch

import oracle as O

_INT_VIEW = {1: np.uint8, 2: np.int16, 4: np.int32}
_TORCH_INT = {1: torch.uint8, 2: torch.int16, 4: torch.int32}
TORCH_STORAGE = {O.F32: torch.float32, O.F16: torch.float16, O.BF16: torch.bfloat16,
                 O.E4M3: torch.float8_e4m3fn, O.E5M2: torch.float8_e5m2, O.E2M1: torch.uint8}
NAME = {O.F32: "f32", O.F16: "f16", O.BF16: "bf16", O.E4M3: "e4m3", O.E5M2: "e5m2",
        O.E2M1: "e2m1"}


def to_dev(arr: np.ndarray, dtype: int) -> torch.Tensor:
    """Upload raw storage (uint8/uint16/uint32/float32 array) as the torch
    storage dtype of `dtype` without changing a bit."""
    arr = np.ascontiguousarray(arr)
    size = arr.dtype.itemsize
    t = torch.from_numpy(arr.view(_INT_VIEW[size])).cuda()
    return t.view(TORCH_STORAGE[dtype])


def to_host(t: torch.Tensor) -> np.ndarray:
    """Raw storage bits of a device tensor as an unsigned numpy array."""
    size = t.element_size()
    raw = t.view(_TORCH_INT[size]).cpu().numpy()
    return raw.view({1: np.uint8, 2: np.uint16, 4: np.uint32}[size])


def first_mismatch(got: np.ndarray, want: np.ndarray, inputs: np.ndarray | None = None):
    bad = np.nonzero(got != want)[0]
    if bad.size == 0:
        return None
    i = bad[0]
    inp = "" if inputs is None else f" input=0x{int(inputs[i]):08x}"
    return f"{bad.size} mismatches; first at {i}:{inp} got=0x{int(got[i]):x} want=0x{int(want[i]):x}"


def bf16_round(a: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 (nearest even) -> fp32, by the oracle's cast: the operand
    values the bf16 MFMA products multiply."""
    flat = np.ascontiguousarray(a, np.float32).reshape(-1)
    return O.cast(O.cast(flat, O.F32, O.BF16), O.BF16, O.F32).reshape(a.shape)


def error_report(y: np.ndarray, r: np.ndarray) -> dict:
    """Normwise max|y - r| / max|r| (the gate) and the elementwise relative
    error with a floor, max |y - r| / max(|r|, f * max|r|), for floors f of
    1e-3 and 1e-2, plus the share of elements within 1e-2 relative error."""
    d = np.abs(y.astype(np.float64) - r)
    m = max(float(np.abs(r).max()), 1e-30)
    a = np.abs(r)
    return {"normwise": float(d.max() / m),
            "elem_floor1e-3": float((d / np.maximum(a, 1e-3 * m)).max()),
            "elem_floor1e-2": float((d / np.maximum(a, 1e-2 * m)).max()),
            "share_within_1e-2": float(np.mean(d <= 1e-2 * a))}
