"""novaq CPU oracle -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only as the checker (or the timed CPU
baseline).  The product path (``novann_amd``) never imports it.

It wraps ``oracle/liboracle.so`` (the C restatement in ``oracle.c``) with numpy
helpers, and holds ``functional_ref`` -- a numpy restatement of NovaNN's
``functional.linear`` / ``functional.conv2d`` (novann/functional.py:147-163,
:275-385).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

F32, F16, BF16, E4M3, E5M2, E2M1 = range(6)
PAD_MODES = {"zeros": 0, "reflect": 1, "replicate": 2, "circular": 3}

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

STORAGE = {F32: np.uint32, F16: np.uint16, BF16: np.uint16, E4M3: np.uint8,
           E5M2: np.uint8, E2M1: np.uint8}


def build() -> str:
    """Compile liboracle.so with the committed Makefile; returns its path."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)
    return _LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        u32, i32, i64, u64, vp, fp = (ctypes.c_uint32, ctypes.c_int, ctypes.c_int64,
                                      ctypes.c_uint64, ctypes.c_void_p, ctypes.c_float)
        for name, res, args in [
            ("novaq_ref_encode", u32, [u32, i32]),
            ("novaq_ref_decode", u32, [u32, i32]),
            ("novaq_bf_encode", u32, [u32, i32]),
            ("novaq_bf_decode", u32, [u32, i32]),
            ("novaq_ref_quantize_scaled", u32, [u32, fp, i32]),
            ("novaq_ref_dequantize_scaled", u32, [u32, fp, i32]),
            ("novaq_ref_cast", i32, [vp, i32, vp, i32, i64, vp, i32]),
            ("novaq_ref_amax", fp, [vp, i32, i64, i32]),
            ("novaq_ref_scale_from_amax", fp, [fp, i32]),
            ("novaq_ref_sweep_encode", i64, [i32, u64, u64, vp, i32]),
            ("novaq_ref_encode_range", None, [i32, u64, u64, vp, i32]),
            ("novaq_bf_encode_array", None, [vp, i64, i32, vp, i32]),
            ("novaq_ref_linear_f64", None, [vp, vp, vp, i64, i64, i64, vp, i32]),
            ("novaq_ref_conv2d_f64", i32, [vp, i64, i64, i64, i64, vp, i64, i32, i32,
                                           i32, i32, i32, i32, i32, vp, vp, i32]),
            ("novaq_ref_pad_index", i64, [i64, i64, i32]),
        ]:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def nbytes_of(dtype: int, n: int) -> int:
    if dtype == E2M1:
        return (n + 1) // 2
    return n * np.dtype(STORAGE[dtype]).itemsize


def cast(src: np.ndarray, src_dtype: int, dst_dtype: int, n: int | None = None,
         scale: float | None = None, nthreads: int = 0) -> np.ndarray:
    """Cast ``n`` elements held in the raw storage array ``src`` (uint view for
    16-bit / 8-bit / packed formats, float32 or uint32 for f32).  Returns the
    raw storage of the destination (float32 arrays come back as float32)."""
    src = np.ascontiguousarray(src)
    if n is None:
        n = src.size * 2 if src_dtype == E2M1 else src.size
    out = np.empty(nbytes_of(dst_dtype, n) // np.dtype(STORAGE[dst_dtype]).itemsize,
                   dtype=STORAGE[dst_dtype])
    sc = None if scale is None else np.array([scale], dtype=np.float32)
    rc = lib().novaq_ref_cast(_ptr(src), src_dtype, _ptr(out), dst_dtype, n, _ptr(sc),
                              nthreads)
    if rc != 0:
        raise ValueError(f"unsupported oracle cast {src_dtype}->{dst_dtype}")
    return out.view(np.float32) if dst_dtype == F32 else out


def amax(x: np.ndarray, dtype: int = F32, nthreads: int = 0) -> float:
    x = np.ascontiguousarray(x)
    return float(lib().novaq_ref_amax(_ptr(x), dtype, x.size, nthreads))


def scale_from_amax(a: float, dtype: int) -> float:
    return float(np.float32(lib().novaq_ref_scale_from_amax(a, dtype)))


def encode(bits: int, dtype: int) -> int:
    return lib().novaq_ref_encode(bits, dtype)


def decode(code: int, dtype: int) -> int:
    return lib().novaq_ref_decode(code, dtype)


def bf_encode(bits: int, dtype: int) -> int:
    return lib().novaq_bf_encode(bits, dtype)


def bf_decode(code: int, dtype: int) -> int:
    return lib().novaq_bf_decode(code, dtype)


def sweep_encode(dtype: int, begin: int, count: int, nthreads: int = 0):
    """(#mismatches fast vs brute force, first mismatching fp32 pattern)."""
    first = ctypes.c_uint32(0)
    bad = lib().novaq_ref_sweep_encode(dtype, begin, count, ctypes.byref(first), nthreads)
    return int(bad), int(first.value)


def bf_encode_array(bits: np.ndarray, dtype: int, nthreads: int = 0) -> np.ndarray:
    """Brute-force codes (uint32) of an array of fp32 bit patterns."""
    bits = np.ascontiguousarray(bits, dtype=np.uint32)
    out = np.empty(bits.size, dtype=np.uint32)
    lib().novaq_bf_encode_array(_ptr(bits), bits.size, dtype, _ptr(out), nthreads)
    return out


def encode_array(bits: np.ndarray, dtype: int, nthreads: int = 0) -> np.ndarray:
    """Fast-path codes (uint32) of an array of fp32 bit patterns."""
    bits = np.ascontiguousarray(bits, dtype=np.uint32)
    if dtype == E2M1:
        out = np.empty(bits.size, dtype=np.uint32)
        for lo in range(0, bits.size, 1 << 24):
            chunk = bits[lo:lo + (1 << 24)]
            packed = cast(chunk, F32, E2M1, nthreads=nthreads)
            nib = np.empty(packed.size * 2, dtype=np.uint32)
            nib[0::2] = packed & 0xF
            nib[1::2] = packed >> 4
            out[lo:lo + chunk.size] = nib[:chunk.size]
        return out
    return cast(bits, F32, dtype, nthreads=nthreads).view(STORAGE[dtype]).astype(np.uint32)


def encode_range(dtype: int, begin: int, count: int, nthreads: int = 0) -> np.ndarray:
    out = np.empty(count, dtype=np.uint16 if dtype in (F16, BF16) else np.uint8)
    lib().novaq_ref_encode_range(dtype, begin, count, _ptr(out), nthreads)
    return out


def linear_f64(x: np.ndarray, w: np.ndarray, bias: np.ndarray | None = None,
               nthreads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, D_in = x.shape
    D_out = w.shape[0]
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    y = np.empty((N, D_out), dtype=np.float32)
    lib().novaq_ref_linear_f64(_ptr(x), _ptr(w), _ptr(b), N, D_in, D_out, _ptr(y), nthreads)
    return y


def conv2d_f64(x: np.ndarray, w: np.ndarray, stride=(1, 1), padding=(0, 0),
               padding_mode: str = "zeros", bias: np.ndarray | None = None,
               nthreads: int = 0) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    w = np.ascontiguousarray(w, dtype=np.float32)
    N, C, H, W = x.shape
    C_out, _, KH, KW = w.shape
    sh, sw = stride
    ph, pw = padding
    OH = (H + 2 * ph - KH) // sh + 1
    OW = (W + 2 * pw - KW) // sw + 1
    b = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32).reshape(-1)
    y = np.empty((N, C_out, OH, OW), dtype=np.float32)
    rc = lib().novaq_ref_conv2d_f64(_ptr(x), N, C, H, W, _ptr(w), C_out, KH, KW, sh, sw,
                                    ph, pw, PAD_MODES[padding_mode], _ptr(b), _ptr(y),
                                    nthreads)
    if rc != 0:
        raise ValueError("bad conv2d arguments")
    return y


def pad_index(i: int, n: int, mode: str) -> int:
    return int(lib().novaq_ref_pad_index(i, n, PAD_MODES[mode]))
