"""ctypes binding of libnovaq.so (the C ABI in include/novaq.h).

The library is loaded from this package directory.  There is no fallback:
if it is missing, importing fails with instructions to build it.
"""
from __future__ import annotations

import ctypes
import os

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_PKG, "libnovaq.so")

F32, F16, BF16, E4M3, E5M2, E2M1 = range(6)
DTYPES = {"f32": F32, "f16": F16, "bf16": BF16, "e4m3": E4M3, "e5m2": E5M2, "e2m1": E2M1}
DTYPE_NAMES = {v: k for k, v in DTYPES.items()}
PAD_MODES = {"zeros": 0, "reflect": 1, "replicate": 2, "circular": 3}

OK, EINVAL, EDTYPE, ESHAPE, EPADMODE, EALIGN, EHIP, ENOTSUP, ESCRATCH = (
    0, -1, -2, -3, -4, -5, -6, -7, -8)



class Epilogue(ctypes.Structure):
    """struct novaq_epilogue (include/novaq.h); pointers are device addresses."""
    _fields_ = [("channel_mul", ctypes.c_void_p), ("channel_add", ctypes.c_void_p),
                ("out_scale", ctypes.c_void_p), ("out_amax", ctypes.c_void_p),
                ("relu", ctypes.c_int), ("out_dtype", ctypes.c_int)]


class AdamW(ctypes.Structure):
    """struct novaq_adamw (include/novaq.h)."""
    _fields_ = [("lr", ctypes.c_double), ("beta1", ctypes.c_double),
                ("beta2", ctypes.c_double), ("eps", ctypes.c_double),
                ("weight_decay", ctypes.c_double), ("step", ctypes.c_int64),
                ("decay", ctypes.c_int)]


# Every symbol include/novaq.h declares, with its ctypes signature.
_vp, _i32, _i64, _f32p = ctypes.c_void_p, ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
_epip = ctypes.POINTER(Epilogue)
SIGNATURES = {
    "novaq_version": (_i32, []),
    "novaq_status_string": (ctypes.c_char_p, [_i32]),
    "novaq_last_hip_error": (_i32, []),
    "novaq_cast": (_i32, [_vp, _i32, _vp, _i32, _i64, _f32p, _vp]),
    "novaq_amax": (_i32, [_vp, _i32, _i64, _f32p, _vp]),
    "novaq_scale_from_amax": (_i32, [_f32p, _i32, _f32p, _vp]),
    "novaq_quantize": (_i32, [_vp, _i32, _vp, _i32, _i64, _f32p, _vp]),
    "novaq_pack_fp4": (_i32, [_f32p, _i64, _f32p, _vp, _vp]),
    "novaq_unpack_fp4": (_i32, [_vp, _i64, _f32p, _f32p, _vp]),
    "novaq_linear_forward": (_i32, [_f32p, _i64, _i64, _vp, _i32, _f32p, _f32p, _i64, _f32p,
                                    _vp]),
    "novaq_conv2d_forward": (_i32, [_f32p, _i64, _i64, _i64, _i64, _vp, _i32, _f32p, _i64,
                                    _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32p, _f32p,
                                    _vp]),
    "novaq_linear_forward_ex": (_i32, [_vp, _i32, _f32p, _i64, _i64, _vp, _i32, _f32p, _f32p,
                                       _i64, _epip, _vp, _vp]),
    "novaq_conv2d_forward_ex": (_i32, [_vp, _i32, _f32p, _i64, _i64, _i64, _i64, _vp, _i32,
                                       _f32p, _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32,
                                       _f32p, _epip, _vp, _vp]),
    "novaq_max_pool2d": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32, _i32,
                                _i32, _i32, _vp, _vp]),
    "novaq_global_avg_pool2d": (_i32, [_vp, _i32, _f32p, _i64, _i64, _i64, _i64, _f32p, _vp]),
    "novaq_max_pool2d_backward": (_i32, [_f32p, _vp, _i32, _i64, _i64, _i64, _i64, _i32, _i32,
                                         _i32, _i32, _i32, _i32, _i32, _f32p, _vp]),
    "novaq_global_avg_pool2d_backward": (_i32, [_f32p, _i64, _i64, _i64, _i64, _f32p, _vp]),
    "novaq_im2col": (_i32, [_vp, _i32, _f32p, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _i32,
                            _i32, _i32, _i32, _f32p, _vp]),
    "novaq_pad2d": (_i32, [_vp, _i32, _i64, _i64, _i64, _i64, _i32, _i32, _i32, _vp, _vp]),
    "novaq_adamw_step": (_i32, [_f32p, _f32p, _f32p, _f32p, _i64, ctypes.POINTER(AdamW), _f32p,
                                _vp]),
    "novaq_adamw_step_f64": (_i32, [_vp, _vp, _i32, _vp, _vp, _i64, ctypes.POINTER(AdamW), _vp]),
    "novaq_adamw_requantize": (_i32, [_f32p, _f32p, _f32p, _f32p, _i64, ctypes.POINTER(AdamW),
                                      _vp, _i32, _f32p, _vp]),
    "novaq_transpose": (_i32, [_vp, _i32, _i64, _i64, _vp, _i32, _vp]),
    "novaq_colsum": (_i32, [_f32p, _i64, _i64, _f32p, _vp]),
    "novaq_linear_backward_workspace": (ctypes.c_size_t, [_i64, _i64, _i64, _i32]),
    "novaq_linear_backward": (_i32, [_f32p, _f32p, _i64, _i64, _vp, _i32, _f32p, _i64, _f32p,
                                     _f32p, _f32p, _vp, ctypes.c_size_t, _vp]),
    "novaq_conv2d_backward_workspace": (ctypes.c_size_t, [_i64, _i64, _i64, _i32, _i32, _i32]),
    "novaq_conv2d_backward": (_i32, [_f32p, _f32p, _i64, _i64, _i64, _i64, _vp, _i32, _f32p,
                                     _i64, _i32, _i32, _i32, _i32, _i32, _i32, _i32, _f32p,
                                     _f32p, _f32p, _vp, ctypes.c_size_t, _vp]),
    "novaq_conv2d_backward_noalloc": (_i32, [_f32p, _f32p, _i64, _i64, _i64, _i64, _vp, _i32,
                                             _f32p, _i64, _i32, _i32, _i32, _i32, _i32, _i32,
                                             _i32, _f32p, _f32p, _f32p, _vp]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libnovaq.so (once) and declare every exported signature."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build it with `python -m novann_amd._build` "
                "(hipcc, gfx950).  There is no CPU fallback.")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


class NovaqError(RuntimeError):
    def __init__(self, status: int, where: str):
        lib = load()
        msg = lib.novaq_status_string(status).decode()
        if status == EHIP:
            msg += f" (hipError {lib.novaq_last_hip_error()})"
        super().__init__(f"{where}: {msg}")
        self.status = status


def check(status: int, where: str) -> None:
    """Map a status code to the exception NovaNN raises for the same case."""
    if status == OK:
        return
    if status in (EINVAL, ESHAPE, EPADMODE, EALIGN):
        err = NovaqError(status, where)
        raise ValueError(str(err))
    if status == EDTYPE:
        raise TypeError(str(NovaqError(status, where)))
    if status == ENOTSUP:
        raise NotImplementedError(str(NovaqError(status, where)))
    raise NovaqError(status, where)
