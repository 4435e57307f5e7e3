"""C ABI checks that need no GPU: libnovaq.so loads, exports every symbol
include/novaq.h declares, and rejects bad arguments before touching HIP."""
import ctypes
import os
import re

import pytest

from novann_amd import _lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "novaq.h")


def declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(novaq_\w+)\s*\(", text))


def test_header_declares_the_entry_points():
    syms = declared_symbols()
    for s in ("novaq_cast", "novaq_amax", "novaq_quantize", "novaq_pack_fp4",
              "novaq_unpack_fp4", "novaq_linear_forward", "novaq_conv2d_forward"):
        assert s in syms


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    missing = [s for s in declared_symbols() if not hasattr(lib, s)]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == declared_symbols()


def test_version_and_status_strings():
    lib = _lib.load()
    assert lib.novaq_version() == 100
    assert lib.novaq_status_string(0) == b"ok"
    assert lib.novaq_status_string(-4) == b"unknown padding mode"
    assert lib.novaq_status_string(123) == b"unknown status"


FAKE = 0x10000  # never dereferenced: every call below fails validation first


@pytest.mark.parametrize("args,status", [
    ((FAKE, 9, FAKE, 0, 16, None, None), _lib.EDTYPE),          # bad src dtype
    ((FAKE, 0, FAKE, -1, 16, None, None), _lib.EDTYPE),         # bad dst dtype
    ((FAKE, 3, FAKE, 4, 16, None, None), _lib.EDTYPE),          # quantized -> quantized
    ((FAKE, 0, FAKE, 3, -1, None, None), _lib.EINVAL),          # negative n
    ((FAKE, 0, FAKE, 1, 16, FAKE, None), _lib.EINVAL),          # scale on f32->f16
    ((None, 0, FAKE, 3, 16, None, None), _lib.EINVAL),          # null src
    ((FAKE + 4, 0, FAKE, 3, 16, None, None), _lib.EALIGN),      # misaligned src
    ((FAKE, 0, FAKE + 8, 3, 16, None, None), _lib.EALIGN),      # misaligned dst
    ((None, 0, None, 3, 0, None, None), _lib.OK),               # n == 0 is a no-op
])
def test_cast_validation(args, status):
    assert _lib.load().novaq_cast(*args) == status


def test_other_entry_points_validation():
    lib = _lib.load()
    assert lib.novaq_amax(FAKE, 3, 16, FAKE, None) == _lib.EDTYPE
    assert lib.novaq_amax(FAKE + 2, 0, 16, FAKE, None) == _lib.EALIGN
    assert lib.novaq_scale_from_amax(FAKE, 1, FAKE, None) == _lib.EDTYPE
    assert lib.novaq_quantize(FAKE, 0, FAKE, 1, 16, FAKE, None) == _lib.EDTYPE
    assert lib.novaq_quantize(FAKE, 3, FAKE, 4, 16, FAKE, None) == _lib.EDTYPE
    assert lib.novaq_quantize(FAKE, 0, FAKE, 3, 16, None, None) == _lib.EINVAL
    # linear: bad dtype, negative size, misaligned (odd E2M1 rows are valid:
    # each row is padded to whole bytes)
    assert lib.novaq_linear_forward(FAKE, 4, 8, FAKE, 7, None, None, 4, FAKE, None) == _lib.EDTYPE
    assert lib.novaq_linear_forward(FAKE, -1, 8, FAKE, 3, None, None, 4, FAKE, None) == _lib.EINVAL
    assert lib.novaq_linear_forward(FAKE, 4, 7, FAKE, 5, None, None, 4, FAKE + 8, None) == _lib.EALIGN
    assert lib.novaq_linear_forward(FAKE, 4, 8, FAKE + 1, 3, None, None, 4, FAKE, None) == _lib.EALIGN
    assert lib.novaq_linear_forward(None, 0, 8, None, 3, None, None, 4, None, None) == _lib.OK
    # conv2d: pad mode, geometry, kernel larger than padded input
    conv = lib.novaq_conv2d_forward
    assert conv(FAKE, 1, 1, 8, 8, FAKE, 3, None, 2, 3, 3, 1, 1, 1, 1, 9, None, FAKE, None) == _lib.EPADMODE
    assert conv(FAKE, 1, 1, 8, 8, FAKE, 3, None, 2, 3, 3, 0, 1, 1, 1, 0, None, FAKE, None) == _lib.EINVAL
    assert conv(FAKE, 1, 1, 2, 2, FAKE, 3, None, 2, 5, 5, 1, 1, 0, 0, 0, None, FAKE, None) == _lib.ESHAPE
    assert conv(FAKE, 1, 1, 8, 8, FAKE, 9, None, 2, 3, 3, 1, 1, 1, 1, 0, None, FAKE, None) == _lib.EDTYPE
    # pool backward passes: dtype, pad mode, window larger than the padded
    # input, alignment, an empty batch
    mpb = lib.novaq_max_pool2d_backward
    assert mpb(FAKE, FAKE, 5, 1, 1, 4, 4, 2, 2, 2, 2, 0, 0, 0, FAKE, None) == _lib.EDTYPE
    assert mpb(FAKE, FAKE, 0, 1, 1, 4, 4, 2, 2, 2, 2, 0, 0, 7, FAKE, None) == _lib.EPADMODE
    assert mpb(FAKE, FAKE, 0, 1, 1, 1, 1, 2, 2, 2, 2, 0, 0, 0, FAKE, None) == _lib.ESHAPE
    assert mpb(FAKE + 2, FAKE, 0, 1, 1, 4, 4, 2, 2, 2, 2, 0, 0, 0, FAKE, None) == _lib.EALIGN
    assert mpb(FAKE, FAKE + 1, 2, 1, 1, 4, 4, 2, 2, 2, 2, 0, 0, 0, FAKE, None) == _lib.EALIGN
    assert mpb(None, None, 0, 0, 1, 4, 4, 2, 2, 2, 2, 0, 0, 0, None, None) == _lib.OK
    gpb = lib.novaq_global_avg_pool2d_backward
    assert gpb(FAKE, 1, 1, 0, 4, FAKE, None) == _lib.EINVAL
    assert gpb(FAKE, 1, 1, 4, 4, FAKE + 1, None) == _lib.EALIGN
    assert gpb(None, 0, 1, 4, 4, None, None) == _lib.OK


def test_backward_entry_points_validation():
    lib = _lib.load()
    # transpose: quantized -> other format, fp8 -> fp32, odd E2M1 sides, alignment, empty
    assert lib.novaq_transpose(FAKE, 3, 4, 4, FAKE, 0, None) == _lib.EDTYPE
    assert lib.novaq_transpose(FAKE, 2, 4, 4, FAKE, 0, None) == _lib.EDTYPE
    assert lib.novaq_transpose(FAKE, 5, 3, 4, FAKE, 5, None) == _lib.ESHAPE
    assert lib.novaq_transpose(FAKE + 4, 0, 4, 4, FAKE, 2, None) == _lib.EALIGN
    assert lib.novaq_transpose(None, 0, 0, 4, None, 0, None) == _lib.OK
    assert lib.novaq_colsum(FAKE, 4, -1, FAKE, None) == _lib.EINVAL
    assert lib.novaq_colsum(FAKE, 4, 0, None, None) == _lib.OK
    # workspace: W^T (64 x 32 E4M3), grad^T (32 x 8 bf16) and x^T (64 x 8 bf16),
    # each 256-byte aligned
    ws = lib.novaq_linear_backward_workspace(8, 64, 32, 3)
    assert ws == 2048 + 512 + 1024
    assert lib.novaq_linear_backward_workspace(8, 64, 32, 9) == 0
    bwd = lib.novaq_linear_backward
    assert bwd(FAKE, FAKE, 8, 64, FAKE, 9, None, 32, FAKE, FAKE, None, FAKE, ws, None) == _lib.EDTYPE
    assert bwd(FAKE, FAKE, 8, 63, FAKE, 5, None, 32, FAKE, FAKE, None, FAKE, ws, None) == _lib.ESHAPE
    # too small a workspace, or none
    assert bwd(FAKE, FAKE, 8, 64, FAKE, 3, None, 32, FAKE, FAKE, None, FAKE, ws - 1, None) == _lib.EINVAL
    assert bwd(FAKE, FAKE, 8, 64, FAKE, 3, None, 32, FAKE, None, None, None, 0, None) == _lib.EINVAL
    assert bwd(FAKE, FAKE, 8, 64, FAKE + 8, 3, None, 32, FAKE, None, None, FAKE, ws, None) == _lib.EALIGN
    # nothing requested: no work, no workspace needed
    assert bwd(FAKE, FAKE, 8, 64, FAKE, 3, None, 32, None, None, None, None, 0, None) == _lib.OK


def test_conv2d_backward_validation():
    lib = _lib.load()
    nb = lib.novaq_conv2d_backward_workspace(2, 3, 4, 3, 3, 5)
    assert nb > 0 and lib.novaq_conv2d_backward_workspace(2, 3, 4, 3, 3, 9) == 0
    bwd = lib.novaq_conv2d_backward
    args = [FAKE, FAKE, 2, 3, 8, 8, FAKE, 5, None, 4, 3, 3, 1, 1, 1, 1, 0, FAKE, FAKE, FAKE,
            FAKE, nb, None]

    def call(**kw):
        a = list(args)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return bwd(*a)
    assert call(a7=9) == _lib.EDTYPE                       # weight dtype
    assert call(a16=7) == _lib.EPADMODE                    # padding mode
    assert call(a12=0) == _lib.EINVAL                      # stride
    assert call(a10=11) == _lib.ESHAPE                     # kernel past the padded input
    assert call(a21=nb - 1) == _lib.EINVAL                 # workspace too small
    assert call(a17=FAKE + 4) == _lib.EALIGN               # misaligned output
    assert call(a17=None, a18=None, a19=None, a20=None, a21=0) == _lib.OK  # nothing asked


def test_status_maps_to_reference_exceptions():
    with pytest.raises(ValueError):
        _lib.check(_lib.EPADMODE, "conv2d")
    with pytest.raises(TypeError):
        _lib.check(_lib.EDTYPE, "cast")
    with pytest.raises(NotImplementedError):
        _lib.check(_lib.ENOTSUP, "x")
    _lib.check(_lib.OK, "x")


def test_fused_forward_validation():
    """novaq_*_forward_ex reject bad x / output dtypes, padding modes, shapes
    and misaligned epilogue pointers before any launch."""
    lib = _lib.load()
    ep = _lib.Epilogue(None, None, None, None, 1, _lib.BF16)
    bad_out = _lib.Epilogue(None, None, None, None, 0, _lib.E2M1)
    odd = _lib.Epilogue(FAKE + 2, None, None, None, 0, _lib.F32)
    lin = lib.novaq_linear_forward_ex
    largs = [FAKE, _lib.F32, None, 4, 8, FAKE, _lib.E4M3, None, None, 8, None, FAKE, None]

    def lcall(**kw):
        a = list(largs)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return lin(*a)
    assert lcall(a1=_lib.E2M1) == _lib.EDTYPE              # x cannot be FP4
    assert lcall(a1=9) == _lib.EDTYPE
    assert lcall(a6=9) == _lib.EDTYPE                      # weight dtype
    assert lcall(a10=ctypes.byref(bad_out)) == _lib.EDTYPE  # FP4 output
    assert lcall(a3=-1) == _lib.EINVAL
    assert lcall(a6=_lib.E2M1, a4=7, a11=FAKE + 8) == _lib.EALIGN  # odd E2M1 rows pass the shape checks
    assert lcall(a0=FAKE + 4) == _lib.EALIGN
    assert lcall(a10=ctypes.byref(odd)) == _lib.EALIGN      # epilogue pointer
    assert lcall(a3=0, a10=ctypes.byref(ep)) == _lib.OK     # empty batch
    conv = lib.novaq_conv2d_forward_ex
    cargs = [FAKE, _lib.BF16, None, 2, 3, 8, 8, FAKE, _lib.E2M1, None, 4, 3, 3, 1, 1, 1, 1, 0,
             None, None, FAKE, None]

    def ccall(**kw):
        a = list(cargs)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return conv(*a)
    assert ccall(a17=4) == _lib.EPADMODE
    assert ccall(a1=_lib.E2M1) == _lib.EDTYPE
    assert ccall(a11=12) == _lib.ESHAPE
    assert ccall(a13=0) == _lib.EINVAL
    assert ccall(a19=ctypes.byref(bad_out)) == _lib.EDTYPE
    assert ccall(a3=0) == _lib.OK


def test_optimizer_and_pool_validation():
    lib = _lib.load()
    hp = _lib.AdamW(1e-3, 0.9, 0.999, 1e-8, 0.0, 1, 1)
    bad = _lib.AdamW(1e-3, 0.9, 0.999, 1e-8, 0.0, 0, 1)   # steps count from 1
    step = lib.novaq_adamw_step
    assert step(FAKE, FAKE, FAKE, FAKE, 8, ctypes.byref(bad), None, None) == _lib.EINVAL
    assert step(FAKE, FAKE, FAKE, FAKE, 8, None, None, None) == _lib.EINVAL
    assert step(FAKE + 4, FAKE, FAKE, FAKE, 8, ctypes.byref(hp), None, None) == _lib.EALIGN
    assert step(None, FAKE, FAKE, FAKE, 8, ctypes.byref(hp), None, None) == _lib.EINVAL
    rq = lib.novaq_adamw_requantize
    assert rq(FAKE, FAKE, FAKE, FAKE, 8, ctypes.byref(hp), FAKE, _lib.F16, FAKE,
              None) == _lib.EDTYPE                         # codes must be FP8 / FP4
    assert rq(FAKE, FAKE, FAKE, FAKE, 8, ctypes.byref(hp), FAKE, _lib.E4M3, None,
              None) == _lib.EINVAL                         # amax_scale is required
    mp = lib.novaq_max_pool2d
    margs = [FAKE, _lib.F32, 2, 3, 8, 8, 2, 2, 2, 2, 0, 0, 0, FAKE, None]

    def mcall(**kw):
        a = list(margs)
        for i, v in kw.items():
            a[int(i[1:])] = v
        return mp(*a)
    assert mcall(a1=_lib.E2M1) == _lib.EDTYPE
    assert mcall(a12=5) == _lib.EPADMODE
    assert mcall(a6=11) == _lib.ESHAPE
    assert mcall(a8=0) == _lib.EINVAL
    assert mcall(a2=0) == _lib.OK
    # views need element alignment only; a pointer inside an element is refused
    assert mcall(a0=FAKE + 2) == _lib.EALIGN
    assert mcall(a13=FAKE + 1, a1=_lib.BF16) == _lib.EALIGN
    gap = lib.novaq_global_avg_pool2d
    assert gap(FAKE, _lib.E2M1, None, 2, 3, 4, 4, FAKE, None) == _lib.EDTYPE
    assert gap(FAKE, _lib.F32, None, 2, 0, 4, 4, FAKE, None) == _lib.EINVAL
    assert gap(FAKE, _lib.F32, None, 0, 3, 4, 4, FAKE, None) == _lib.OK
    # a scale goes with FP8 codes only
    assert gap(FAKE, _lib.BF16, FAKE, 2, 3, 4, 4, FAKE, None) == _lib.EDTYPE
    assert gap(FAKE, _lib.F32, FAKE, 2, 3, 4, 4, FAKE, None) == _lib.EDTYPE
    # the plane loads are 4-element vectors: x must be 16-byte aligned
    assert gap(FAKE + 4, _lib.F32, None, 2, 3, 4, 4, FAKE, None) == _lib.EALIGN
    assert gap(FAKE, _lib.F32, None, 2, 3, 4, 4, FAKE + 2, None) == _lib.EALIGN
    # extras: element-aligned x, 16-byte aligned outputs; bad dtype / mode / scale
    im = lib.novaq_im2col
    assert im(FAKE, _lib.E2M1, None, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 0, FAKE, None) == _lib.EDTYPE
    assert im(FAKE, _lib.F32, FAKE, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 0, FAKE, None) == _lib.EDTYPE
    assert im(FAKE, _lib.F32, None, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 7, FAKE, None) == _lib.EPADMODE
    assert im(FAKE, _lib.F32, None, 1, 1, 2, 2, 5, 5, 1, 1, 0, 0, 0, FAKE, None) == _lib.ESHAPE
    assert im(FAKE + 2, _lib.F32, None, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 0, FAKE, None) == _lib.EALIGN
    assert im(FAKE, _lib.F32, None, 1, 1, 4, 4, 3, 3, 1, 1, 1, 1, 0, FAKE + 4, None) == _lib.EALIGN
    assert im(None, _lib.F32, None, 0, 1, 4, 4, 3, 3, 1, 1, 1, 1, 0, None, None) == _lib.OK
    pad = lib.novaq_pad2d
    assert pad(FAKE, _lib.E2M1, 1, 1, 4, 4, 1, 1, 0, FAKE, None) == _lib.EDTYPE
    assert pad(FAKE, _lib.F32, 1, 1, 4, 4, 1, 1, 9, FAKE, None) == _lib.EPADMODE
    assert pad(FAKE, _lib.F32, 1, 1, 4, 4, -1, 1, 0, FAKE, None) == _lib.EINVAL
    assert pad(FAKE + 1, _lib.BF16, 1, 1, 4, 4, 1, 1, 0, FAKE, None) == _lib.EALIGN
    assert pad(FAKE, _lib.F32, 1, 1, 4, 4, 1, 1, 0, FAKE + 8, None) == _lib.EALIGN
