"""Pins the C oracle's cast rules (CPU only).

Every check compares the oracle with something it does not share code with:
its own brute-force nearest-code search, numpy's float16, torch's bfloat16 /
float8 casts, the spec tables, or the committed golden fixtures.
"""
import numpy as np
import pytest
import torch

import oracle as O
from tests.patterns import MBITS, random_f32_bits, structured_f32

NARROW = [O.F16, O.BF16, O.E4M3, O.E5M2, O.E2M1]
NAMES = {O.F16: "f16", O.BF16: "bf16", O.E4M3: "e4m3", O.E5M2: "e5m2", O.E2M1: "e2m1"}


@pytest.mark.parametrize("dt", NARROW, ids=lambda d: NAMES[d])
def test_fast_encoder_matches_brute_force_structured(dt):
    bits = np.concatenate([structured_f32(MBITS[dt]), random_f32_bits(1 << 20, seed=dt)])
    fast = O.encode_array(bits, dt)
    slow = O.bf_encode_array(bits, dt)
    bad = np.nonzero(fast != slow)[0]
    assert bad.size == 0, (f"{bad.size} mismatches, first x=0x{bits[bad[0]]:08x} "
                           f"fast=0x{fast[bad[0]]:x} brute=0x{slow[bad[0]]:x}")


@pytest.mark.slow
@pytest.mark.parametrize("dt", NARROW, ids=lambda d: NAMES[d])
def test_fast_encoder_matches_brute_force_exhaustive(dt):
    bad, first = O.sweep_encode(dt, 0, 1 << 32)
    assert bad == 0, f"{bad} mismatches, first 0x{first:08x}"


@pytest.mark.parametrize("dt", NARROW, ids=lambda d: NAMES[d])
def test_golden_fixture_encode(golden, dt):
    g = golden["casts"]
    bits = g["inputs"]
    got = O.encode_array(bits, dt)
    want = g[NAMES[dt]].astype(np.uint32)
    bad = np.nonzero(got != want)[0]
    assert bad.size == 0, (f"{bad.size} mismatches vs fixture, first x=0x{bits[bad[0]]:08x} "
                           f"got=0x{got[bad[0]]:x} want=0x{want[bad[0]]:x}")


def test_f16_matches_numpy_astype():
    """numpy is NovaNN's numeric backend: x.astype(np.float16) bit for bit,
    NaN payloads included, over structured + random patterns."""
    bits = np.concatenate([structured_f32(10), random_f32_bits(1 << 22, seed=11)])
    with np.errstate(all="ignore"):
        want = bits.view(np.float32).astype(np.float16).view(np.uint16)
    got = O.cast(bits, O.F32, O.F16)
    assert np.array_equal(got, want)


def test_f16_widening_matches_numpy_all_codes():
    h = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    want = h.view(np.float16).astype(np.float32).view(np.uint32)
    got = O.cast(h, O.F16, O.F32).view(np.uint32)
    assert np.array_equal(got, want)


def test_bf16_matches_torch_on_non_nan():
    bits = np.concatenate([structured_f32(7), random_f32_bits(1 << 22, seed=12)])
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    want = torch.from_numpy(bits.view(np.float32).copy()).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16)
    got = O.cast(bits, O.F32, O.BF16)
    assert np.array_equal(got[~nan], want[~nan])
    # NaN rule: quiet bit set, sign and top payload kept
    assert np.array_equal(got[nan], ((bits[nan] >> 16) | 0x40).astype(np.uint16))


@pytest.mark.parametrize("dt,tdt,lim", [(O.E4M3, torch.float8_e4m3fn, 464.0),
                                        (O.E5M2, torch.float8_e5m2, 61440.0)],
                         ids=["e4m3", "e5m2"])
def test_fp8_matches_torch_inside_its_saturating_range(dt, tdt, lim):
    """torch's float8 casts do not saturate (NaN / Inf beyond the max); inside
    |x| < lim they must agree bit for bit, NaN sign rule included."""
    bits = np.concatenate([structured_f32(MBITS[dt]), random_f32_bits(1 << 22, seed=dt)])
    x = bits.view(np.float32)
    with np.errstate(all="ignore"):
        keep = np.isnan(x) | (np.abs(x.astype(np.float64)) < lim)
    want = torch.from_numpy(x.copy()).to(tdt).view(torch.uint8).numpy()
    got = O.cast(bits, O.F32, dt)
    assert np.array_equal(got[keep], want[keep])
    # saturation outside: +-max code
    maxc = 0x7E if dt == O.E4M3 else 0x7B
    out = ~keep
    assert np.array_equal(got[out], ((bits[out] >> 24) & 0x80).astype(np.uint8) | maxc)


@pytest.mark.parametrize("dt", [O.E4M3, O.E5M2], ids=["e4m3", "e5m2"])
def test_fp8_decode_tables(golden, dt):
    codes = np.arange(256, dtype=np.uint8)
    got = O.cast(codes, dt, O.F32).view(np.uint32)
    ref = golden["casts"]["dec_" + NAMES[dt]]
    fnan = np.isnan(ref.view(np.float32))
    assert np.array_equal(got[~fnan], ref[~fnan])
    assert np.array_equal(got[fnan], (codes[fnan].astype(np.uint32) & 0x80) << 24 | 0x7FC00000)
    # third, formula-based decoder
    bf = np.array([O.bf_decode(int(c), dt) for c in codes], dtype=np.uint32)
    assert np.array_equal(got, bf)


def test_e2m1_spec_table_and_ties():
    values = [0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0]
    for code in range(16):
        v = np.uint32(O.decode(code, O.E2M1)).view(np.float32)
        want = (-1.0 if code & 8 else 1.0) * values[code & 7]
        assert v == want and np.signbit(v) == bool(code & 8)
    # RNE ties of the spec: 0.25->0, 0.75->1, 1.25->1, 1.75->2, 2.5->2, 3.5->4, 5->4
    for x, want in [(0.25, 0.0), (0.75, 1.0), (1.25, 1.0), (1.75, 2.0), (2.5, 2.0),
                    (3.5, 4.0), (5.0, 4.0), (6.5, 6.0), (1e30, 6.0), (np.inf, 6.0)]:
        for s in (1.0, -1.0):
            b = int(np.float32(s * x).view(np.uint32))
            got = np.uint32(O.decode(O.encode(b, O.E2M1), O.E2M1)).view(np.float32)
            assert got == s * want and np.signbit(got) == (s < 0), (s * x, got)
    nan = int(np.uint32(0xFFC00000))
    assert O.encode(nan, O.E2M1) == 0  # NaN -> +0


def test_e2m1_pack_nibble_order_and_odd_tail():
    x = np.array([0.5, -6.0, 1.5], dtype=np.float32)  # codes 1, 0xF, 3
    packed = O.cast(x, O.F32, O.E2M1)
    assert packed.tolist() == [0x1 | (0xF << 4), 0x3]
    back = O.cast(packed, O.E2M1, O.F32, n=3)
    assert back.tolist() == [0.5, -6.0, 1.5]


def test_signed_zero_kept_everywhere():
    for dt in NARROW:
        tiny_neg = 0x80000001  # -(smallest fp32 denormal): rounds to -0 everywhere
        c = O.encode(tiny_neg, dt)
        v = np.uint32(O.decode(c, dt)).view(np.float32)
        assert v == 0.0 and np.signbit(v), NAMES[dt]


def test_scaled_quantize_closed_form():
    rng = np.random.default_rng(5)
    x = rng.standard_normal(1 << 16).astype(np.float32) * np.float32(37.0)
    for dt in (O.E4M3, O.E5M2, O.E2M1):
        s = np.float32(O.scale_from_amax(O.amax(x), dt))
        inv = np.float32(1.0) / s
        got = O.encode_array((x * inv).view(np.uint32), dt)
        # quantize with scale == encode(x * (1/s)) for finite x
        q = O.cast(x, O.F32, dt, scale=float(s))
        if dt == O.E2M1:
            q = np.stack([q & 0xF, q >> 4], axis=-1).reshape(-1)[: x.size]
        assert np.array_equal(q.astype(np.uint32), got)
        # dequantize == decode(q) * s
        deq = O.cast(O.cast(x, O.F32, dt, scale=float(s)), dt, O.F32, n=x.size,
                     scale=float(s))
        dec = O.cast(O.cast(x, O.F32, dt, scale=float(s)), dt, O.F32, n=x.size)
        assert np.array_equal(deq, dec * s)
        # the max element lands on (or saturates to) the format max
        fmax = {O.E4M3: 448.0, O.E5M2: 57344.0, O.E2M1: 6.0}[dt]
        assert np.abs(dec).max() == fmax


def test_scaled_nan_and_negative_scale_sign_rule():
    nan_pos, nan_neg = 0x7FC00000, 0xFFC00001
    assert O.lib().novaq_ref_quantize_scaled(nan_pos, -2.0, O.E4M3) == 0xFF
    assert O.lib().novaq_ref_quantize_scaled(nan_neg, 2.0, O.E4M3) == 0xFF
    assert O.lib().novaq_ref_quantize_scaled(nan_neg, -2.0, O.E5M2) == 0x7F
    # Inf * 0 -> NaN code
    inf = 0x7F800000
    assert O.lib().novaq_ref_quantize_scaled(inf, 0.0, O.E4M3) == 0x7F
    # dequantize NaN code with a negative scale: canonical NaN, flipped sign
    assert O.lib().novaq_ref_dequantize_scaled(0x7F, -1.0, O.E4M3) == 0xFFC00000


def test_amax_and_scale():
    x = np.array([1.0, -7.5, np.nan, 3.0, -0.0], dtype=np.float32)
    assert O.amax(x) == 7.5
    assert O.amax(np.array([], dtype=np.float32)) == 0.0
    assert O.amax(np.array([np.inf, 1.0], dtype=np.float32)) == np.inf
    assert O.scale_from_amax(7.5, O.E4M3) == np.float32(7.5) / np.float32(448.0)
    assert O.scale_from_amax(0.0, O.E4M3) == 1.0
    assert O.scale_from_amax(np.inf, O.E5M2) == 1.0
    h = np.array([1.0, -65504.0, np.nan], dtype=np.float16).view(np.uint16)
    assert O.amax(h, O.F16) == 65504.0
    rng = np.random.default_rng(9)
    big = rng.standard_normal(1 << 20).astype(np.float32)
    assert O.amax(big) == np.abs(big).max()


def test_cast_rejects_quantized_to_quantized():
    with pytest.raises(ValueError):
        O.cast(np.zeros(4, np.uint8), O.E4M3, O.E5M2)


def test_config1_tensor_holds_every_special():
    """BASELINE config [1]'s specials really occur: signed zeros, both
    infinities, quiet and signalling NaNs of both signs, values past +-448
    (464 and 480 exactly), E4M3-subnormal neighbours and fp32 subnormals."""
    from tests.patterns import config1_tensor
    x = config1_tensor().reshape(-1)
    b = x.view(np.uint32)
    mag, neg = b & 0x7FFFFFFF, (b >> 31) == 1
    nan = mag > 0x7F800000
    quiet = (b & 0x00400000) != 0
    for sel in (nan & quiet & neg, nan & quiet & ~neg, nan & ~quiet & neg, nan & ~quiet & ~neg):
        assert sel.sum() > 1000
    assert ((mag == 0x7F800000) & neg).any() and ((mag == 0x7F800000) & ~neg).any()
    assert ((mag == 0) & neg).any() and ((mag == 0) & ~neg).any()
    assert (np.abs(x) == 464).any() and (np.abs(x) == 480).any()
    assert ((np.abs(x) > 448) & np.isfinite(x) & neg).any()
    assert ((mag > 0) & (mag < 0x00800000)).sum() > 1000


@pytest.mark.parametrize("st", [O.F16, O.BF16])
@pytest.mark.parametrize("dt", [O.E4M3, O.E5M2, O.E2M1])
def test_scaled_cast_from_16bit_sources_is_the_widened_cast(st, dt):
    """Widening fp16 / bf16 to fp32 is exact, so a scaled cast from a 16-bit
    source must equal the (pinned) scaled fp32 cast of the widened values --
    for every 16-bit code, with a positive, a negative and a zero scale; the
    amax of a 16-bit tensor is the amax of its widening."""
    codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    wide = O.cast(codes, st, O.F32)
    for s in (0.0123, -3.5, 0.0):
        got = O.cast(codes, st, dt, scale=s)
        want = O.cast(wide, O.F32, dt, scale=s)
        assert np.array_equal(got, want)
    finite = codes[np.isfinite(wide)]
    assert O.amax(finite, st) == O.amax(O.cast(finite, st, O.F32))
