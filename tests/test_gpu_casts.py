"""GPU casts vs the C oracle, bit for bit, through the C ABI (libnovaq.so)."""
import numpy as np
import pytest
import torch

import oracle as O
from novann_amd import quant
from tests.gpu_util import NAME, first_mismatch, to_dev, to_host
from tests.patterns import (MBITS, config1_tensor, config2_tensor, config3_tensor,
                            random_f32_bits, structured_f32)

pytestmark = pytest.mark.gpu

NARROW = [O.F16, O.BF16, O.E4M3, O.E5M2, O.E2M1]
FLOATS = [O.F32, O.F16, O.BF16]
QUANT = [O.E4M3, O.E5M2, O.E2M1]


def gpu_cast(arr, st, dt, n=None, scale=None):
    src = to_dev(arr, st)
    sc = None if scale is None else torch.tensor([scale], dtype=torch.float32, device="cuda")
    out = quant.cast(src, NAME[dt], src_dtype=NAME[st], n=n, scale=sc)
    torch.cuda.synchronize()
    return to_host(out)


@pytest.mark.parametrize("dt", NARROW, ids=lambda d: NAME[d])
def test_encode_structured_random(dt):
    bits = np.concatenate([structured_f32(MBITS[dt]), random_f32_bits(1 << 22, seed=100 + dt)])
    got = gpu_cast(bits, O.F32, dt)
    want = O.cast(bits, O.F32, dt)
    assert (m := first_mismatch(got, want)) is None, m


@pytest.mark.parametrize("dt", NARROW, ids=lambda d: NAME[d])
def test_encode_golden_fixture(golden, dt):
    g = golden["casts"]
    got = gpu_cast(g["inputs"], O.F32, dt)
    want = g[NAME[dt]]
    if dt == O.E2M1:
        got = np.stack([got & 0xF, got >> 4], axis=-1).reshape(-1)[: g["inputs"].size]
    assert (m := first_mismatch(got, want, g["inputs"])) is None, m


@pytest.mark.parametrize("st", NARROW, ids=lambda d: NAME[d])
@pytest.mark.parametrize("dt", FLOATS, ids=lambda d: NAME[d])
def test_decode_every_code(st, dt):
    if st == dt:
        pytest.skip("identity")
    if st in (O.F16, O.BF16):
        codes = np.arange(1 << 16, dtype=np.uint32).astype(np.uint16)
    else:
        codes = np.arange(256, dtype=np.uint32).astype(np.uint8)  # E2M1: all nibble pairs
    n = codes.size * 2 if st == O.E2M1 else codes.size
    got = gpu_cast(codes, st, dt, n=n)
    want = O.cast(codes, st, dt, n=n)
    assert (m := first_mismatch(got, want.view(got.dtype))) is None, m


@pytest.mark.parametrize("dt", NARROW, ids=lambda d: NAME[d])
def test_encode_exhaustive_2p32(dt):
    """All 2^32 fp32 bit patterns, in 2^28 chunks, GPU vs oracle."""
    chunk = 1 << 28
    for lo in range(0, 1 << 32, chunk):
        x = torch.arange(lo, lo + chunk, dtype=torch.int64, device="cuda").to(torch.int32)
        out = quant.cast(x.view(torch.float32), NAME[dt])
        torch.cuda.synchronize()
        got = to_host(out)
        del x, out
        want = O.encode_range(dt, lo, chunk)
        if dt == O.E2M1:
            want = (want[0::2] | (want[1::2] << 4)).astype(np.uint8)
        bad = np.nonzero(got != want)[0]
        assert bad.size == 0, (f"chunk 0x{lo:08x}: {bad.size} mismatches, first pattern "
                               f"0x{lo + int(bad[0]) * (2 if dt == O.E2M1 else 1):08x}")


@pytest.mark.parametrize("st", FLOATS, ids=lambda d: NAME[d])
@pytest.mark.parametrize("dt", NARROW + [O.F32], ids=lambda d: NAME[d])
@pytest.mark.parametrize("n", [1, 7, 33, 4097, 1000003])
def test_every_pair_ragged_sizes(st, dt, n):
    rng = np.random.default_rng(n + 17 * st + dt)
    f = (rng.standard_normal(n) * np.exp2(rng.uniform(-12, 12, n))).astype(np.float32)
    src = O.cast(f, O.F32, st) if st != O.F32 else f.view(np.uint32)
    got = gpu_cast(src, st, dt, n=n)
    want = O.cast(src, st, dt, n=n)
    assert (m := first_mismatch(got, want.view(got.dtype))) is None, m


@pytest.mark.parametrize("dt", QUANT, ids=lambda d: NAME[d])
@pytest.mark.parametrize("scale", [0.0123, 3.5, 1e-30, 7e30, -0.75, 0.0])
def test_scaled_quantize_and_dequantize(dt, scale):
    bits = np.concatenate([structured_f32(MBITS[dt]), random_f32_bits(1 << 20, seed=3)])
    got = gpu_cast(bits, O.F32, dt, scale=scale)
    want = O.cast(bits, O.F32, dt, scale=scale)
    assert (m := first_mismatch(got, want)) is None, m
    codes = np.arange(256, dtype=np.uint32).astype(np.uint8)
    n = 512 if dt == O.E2M1 else 256
    for ft in FLOATS:
        got = gpu_cast(codes, dt, ft, n=n, scale=scale)
        want = O.cast(codes, dt, ft, n=n, scale=scale)
        assert (m := first_mismatch(got, want.view(got.dtype))) is None, (NAME[ft], m)


def test_config1_e4m3_roundtrip_bit_exact():
    """BASELINE config [1]: 4096x4096 fp32 with 10% specials -> E4M3 -> fp32."""
    x = config1_tensor()
    bits = x.view(np.uint32).reshape(-1)
    q = quant.cast(to_dev(bits, O.F32), "e4m3")
    y = quant.cast(q, "f32")
    torch.cuda.synchronize()
    want_q = O.cast(bits, O.F32, O.E4M3)
    want_y = O.cast(want_q, O.E4M3, O.F32).view(np.uint32)
    assert (m := first_mismatch(to_host(q), want_q)) is None, m
    assert (m := first_mismatch(to_host(y), want_y)) is None, m


def test_config2_sweep_full_size_bit_exact():
    """BASELINE config [2] at full size: 2^28 fp32 -> {f16, bf16} -> fp32 and
    per-tensor amax-scaled {E4M3, E5M2} -> fp32, all bit-compared."""
    n = 1 << 28
    x = config2_tensor(n)
    xd = to_dev(x.view(np.uint32), O.F32)
    for dt in ("f16", "bf16"):
        code = {"f16": O.F16, "bf16": O.BF16}[dt]
        h = quant.cast(xd, dt)
        back = quant.cast(h, "f32")
        torch.cuda.synchronize()
        want_h = O.cast(x, O.F32, code)
        assert (m := first_mismatch(to_host(h), want_h)) is None, (dt, m)
        want_b = O.cast(want_h, code, O.F32).view(np.uint32)
        assert (m := first_mismatch(to_host(back), want_b)) is None, (dt, m)
        del h, back
    amax = O.amax(x)
    for dt in ("e4m3", "e5m2"):
        code = {"e4m3": O.E4M3, "e5m2": O.E5M2}[dt]
        q = quant.quantize(xd, dt)
        back = quant.dequantize(q)
        torch.cuda.synchronize()
        s = O.scale_from_amax(amax, code)
        assert q.amax.item() == amax and q.scale.item() == s
        want_q = O.cast(x, O.F32, code, scale=s)
        assert (m := first_mismatch(to_host(q.data), want_q)) is None, (dt, m)
        want_b = O.cast(want_q, code, O.F32, scale=s).view(np.uint32)
        assert (m := first_mismatch(to_host(back).reshape(-1), want_b)) is None, (dt, m)
        del q, back


@pytest.mark.parametrize("n", [1 << 26, (1 << 26) - 3])
def test_config3_fp4_pack_unpack_bit_exact(n):
    """BASELINE config [3]: 2^26 elements (and an odd size), pack with the
    per-tensor amax/6 scale, unpack; the packed bytes are bit-compared."""
    x = config3_tensor(n)
    xd = to_dev(x.view(np.uint32), O.F32)
    q = quant.quantize(xd, "e2m1")
    y = quant.unpack_fp4(q.data, n, scale=q.scale)
    torch.cuda.synchronize()
    s = O.scale_from_amax(O.amax(x), O.E2M1)
    want = O.cast(x, O.F32, O.E2M1, scale=s)
    assert (m := first_mismatch(to_host(q.data), want)) is None, m
    want_y = O.cast(want, O.E2M1, O.F32, n=n, scale=s).view(np.uint32)
    assert (m := first_mismatch(to_host(y), want_y)) is None, m
    # unscaled pack too
    p = quant.pack_fp4(xd)
    torch.cuda.synchronize()
    assert (m := first_mismatch(to_host(p), O.cast(x, O.F32, O.E2M1))) is None, m


@pytest.mark.parametrize("st", FLOATS, ids=lambda d: NAME[d])
@pytest.mark.parametrize("n", [0, 1, 5, 1000, 1 << 24, (1 << 24) + 13])
def test_amax(st, n):
    rng = np.random.default_rng(n + st)
    f = (rng.standard_normal(n) * 100).astype(np.float32)
    if n > 10:
        f[rng.integers(0, n, 5)] = np.nan
    src = O.cast(f, O.F32, st) if st != O.F32 else f.view(np.uint32)
    a = quant.amax(to_dev(src, st))
    torch.cuda.synchronize()
    assert a.item() == O.amax(src, st)


def test_amax_with_inf_gives_unit_scale():
    f = np.array([1.0, -np.inf, 3.0, np.nan] * 100, dtype=np.float32)
    q = quant.quantize(to_dev(f.view(np.uint32), O.F32), "e4m3")
    torch.cuda.synchronize()
    assert q.amax.item() == np.inf and q.scale.item() == 1.0


def test_quantize_empty_tensor():
    x = torch.empty(0, dtype=torch.float32, device="cuda")
    q = quant.quantize(x, "e5m2")
    torch.cuda.synchronize()
    assert q.amax.item() == 0.0 and q.scale.item() == 1.0


def test_host_layer_refuses_short_buffers():
    """quant.cast / dequantize / the products check element counts against
    the buffers before launching (ValueError, as numpy raises for a size
    mismatch)."""
    from novann_amd import functional as F
    from novann_amd import quant
    from novann_amd.module import Parameters
    x = torch.ones(100, device="cuda")
    with pytest.raises(ValueError):
        quant.cast(x, "e4m3", n=101)
    with pytest.raises(ValueError):
        quant.cast(x, "f16", out=torch.empty(99, dtype=torch.float16, device="cuda"))
    with pytest.raises(TypeError):
        quant.cast(x, "f16", out=torch.empty(100, dtype=torch.bfloat16, device="cuda"))
    q = quant.quantize(x, "e4m3")
    bad = quant.Quantized(q.data[:50], (100,), "e4m3", q.scale)
    with pytest.raises(ValueError):
        quant.dequantize(bad)
    xq = quant.quantize(torch.ones((4, 8), device="cuda"), "e4m3")
    short = quant.Quantized(xq.data[:16], (4, 8), "e4m3", xq.scale)
    with pytest.raises(ValueError):
        F.linear(short, Parameters(np.ones((2, 8), np.float32)), None)
    assert quant.cast(x, "f16", n=100).numel() == 100


@pytest.mark.parametrize("st", [O.F16, O.BF16], ids=lambda d: NAME[d])
@pytest.mark.parametrize("dt", QUANT, ids=lambda d: NAME[d])
@pytest.mark.parametrize("n", [1, 4097, (1 << 20) + 5])
def test_scaled_quantize_from_16bit_sources(st, dt, n):
    """novaq_quantize from fp16 / bf16 sources (amax of the 16-bit values,
    s = amax / fmt_max, enc(x * (1/s))) and novaq_cast with explicit scales,
    bit-exact against the oracle; the input carries NaNs (ignored by the
    amax), signed zeros and exact E2M1 / FP8 ties after scaling."""
    print(f"scaled quantize {NAME[st]} -> {NAME[dt]} n={n}", flush=True)
    rng = np.random.default_rng(n + 31 * st + dt)
    f = (rng.standard_normal(n) * np.exp2(rng.uniform(-10, 10, n))).astype(np.float32)
    if n > 10:
        f[rng.integers(0, n, 7)] = np.nan
        f[rng.integers(0, n, 7)] = -0.0
        f[rng.integers(0, n, 7)] = np.float32(2.5) * np.float32(np.abs(f[0]) + 1)
    src = O.cast(f, O.F32, st)
    q = quant.quantize(to_dev(src, st), NAME[dt])
    torch.cuda.synchronize()
    a = O.amax(src, st)
    s = O.scale_from_amax(a, dt)
    assert q.amax.item() == a and q.scale.item() == s
    want = O.cast(src, st, dt, n=n, scale=s)
    assert (m := first_mismatch(to_host(q.data), want)) is None, m
    for scale in (0.0123, -0.75, 7e30, 0.0):
        got = gpu_cast(src, st, dt, n=n, scale=scale)
        want = O.cast(src, st, dt, n=n, scale=scale)
        assert (m := first_mismatch(got, want)) is None, (scale, m)
