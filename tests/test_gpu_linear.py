"""Quantized Linear on the GPU vs the CPU oracle (y = x @ (s*dec(Wq))^T + b).

Tolerance: normwise max|y - r| / max|r| <= 1e-2 against
the fp64 product of the same fp32 inputs and the dequantized fp32 weights.
The identity-input case is bit-exact: it routes every weight code through the
in-kernel decode and the MFMA lane layout unchanged."""
import numpy as np
import pytest
import torch

import oracle as O
from novann_amd import _lib, quant
from novann_amd import functional as F
from novann_amd.module import Linear, Parameters, QuantizedParameters
from tests.gpu_util import NAME, bf16_round, error_report, to_dev, to_host

pytestmark = pytest.mark.gpu

TOL = 1e-2
QCODE = {"e4m3": O.E4M3, "e5m2": O.E5M2, "e2m1": O.E2M1}


def run_linear(x, codes, wdt, scale, bias, N, K):
    """Raw C-ABI call on device buffers; returns y (M, N) as numpy fp32."""
    M = x.shape[0]
    xd = torch.from_numpy(np.ascontiguousarray(x, np.float32)).cuda()
    wd = to_dev(codes, QCODE.get(wdt, {"bf16": O.BF16, "f16": O.F16, "f32": O.F32}.get(wdt)))
    sd = None if scale is None else torch.tensor([scale], dtype=torch.float32, device="cuda")
    bd = None if bias is None else torch.from_numpy(np.ascontiguousarray(bias, np.float32)).cuda()
    yd = torch.empty((M, N), dtype=torch.float32, device="cuda")
    code = _lib.DTYPES[wdt]
    rc = _lib.load().novaq_linear_forward(
        xd.data_ptr(), M, K, wd.data_ptr(), code, None if sd is None else sd.data_ptr(),
        None if bd is None else bd.data_ptr(), N, yd.data_ptr(),
        torch.cuda.current_stream().cuda_stream)
    _lib.check(rc, "linear")
    torch.cuda.synchronize()
    return yd.cpu().numpy()


def dequant(codes, wdt, n, scale):
    c = QCODE[wdt]
    return O.cast(codes, c, O.F32, n=n, scale=scale)


def normwise(y, r):
    return float(np.abs(y.astype(np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


def valid_codes(wdt):
    if wdt == "e4m3":
        return np.array([c for c in range(256) if (c & 0x7F) != 0x7F], dtype=np.uint8)
    if wdt == "e5m2":
        return np.array([c for c in range(256) if (c & 0x7F) < 0x7C], dtype=np.uint8)
    return np.arange(16, dtype=np.uint8)


@pytest.mark.parametrize("wdt", ["e4m3", "e5m2", "e2m1"])
@pytest.mark.parametrize("scale", [1.0, 0.0123])
@pytest.mark.parametrize("K,N", [(256, 320), (256, 512), (192, 512), (256, 384)],
                         ids=["edge-tiles", "wide-k", "staged-256", "staged-128"])
def test_identity_input_reproduces_dequantized_weights_exactly(wdt, scale, K, N):
    """x = I: y[i, j] = s * dec(W[j, i]) exactly, for every finite code.  The
    shapes reach each kernel: guarded edge tiles (N % 128 != 0), the K-block
    kernels for N % 256 == 0, K % 128 == 0 (ping-pong for FP8, wide for FP4)
    and the staged-decode kernel at both tile widths (K % 128 != 0;
    N % 256 != 0)."""
    rng = np.random.default_rng(1)
    vals = valid_codes(wdt)
    nib = vals[rng.integers(0, vals.size, size=N * K)]
    nib[: vals.size] = vals  # every code at least once
    if wdt == "e2m1":
        codes = (nib[0::2] | (nib[1::2] << 4)).astype(np.uint8)
    else:
        codes = nib.astype(np.uint8)
    M = -(-K // 128) * 128  # whole 128-row tiles; rows past K are zero
    x = np.zeros((M, K), dtype=np.float32)
    x[:K] = np.eye(K, dtype=np.float32)
    y = run_linear(x, codes, wdt, scale, None, N, K)
    w = dequant(codes, wdt, N * K, scale).reshape(N, K)
    # exact values; a -0 weight legitimately sums to +0 (0*w + 1*(-0) = +0)
    assert np.array_equal(y[:K], np.ascontiguousarray(w.T))
    assert not np.any(y[K:])


def test_golden_fixture(golden):
    g = golden["products"]
    codes = g["lin_codes"]
    N, K = codes.shape
    y = run_linear(g["lin_x"], codes.reshape(-1), "e4m3", float(g["lin_scale"][0]),
                   g["lin_bias"], N, K)
    assert normwise(y, g["lin_y"].astype(np.float64)) <= TOL


@pytest.mark.parametrize("wdt", ["e4m3", "e5m2", "e2m1"])
@pytest.mark.parametrize("M,N,K", [(1, 5, 10), (7, 300, 64), (130, 257, 130), (256, 512, 96),
                                   (33, 31, 4098), (2, 3, 2), (1, 5, 11), (33, 31, 4097),
                                   (130, 257, 129), (3, 4, 1)])
@pytest.mark.parametrize("with_bias", [True, False])
def test_ragged_shapes_vs_oracle(wdt, M, N, K, with_bias):
    """Any shape; E2M1 rows of odd length are stored as whole bytes (a +0
    pad nibble ends each row)."""
    print(f"linear ragged {wdt} {M}x{N}x{K} bias={with_bias}", flush=True)
    rng = np.random.default_rng(M * 7 + N * 3 + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * np.sqrt(2.0 / K)).astype(np.float32)
    c = QCODE[wdt]
    s = O.scale_from_amax(O.amax(w), c)
    kp = K + (K % 2 if wdt == "e2m1" else 0)
    wp = np.pad(w, ((0, 0), (0, kp - K)))
    codes = O.cast(wp.reshape(-1), O.F32, c, scale=s)
    b = rng.standard_normal(N).astype(np.float32) if with_bias else None
    y = run_linear(x, codes, wdt, s, b, N, K)
    r = O.linear_f64(x, dequant(codes, wdt, N * kp, s).reshape(N, kp)[:, :K], b)
    assert normwise(y, r.astype(np.float64)) <= TOL


@pytest.mark.parametrize("wdt", ["e4m3", "e5m2", "e2m1", "bf16", "f16"])
@pytest.mark.parametrize("M,N,K", [(128, 256, 64), (256, 512, 128), (384, 768, 320),
                                   (256, 384, 192), (128, 256, 1024), (128, 256, 384),
                                   (256, 768, 640)])
def test_whole_tile_shapes_vs_oracle(wdt, M, N, K):
    """Shapes that take the guard-free kernels (M % 128, N % 128, K % 64 == 0):
    ping-pong (FP8) / wide-K (FP4) when N % 256 and K % 128 are 0,
    staged-decode at tile width 256 or 128 otherwise and for 16-bit weights."""
    rng = np.random.default_rng(M + N + K)
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * np.sqrt(2.0 / K)).astype(np.float32)
    b = rng.standard_normal(N).astype(np.float32)
    code = QCODE.get(wdt, {"bf16": O.BF16, "f16": O.F16}.get(wdt))
    if wdt in QCODE:
        s = O.scale_from_amax(O.amax(w), code)
        codes = O.cast(w.reshape(-1), O.F32, code, scale=s)
        wf = dequant(codes, wdt, N * K, s).reshape(N, K)
    else:
        s = None
        codes = O.cast(w.reshape(-1), O.F32, code)
        wf = O.cast(codes, code, O.F32).reshape(N, K)
    y = run_linear(x, codes, wdt, s, b, N, K)
    assert normwise(y, O.linear_f64(x, wf, b).astype(np.float64)) <= TOL


@pytest.mark.parametrize("wdt", ["bf16", "f16", "f32"])
def test_unquantized_weight_dtypes(wdt):
    rng = np.random.default_rng(3)
    M, N, K = 96, 200, 300
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * 0.05).astype(np.float32)
    code = {"bf16": O.BF16, "f16": O.F16, "f32": O.F32}[wdt]
    stored = O.cast(w.reshape(-1), O.F32, code) if wdt != "f32" else w.reshape(-1)
    y = run_linear(x, stored, wdt, None, None, N, K)
    wf = O.cast(stored, code, O.F32).reshape(N, K) if wdt != "f32" else w
    assert normwise(y, O.linear_f64(x, wf).astype(np.float64)) <= TOL


def test_config4_full_size():
    """BASELINE config [4]: x (2048, 4096) N(0,1), W (4096, 4096) Kaiming-normal
    -> E4M3 with per-tensor amax scale, b = 0."""
    rng = np.random.default_rng(4)
    M, K, N = 2048, 4096, 4096
    x = rng.standard_normal((M, K), dtype=np.float32)
    w = (rng.standard_normal((N, K), dtype=np.float32) * np.float32(np.sqrt(2.0 / K)))
    wq = QuantizedParameters.from_float(w, "e4m3")
    b = Parameters(np.zeros((1, N), dtype=np.float32))
    xd = torch.from_numpy(x).cuda()
    y = F.linear(xd, wq, b)
    torch.cuda.synchronize()
    yh = y.cpu().numpy()
    wdeq = wq.dequantize().cpu().numpy().astype(np.float64)
    r = x.astype(np.float64) @ wdeq.T
    rep = error_report(yh, r)
    err = rep["normwise"]
    assert err <= TOL, err
    # against the fp64 product of the operands the MFMAs multiply (x rounded
    # to bf16, W decoded exactly): only fp32 summation error is left, so a
    # staging or ordering slip that costs even a few 1e-4 fails here
    exact = error_report(yh, bf16_round(x).astype(np.float64) @ wdeq.T)
    print(f"config [4] vs fp32-input fp64 product: {rep}", flush=True)
    print(f"config [4] vs exact-operand fp64 product: {exact}", flush=True)
    assert exact["normwise"] <= 1e-5, exact
    # quantized weights themselves are the oracle's, bit for bit
    s = O.scale_from_amax(O.amax(w), O.E4M3)
    assert wq.scale.item() == s
    assert np.array_equal(to_host(wq.codes), O.cast(w.reshape(-1), O.F32, O.E4M3, scale=s))


def test_zero_sizes():
    lib = _lib.load()
    stream = torch.cuda.current_stream().cuda_stream
    y = torch.full((4, 3), 7.0, device="cuda")
    b = torch.tensor([1.0, 2.0, 3.0], device="cuda")
    x = torch.empty((4, 0), device="cuda")
    w = torch.empty(16, dtype=torch.uint8, device="cuda")
    _lib.check(lib.novaq_linear_forward(x.data_ptr() or y.data_ptr(), 4, 0, w.data_ptr(), 3,
                                        None, b.data_ptr(), 3, y.data_ptr(), stream), "linear")
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), b.cpu().expand(4, 3))


def test_layer_shape_contracts_like_reference():
    """novann tests/layers/linear/test_linear.py:11-28 shape contracts."""
    rng = np.random.RandomState(8)
    layer = Linear(10, 5, bias=True, weight_dtype="e4m3")
    x = rng.randn(32, 10).astype(np.float32)
    out = layer(x)
    assert isinstance(out, np.ndarray) and out.shape == (32, 5) and out.dtype == np.float32
    layer = Linear(10, 5, bias=False, weight_dtype="e2m1")
    assert layer.bias is None and layer(x).shape == (32, 5)
    # fp32 weights, numpy in / numpy out
    layer = Linear(10, 5, bias=True)
    out = layer(x)
    ref = x.astype(np.float64) @ layer.weight.data.T.astype(np.float64)
    assert normwise(out, ref) <= TOL


# ---------------------------------------------------------------------------

def identity_e4m3(n, rows=None):
    """E4M3 codes of an (rows, n) weight whose first n rows are I (1.0 =
    0x38) and the rest zero."""
    rows = n if rows is None else rows
    codes = np.zeros(rows * n, np.uint8)
    codes[: n * n : n + 1] = 0x38
    return codes


def test_identity_weight_reproduces_bf16_rounded_input():
    """W = I: y = x rounded to bf16 (nearest even) exactly, the operand the
    bf16 product multiplies; rows holding Inf or NaN give the IEEE results of
    the fp32 product (Inf * 0 = NaN)."""
    K = N = 256
    rng = np.random.default_rng(3)
    x = rng.standard_normal((128, K)).astype(np.float32)
    x *= (2.0 ** rng.integers(-40, 41, size=(128, 1))).astype(np.float32)
    x[1, 5] = np.inf
    x[2, 7] = -np.inf
    x[3, 9] = np.nan
    x[4, 1], x[4, 2] = np.inf, -np.inf
    y = run_linear(x, identity_e4m3(K), "e4m3", 1.0, None, N, K)
    xb = O.cast(O.cast(x, O.F32, O.BF16), O.BF16, O.F32).reshape(x.shape)
    with np.errstate(invalid="ignore"):
        want = xb @ np.eye(K, dtype=np.float32)
    assert np.array_equal(np.isnan(y), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(y[fin], want[fin])
    assert np.array_equal(y[5:], xb[5:])


@pytest.mark.parametrize("wdt", ["e4m3", "e5m2", "e2m1"])
def test_wide_dynamic_range_vs_oracle(wdt):
    """Rows whose magnitudes span 2^-60 .. 2^60, against the fp64 product,
    each row on its own scale."""
    rng = np.random.default_rng(11)
    M, K, N = 256, 512, 512
    x = rng.standard_normal((M, K)).astype(np.float32)
    x *= (2.0 ** rng.integers(-60, 61, size=(M, 1))).astype(np.float32)
    w = (rng.standard_normal((N, K)) * np.sqrt(2.0 / K)).astype(np.float32)
    q = quant.quantize(torch.from_numpy(w).cuda(), wdt)
    codes = q.data.view(torch.uint8).cpu().numpy().reshape(-1)
    s = float(q.scale.cpu().reshape(-1)[0])
    y = run_linear(x, codes, wdt, s, None, N, K)
    wd = dequant(codes, wdt, N * K, s).reshape(N, K).astype(np.float64)
    r = x.astype(np.float64) @ wd.T
    for i in range(M):
        assert normwise(y[i : i + 1], r[i : i + 1]) <= TOL, i


# ---------------------------------------------------------------------------
# x stored as E4M3 / E5M2 (M % 128, N % 256, K % 128 with FP8 / FP4 weights):
# the codes of both operands go to gfx950's FP8 MFMA as they are stored.

def run_linear_x(xcodes, xdt, sx, M, K, codes, wdt, sw, N):
    xd = to_dev(xcodes, QCODE[xdt])
    wd = to_dev(codes, QCODE[wdt])
    sxd = torch.tensor([sx], dtype=torch.float32, device="cuda")
    swd = torch.tensor([sw], dtype=torch.float32, device="cuda")
    yd = torch.empty((M, N), dtype=torch.float32, device="cuda")
    _lib.check(_lib.load().novaq_linear_forward_ex(
        xd.data_ptr(), _lib.DTYPES[xdt], sxd.data_ptr(), M, K, wd.data_ptr(), _lib.DTYPES[wdt],
        swd.data_ptr(), None, N, None, yd.data_ptr(), torch.cuda.current_stream().cuda_stream),
        "linear_ex")
    torch.cuda.synchronize()
    return yd.cpu().numpy()


@pytest.mark.parametrize("xdt", ["e4m3", "e5m2"])
def test_fp8_x_identity_weight_exact(xdt):
    """W = I: y = s_x * dec(x) exactly for every code of x, Inf and NaN codes
    (E5M2) included, with the IEEE results of the fp32 product (Inf * 0 =
    NaN in the other columns of the row)."""
    K = N = 256
    M = 256
    rng = np.random.default_rng(5)
    xc = rng.integers(0, 256, size=M * K, dtype=np.uint8)
    xc[:256] = np.arange(256, dtype=np.uint8)  # every code
    sx = 0.375
    y = run_linear_x(xc, xdt, sx, M, K, identity_e4m3(K), "e4m3", 1.0, N)
    xv = (O.cast(xc, QCODE[xdt], O.F32).astype(np.float32) * np.float32(sx)).reshape(M, K)
    with np.errstate(invalid="ignore"):
        want = xv @ np.eye(K, dtype=np.float32)
    assert np.array_equal(np.isnan(y), np.isnan(want))
    fin = ~np.isnan(want)
    assert np.array_equal(y[fin], want[fin])


@pytest.mark.parametrize("xdt", ["e4m3", "e5m2"])
@pytest.mark.parametrize("wdt", ["e4m3", "e5m2", "e2m1"])
def test_fp8_x_vs_oracle(xdt, wdt):
    """Quantized activations times quantized weights, against the fp64
    product of the two dequantized operands, with a bias."""
    rng = np.random.default_rng(17)
    M, K, N = 256, 768, 512
    x = rng.standard_normal((M, K)).astype(np.float32)
    w = (rng.standard_normal((N, K)) * np.sqrt(2.0 / K)).astype(np.float32)
    qx = quant.quantize(torch.from_numpy(x).cuda(), xdt)
    qw = quant.quantize(torch.from_numpy(w).cuda(), wdt)
    xc = qx.data.view(torch.uint8).cpu().numpy().reshape(-1)
    wc = qw.data.view(torch.uint8).cpu().numpy().reshape(-1)
    sx, sw = float(qx.scale.cpu().reshape(-1)[0]), float(qw.scale.cpu().reshape(-1)[0])
    y = run_linear_x(xc, xdt, sx, M, K, wc, wdt, sw, N)
    xd = dequant(xc, xdt, M * K, sx).reshape(M, K).astype(np.float64)
    wd = dequant(wc, wdt, N * K, sw).reshape(N, K).astype(np.float64)
    assert normwise(y, xd @ wd.T) <= 1e-4


def test_odd_width_e2m1_layer_forward_backward_step():
    """A Linear(11 -> 6) with E2M1 weights: rows stored as whole bytes, the
    forward and all three gradients against the oracle, and an AdamW step that
    keeps the pad column at zero and the re-quantized codes consistent."""
    from oracle import functional_ref as R
    from novann_amd.optim import AdamW
    rng = np.random.RandomState(3)
    layer = Linear(11, 6, bias=True, weight_dtype="e2m1")
    assert layer.weight.stored_shape == (6, 12) and layer.weight.codes.numel() == 36
    x = rng.randn(9, 11).astype(np.float32)
    wdeq = layer.weight.dequantize().cpu().numpy()
    assert wdeq.shape == (6, 11)
    y = layer(x)
    r = O.linear_f64(x, wdeq, layer.bias.data)
    assert normwise(y, r) <= TOL
    G = rng.randn(9, 6).astype(np.float32)
    gi = layer.backward(G)
    ri, rw, rb = R.linear_backward(G.astype(np.float64), x.astype(np.float64),
                                   wdeq.astype(np.float64))
    assert normwise(gi, ri) <= TOL and normwise(layer.weight.grad, rw) <= TOL
    assert normwise(layer.bias.grad, rb) <= TOL
    opt = AdamW(layer.parameters(), lr=1e-2)
    opt.step()
    torch.cuda.synchronize()
    m = layer.weight.master.cpu().numpy()
    assert m.shape == (6, 12) and not m[:, 11].any()
    codes = to_host(layer.weight.codes)
    s = float(layer.weight.scale.cpu()[0])
    assert np.array_equal(codes, O.cast(m.reshape(-1), O.F32, O.E2M1, scale=s))
    assert codes.reshape(6, 6)[:, 5].max() >> 4 == 0   # pad nibbles are +0


def test_misaligned_device_views_are_copied_not_refused():
    """Views starting inside a 16-byte group (slices of a larger tensor) work
    through the host layer: products, casts (input and output views) and
    quantize give the results of the aligned tensors."""
    rng = np.random.default_rng(12)
    M, K, N = 8, 64, 32
    big = torch.from_numpy(rng.standard_normal(M * K + 1).astype(np.float32)).cuda()
    x = big[1:].view(M, K)
    assert x.data_ptr() % 16 != 0
    w = (rng.standard_normal((N, K)) * 0.1).astype(np.float32)
    wq = QuantizedParameters.from_float(w, "e4m3")
    y = F.linear(x, wq, None)
    y_ref = F.linear(x.clone(), wq, None)
    torch.cuda.synchronize()
    assert torch.equal(y.cpu(), y_ref.cpu())
    out = torch.empty(M * K + 3, dtype=torch.float16, device="cuda")
    got = quant.cast(big[1:], "f16", out=out[3:])
    torch.cuda.synchronize()
    assert got.data_ptr() == out[3:].data_ptr()
    assert torch.equal(out[3:].cpu(), quant.cast(big[1:].clone(), "f16").cpu())
    q1, q2 = quant.quantize(big[1:], "e4m3"), quant.quantize(big[1:].clone(), "e4m3")
    torch.cuda.synchronize()
    assert torch.equal(q1.data.view(torch.uint8).cpu(), q2.data.view(torch.uint8).cpu())
    assert q1.scale.item() == q2.scale.item()


@pytest.mark.parametrize("wdt", ["e4m3", "e5m2"])
def test_longest_k_one_hot_rows(wdt):
    """K = 2^21, the longest K the K-block kernels take, forward (W rows of 2
    MiB) and backward grad_input (W read in its [K][N] layout): every row of x
    (of grad) is one-hot at a K index spread over the whole range, the first
    and the last included, so y[i, :] = s * dec(W[:, k_i]) (grad_input[i, :]
    = s * dec(W[k_i, :])) exactly -- the offsets of the last K blocks, near
    the top of the 31-bit buffer ranges, are exercised."""
    M, N, K = 128, 256, 1 << 21
    print(f"longest K one-hot {wdt}", flush=True)
    g = torch.Generator(device="cuda")
    g.manual_seed(21)
    codes = torch.randint(0, 256, (N, K), generator=g, device="cuda", dtype=torch.int32)
    if wdt == "e4m3":  # no NaN codes (0x7F / 0xFF)
        codes = torch.where((codes & 0x7F) == 0x7F, codes - 1, codes)
    else:  # no Inf / NaN codes (exponent all ones): clear the exponent's low bit
        codes = torch.where((codes & 0x7C) == 0x7C, codes & 0xFB, codes)
    codes = codes.to(torch.uint8).contiguous()
    s = 0.0123
    sd = torch.tensor([s], dtype=torch.float32, device="cuda")
    rng = np.random.default_rng(21)
    ks = rng.integers(0, K, size=M)
    ks[0], ks[1], ks[2] = 0, K - 1, K - 128
    kd = torch.from_numpy(ks).cuda()
    rows = torch.arange(M, device="cuda")
    lib, stream = _lib.load(), torch.cuda.current_stream().cuda_stream
    code = _lib.DTYPES[wdt]

    x = torch.zeros((M, K), dtype=torch.float32, device="cuda")
    x[rows, kd] = 1.0
    y = torch.empty((M, N), dtype=torch.float32, device="cuda")
    _lib.check(lib.novaq_linear_forward(x.data_ptr(), M, K, codes.data_ptr(), code, sd.data_ptr(),
                                        None, N, y.data_ptr(), stream), "linear")
    cols = codes[:, kd].t().contiguous().cpu().numpy()  # (M, N): W[:, k_i]
    want = O.cast(cols.reshape(-1), QCODE[wdt], O.F32, scale=s).view(np.float32).reshape(M, N)
    torch.cuda.synchronize()
    assert np.array_equal(y.cpu().numpy(), want)
    del x, y

    # backward: W (D_out = K, D_in = N) is the same bytes read as [K][N]
    wkn = codes.view(K, N)
    assert lib.novaq_linear_backward_workspace(M, N, K, code) == 0
    grad = torch.zeros((M, K), dtype=torch.float32, device="cuda")
    grad[rows, kd] = 1.0
    gi = torch.empty((M, N), dtype=torch.float32, device="cuda")
    _lib.check(lib.novaq_linear_backward(grad.data_ptr(), None, M, N, wkn.data_ptr(), code,
                                         sd.data_ptr(), K, gi.data_ptr(), None, None, None, 0,
                                         stream), "linear backward")
    rows_w = wkn[kd].contiguous().cpu().numpy()  # (M, N): W[k_i, :]
    want_b = O.cast(rows_w.reshape(-1), QCODE[wdt], O.F32, scale=s).view(np.float32).reshape(M, N)
    torch.cuda.synchronize()
    assert np.array_equal(gi.cpu().numpy(), want_b)
