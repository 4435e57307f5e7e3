"""Backward products of the quantized Linear on the GPU (through the C ABI) vs
the CPU restatement of Linear.backward (novann/layers/linear/linear.py:85-108),
plus the layout kernels they are built from.

Tolerances: transposes are bit-exact (codes permuted; fp32 -> bf16 / fp16 by
the oracle's cast); the column sum is an fp32 sum, within 1e-5 relative of
fp64; the gradients are normwise max|g - r| / max|r| <= 1e-2 against fp64 on
the same fp32 inputs and the dequantized weight (the BASELINE tolerance of the
forward product)."""
import numpy as np
import pytest
import torch

import oracle as O
from oracle import functional_ref as R
from novann_amd import _lib
from novann_amd import functional as F
from novann_amd.module import Linear, Parameters, QuantizedParameters
from tests.gpu_util import to_dev, to_host

pytestmark = pytest.mark.gpu

TOL = 1e-2
STORAGE = {O.F32: np.uint32, O.F16: np.uint16, O.BF16: np.uint16, O.E4M3: np.uint8,
           O.E5M2: np.uint8}


def normwise(g, r):
    return float(np.abs(g.astype(np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


def transpose_dev(src_codes, st, rows, cols, dt):
    """novaq_transpose on raw storage; returns the destination storage."""
    src = to_dev(src_codes, st)
    if dt == O.E2M1:
        dst = torch.empty(rows * cols // 2, dtype=torch.uint8, device="cuda")
    else:
        dst = torch.empty(rows * cols, dtype={O.F32: torch.float32, O.F16: torch.float16,
                                              O.BF16: torch.bfloat16, O.E4M3: torch.uint8,
                                              O.E5M2: torch.uint8}[dt], device="cuda")
    _lib.check(_lib.load().novaq_transpose(src.data_ptr(), st, rows, cols, dst.data_ptr(), dt,
                                           torch.cuda.current_stream().cuda_stream), "transpose")
    torch.cuda.synchronize()
    return to_host(dst)


def unpack_nibbles(b, n):
    b = np.asarray(b, np.uint8)
    return np.stack([b & 0xF, b >> 4], axis=1).reshape(-1)[:n]


def pack_nibbles(c):
    c = np.asarray(c, np.uint8).reshape(-1, 2)
    return (c[:, 0] | (c[:, 1] << 4)).astype(np.uint8)


@pytest.mark.parametrize("shape", [(1, 1), (3, 5), (64, 64), (65, 130), (200, 77), (128, 4096),
                                   (16, 16), (48, 272), (400, 144)])
@pytest.mark.parametrize("dt", [O.F32, O.F16, O.BF16, O.E4M3, O.E5M2])
def test_transpose_permutes_codes_exactly(shape, dt):
    rows, cols = shape
    rng = np.random.default_rng(rows * 1000 + cols + dt)
    codes = rng.integers(0, np.iinfo(STORAGE[dt]).max, size=rows * cols,
                         dtype=np.uint64).astype(STORAGE[dt])
    got = transpose_dev(codes, dt, rows, cols, dt)
    want = codes.reshape(rows, cols).T.reshape(-1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("shape", [(2, 2), (4, 6), (64, 128), (130, 66), (256, 4096)])
def test_transpose_e2m1_nibbles(shape):
    rows, cols = shape
    rng = np.random.default_rng(rows + cols)
    codes = rng.integers(0, 16, size=rows * cols).astype(np.uint8)
    got = transpose_dev(pack_nibbles(codes), O.E2M1, rows, cols, O.E2M1)
    want = pack_nibbles(codes.reshape(rows, cols).T.reshape(-1))
    assert np.array_equal(got, want)


# (97, 130): the element tile kernel; the rest (rows % 8 == 0, cols % 4 == 0)
# the 16-byte tile kernel, partial tiles included
@pytest.mark.parametrize("shape", [(97, 130), (8, 4), (96, 132), (200, 68), (1024, 256)])
@pytest.mark.parametrize("dt", [O.BF16, O.F16])
def test_transpose_rounds_f32_like_the_cast(dt, shape):
    rows, cols = shape
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(rows * cols) * np.exp2(rng.integers(-30, 30, rows * cols))
         ).astype(np.float32)
    x[:8] = [0.0, -0.0, np.inf, -np.inf, np.nan, 1e-40, -1e-42, 65520.0]
    got = transpose_dev(x.view(np.uint32), O.F32, rows, cols, dt)
    want = O.cast(np.ascontiguousarray(x.reshape(rows, cols).T).reshape(-1), O.F32, dt)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("shape", [(1, 1), (2048, 4096), (5, 70), (1000, 3)])
def test_colsum(shape):
    rows, cols = shape
    rng = np.random.default_rng(rows + cols)
    x = rng.standard_normal((rows, cols)).astype(np.float32)
    xd = torch.from_numpy(x).cuda()
    out = torch.empty(cols, dtype=torch.float32, device="cuda")
    _lib.check(_lib.load().novaq_colsum(xd.data_ptr(), rows, cols, out.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream), "colsum")
    want = x.astype(np.float64).sum(axis=0)
    np.testing.assert_allclose(out.cpu().numpy(), want, rtol=1e-5, atol=1e-5 * np.sqrt(rows))


def weight_of(w, wdt):
    if wdt in ("e4m3", "e5m2", "e2m1"):
        q = QuantizedParameters.from_float(w, wdt)
        return q, q.dequantize().cpu().numpy().astype(np.float64)
    if wdt == "f32":
        return Parameters(w), w.astype(np.float64)
    raise ValueError(wdt)


@pytest.mark.parametrize("wdt", ["e4m3", "e5m2", "e2m1", "f32"])
@pytest.mark.parametrize("N,D_in,D_out", [
    (256, 512, 256),     # whole tiles: the fast forward kernels on both products
    (2048, 1024, 512),
    (64, 96, 40),        # ragged: guarded kernels
    (33, 70, 46),
])
def test_linear_backward_vs_oracle(wdt, N, D_in, D_out):
    rng = np.random.default_rng(N + D_in + D_out)
    x = rng.standard_normal((N, D_in)).astype(np.float32)
    g = rng.standard_normal((N, D_out)).astype(np.float32)
    w = (rng.standard_normal((D_out, D_in)) * np.sqrt(2.0 / D_in)).astype(np.float32)
    weight, wdeq = weight_of(w, wdt)
    gi, gw, gb = F.linear_backward(torch.from_numpy(g).cuda(), torch.from_numpy(x).cuda(),
                                   weight, True)
    torch.cuda.synchronize()
    ri, rw, rb = R.linear_backward(g.astype(np.float64), x.astype(np.float64), wdeq)
    assert gi.shape == (N, D_in) and gw.shape == (D_out, D_in) and gb.shape == (1, D_out)
    assert normwise(gi.cpu().numpy(), ri) <= TOL
    assert normwise(gw.cpu().numpy(), rw) <= TOL
    assert normwise(gb.cpu().numpy(), rb) <= TOL


def bf16_round(a):
    """fp32 -> bf16 (nearest even) -> fp32, by the oracle's cast."""
    flat = np.ascontiguousarray(a, np.float32).reshape(-1)
    return O.cast(O.cast(flat, O.F32, O.BF16), O.BF16, O.F32).reshape(a.shape)


# D_out % 128, D_in % 256, N % 64: the weight gradient reads grad and x in
# place (transposing LDS reads); tile counts 1, 9 (not a multiple of 8) and 16,
# and config [4]'s weight (256 x 256 tiles, one per CU)
@pytest.mark.parametrize("N,D_in,D_out", [(64, 256, 128), (128, 768, 384), (192, 1024, 512),
                                          (1024, 4096, 4096)])
def test_weight_gradient_in_place_product(N, D_in, D_out):
    """grad_weight = grad^T x equals the fp64 product of the bf16-rounded
    operands up to fp32 summation error (1e-5 normwise): an index or layout
    slip in the transposing reads is far outside that; likewise grad_input on
    the bf16 copy of grad that product stores, and the fused bias sum."""
    print(f"grad_weight in place N={N} D_in={D_in} D_out={D_out}", flush=True)
    rng = np.random.default_rng(N * 7 + D_in)
    x = rng.standard_normal((N, D_in)).astype(np.float32)
    g = rng.standard_normal((N, D_out)).astype(np.float32)
    w, wdeq = weight_of((rng.standard_normal((D_out, D_in)) * 0.05).astype(np.float32), "e4m3")
    gi, gw, gb = F.linear_backward(torch.from_numpy(g).cuda(), torch.from_numpy(x).cuda(), w,
                                   True)
    torch.cuda.synchronize()
    g16 = bf16_round(g).astype(np.float64)
    assert normwise(gw.cpu().numpy(), g16.T @ bf16_round(x).astype(np.float64)) <= 1e-5
    assert normwise(gb.cpu().numpy(), g.astype(np.float64).sum(0, keepdims=True)) <= 1e-5
    # grad_input multiplies the bf16 grad the weight-gradient product left behind
    assert normwise(gi.cpu().numpy(), g16 @ wdeq) <= 1e-5
    lib = _lib.load()
    assert lib.novaq_linear_backward_workspace(N, D_in, D_out, 3) < \
        lib.novaq_linear_backward_workspace(N + 1, D_in, D_out, 3)


@pytest.mark.parametrize("N,D_in,D_out,dt", [(128, 256, 128, "e4m3"), (256, 512, 384, "e5m2"),
                                          (384, 768, 1024, "e4m3"), (128, 512, 256, "e2m1")])
def test_input_gradient_on_weight_codes_in_place(N, D_in, D_out, dt):
    """grad_input = bf16(grad) @ (s * dec(W)) with W's FP8 codes read in their
    stored (D_out, D_in) layout through transposing LDS reads, and the fp32
    grad rounded to bf16 while staged: within 1e-5 normwise of the fp64
    product, with and without grad_weight asked for; E2M1 takes the transposed
    copy.  The in-place shapes need no workspace (NULL is accepted)."""
    print(f"grad_input in place N={N} D_in={D_in} D_out={D_out} {dt}", flush=True)
    rng = np.random.default_rng(N + D_in * 3 + D_out)
    x = rng.standard_normal((N, D_in)).astype(np.float32)
    g = rng.standard_normal((N, D_out)).astype(np.float32)
    w, wdeq = weight_of((rng.standard_normal((D_out, D_in)) * 0.05).astype(np.float32), dt)
    ref = bf16_round(g).astype(np.float64) @ wdeq
    gi, gw, _ = F.linear_backward(torch.from_numpy(g).cuda(), torch.from_numpy(x).cuda(), w,
                                  False)
    torch.cuda.synchronize()
    assert normwise(gi.cpu().numpy(), ref) <= 1e-5
    assert normwise(gw.cpu().numpy(), bf16_round(g).astype(np.float64).T @
                    bf16_round(x).astype(np.float64)) <= 1e-5
    lib = _lib.load()
    wdt = {"e4m3": O.E4M3, "e5m2": O.E5M2, "e2m1": O.E2M1}[dt]
    nbytes = lib.novaq_linear_backward_workspace(N, D_in, D_out, wdt)
    work = torch.empty(max(nbytes, 1), dtype=torch.uint8, device="cuda")
    gd = torch.from_numpy(g).cuda()
    gi2 = torch.full((N, D_in), float("nan"), device="cuda")
    st = torch.cuda.current_stream().cuda_stream
    _lib.check(lib.novaq_linear_backward(gd.data_ptr(), None, N, D_in, w.codes.data_ptr(), wdt,
                                         w.scale.data_ptr(), D_out, gi2.data_ptr(), None, None,
                                         work.data_ptr() if nbytes else None, nbytes, st), "bwd")
    torch.cuda.synchronize()
    assert normwise(gi2.cpu().numpy(), ref) <= 1e-5
    # FP8 W: no workspace (W's codes and the fp32 grad read in place); E2M1:
    # W^T, then the bf16 grad the weight-gradient product leaves
    grad_bytes = -(-N * D_out * 2 // 256) * 256
    wt_bytes = -(-D_in * D_out * 4 // 8 // 256) * 256
    assert nbytes == (wt_bytes + grad_bytes if dt == "e2m1" else 0)


def test_linear_backward_skips_null_outputs_and_empty_batch():
    rng = np.random.default_rng(3)
    w = QuantizedParameters.from_float(rng.standard_normal((64, 128)).astype(np.float32), "e4m3")
    lib = _lib.load()
    st = torch.cuda.current_stream().cuda_stream
    # N = 0: grad_weight and grad_bias are zeros
    gw = torch.full((64, 128), 7.0, device="cuda")
    gb = torch.full((64,), 7.0, device="cuda")
    ws = torch.empty(lib.novaq_linear_backward_workspace(0, 128, 64, 3) + 16,
                     dtype=torch.uint8, device="cuda")
    dummy = torch.empty(4, device="cuda")
    _lib.check(lib.novaq_linear_backward(dummy.data_ptr(), dummy.data_ptr(), 0, 128,
                                         w.codes.data_ptr(), 3, w.scale.data_ptr(), 64, None,
                                         gw.data_ptr(), gb.data_ptr(), ws.data_ptr(),
                                         ws.numel(), st), "bwd")
    torch.cuda.synchronize()
    assert torch.count_nonzero(gw).item() == 0 and torch.count_nonzero(gb).item() == 0
    # only the bias gradient: no workspace needed
    g = torch.from_numpy(rng.standard_normal((5, 64)).astype(np.float32)).cuda()
    _lib.check(lib.novaq_linear_backward(g.data_ptr(), None, 5, 128, None, 3, None, 64, None,
                                         None, gb.data_ptr(), None, 0, st), "bwd")
    torch.cuda.synchronize()
    np.testing.assert_allclose(gb.cpu().numpy(), g.cpu().numpy().astype(np.float64).sum(0),
                               rtol=1e-5, atol=1e-6)


def test_layer_backward_like_reference():
    """novann tests/layers/linear/test_linear.py:31-64 on the quantized layer:
    gradients against the oracle (whose finite-difference agreement is pinned
    on the CPU) and the grad_input shape."""
    rng = np.random.RandomState(0)
    layer = Linear(in_features=64, out_features=32, bias=True, weight_dtype="e4m3")
    x = rng.randn(16, 64).astype(np.float32) * 0.1
    G = rng.randn(16, 32).astype(np.float32) * 0.1
    out = layer(x)
    assert out.shape == (16, 32)
    grad_input = layer.backward(G)
    wdeq = layer.weight.dequantize().cpu().numpy().astype(np.float64)
    ri, rw, rb = R.linear_backward(G.astype(np.float64), x.astype(np.float64), wdeq)
    assert isinstance(grad_input, np.ndarray) and grad_input.shape == x.shape
    assert layer.weight.grad.shape == (32, 64) and layer.bias.grad.shape == (1, 32)
    assert normwise(layer.weight.grad, rw) <= TOL
    assert normwise(layer.bias.grad, rb) <= TOL
    assert normwise(grad_input, ri) <= TOL
