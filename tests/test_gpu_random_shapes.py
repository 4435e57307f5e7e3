"""Random geometries through the C ABI against the oracle: Conv2d forward
(every padding mode and weight dtype, strides 1-3, windows up to 5 x 5, 1 to
80 channels), Conv2d and Linear backward, Linear forward (ragged and
whole-tile shapes), MaxPool2d and GlobalAvgPool2d.  Each case is drawn from a
seeded generator and printed before it runs; the bars are the suites' own
(normwise 1e-2 against fp64 for the products and gradients, bit-exact for the
pools; the fused epilogues bit-exact on the unfused output, every narrow store
equal to the oracle's cast)."""
import numpy as np
import pytest
import torch

import oracle as O
from oracle import functional_ref as R
from novann_amd import functional as F
from tests import test_gpu_backward as TLB
from tests import test_gpu_conv2d as TC
from tests import test_gpu_conv2d_backward as TB
from tests import test_gpu_epilogue as TE
from tests import test_gpu_linear as TL

pytestmark = pytest.mark.gpu

TOL = 1e-2
SEEDS = [11, 12, 13]
MODES = ["zeros", "reflect", "replicate", "circular"]


def conv_case(rng):
    while True:
        N = int(rng.integers(1, 4))
        C = int(rng.choice([1, 2, 3, 4, 5, 8, 16, 24, 32, 40, 64, 70]))
        H, W = int(rng.integers(1, 41)), int(rng.integers(1, 41))
        KH, KW = int(rng.integers(1, 6)), int(rng.integers(1, 6))
        sh, sw = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        ph, pw = int(rng.integers(0, 4)), int(rng.integers(0, 4))
        C_out = int(rng.choice([1, 3, 8, 16, 32, 40, 64, 65, 80]))
        mode = str(rng.choice(MODES))
        if H + 2 * ph < KH or W + 2 * pw < KW:
            continue
        if mode == "reflect" and (ph >= H or pw >= W):
            continue
        if mode == "circular" and (ph > H or pw > W):
            continue
        wdt = str(rng.choice(["e2m1", "e4m3", "e5m2", "bf16", "f16", "f32"]))
        return N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, mode, wdt


@pytest.mark.parametrize("seed", SEEDS)
def test_conv2d_random_geometries(seed):
    rng = np.random.default_rng(seed)
    for i in range(40):
        case = conv_case(rng)
        N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, mode, wdt = case
        print(f"conv2d seed {seed} case {i}: {case}", flush=True)
        x = rng.standard_normal((N, C, H, W)).astype(np.float32)
        w = (rng.standard_normal((C_out, C, KH, KW)) *
             np.sqrt(2.0 / (C * KH * KW))).astype(np.float32)
        b = rng.standard_normal(C_out).astype(np.float32)
        codes, s, wdeq = TC.quantize_weights(w, wdt)
        y = TC.run_conv(x, codes, wdt, w.shape, s, b, (sh, sw), (ph, pw), mode)
        r = O.conv2d_f64(x, wdeq, (sh, sw), (ph, pw), mode, b)
        assert TC.normwise(y, r.astype(np.float64)) <= TOL, case


@pytest.mark.parametrize("seed", SEEDS)
def test_conv2d_backward_random_geometries(seed):
    rng = np.random.default_rng(seed + 100)
    for i in range(15):
        while True:
            N, C = int(rng.integers(1, 4)), int(rng.choice([1, 2, 3, 8, 16, 32, 64, 70]))
            H, W = int(rng.integers(2, 24)), int(rng.integers(2, 24))
            KH, KW = int(rng.integers(1, 5)), int(rng.integers(1, 5))
            st = (int(rng.integers(1, 3)), int(rng.integers(1, 3)))
            pd = (int(rng.integers(0, 3)), int(rng.integers(0, 3)))
            C_out = int(rng.choice([1, 4, 16, 24, 64, 70]))
            mode = str(rng.choice(["zeros", "zeros"] + MODES[1:]))
            if H + 2 * pd[0] < KH or W + 2 * pd[1] < KW:
                continue
            if mode != "zeros" and (pd[0] >= H or pd[1] >= W):
                continue
            break
        wdt = str(rng.choice(["e2m1", "e4m3", "e5m2", "f32"]))
        TB.check_case(N, C, H, W, C_out, KH, KW, st, pd, wdt, mode, seed=seed * 1000 + i)


@pytest.mark.parametrize("seed", SEEDS)
def test_linear_random_shapes(seed):
    rng = np.random.default_rng(seed + 200)
    for i in range(25):
        M, N, K = int(rng.integers(1, 300)), int(rng.integers(1, 600)), int(rng.integers(1, 700))
        if rng.random() < 0.3:  # whole tiles: the wide / pipe kernels
            M, N, K = (128 * int(rng.integers(1, 4)), 256 * int(rng.integers(1, 3)),
                       64 * int(rng.integers(1, 9)))
        wdt = str(rng.choice(["e4m3", "e5m2", "e2m1"]))
        with_bias = bool(rng.random() < 0.5)
        print(f"linear seed {seed} case {i}: {(M, N, K, wdt, with_bias)}", flush=True)
        x = rng.standard_normal((M, K)).astype(np.float32)
        w = (rng.standard_normal((N, K)) * np.sqrt(2.0 / K)).astype(np.float32)
        c = TL.QCODE[wdt]
        s = O.scale_from_amax(O.amax(w), c)
        kp = K + (K % 2 if wdt == "e2m1" else 0)
        codes = O.cast(np.pad(w, ((0, 0), (0, kp - K))).reshape(-1), O.F32, c, scale=s)
        b = rng.standard_normal(N).astype(np.float32) if with_bias else None
        y = TL.run_linear(x, codes, wdt, s, b, N, K)
        r = O.linear_f64(x, TL.dequant(codes, wdt, N * kp, s).reshape(N, kp)[:, :K], b)
        assert TL.normwise(y, r.astype(np.float64)) <= TOL, (M, N, K, wdt)


@pytest.mark.parametrize("seed", SEEDS)
def test_linear_backward_random_shapes(seed):
    rng = np.random.default_rng(seed + 300)
    for i in range(15):
        Nb, D_in, D_out = (int(rng.integers(1, 300)), int(rng.integers(1, 600)),
                           int(rng.integers(1, 500)))
        if rng.random() < 0.4:  # the in-place products' shapes
            Nb, D_in, D_out = (64 * int(rng.integers(1, 6)), 256 * int(rng.integers(1, 4)),
                               128 * int(rng.integers(1, 5)))
        wdt = str(rng.choice(["e4m3", "e5m2", "e2m1", "f32"]))
        if wdt == "e2m1":
            D_in, D_out = D_in + D_in % 2, D_out + D_out % 2
        print(f"linear backward seed {seed} case {i}: {(Nb, D_in, D_out, wdt)}", flush=True)
        x = rng.standard_normal((Nb, D_in)).astype(np.float32)
        g = rng.standard_normal((Nb, D_out)).astype(np.float32)
        w = (rng.standard_normal((D_out, D_in)) * np.sqrt(2.0 / D_in)).astype(np.float32)
        weight, wdeq = TLB.weight_of(w, wdt)
        gi, gw, gb = F.linear_backward(torch.from_numpy(g).cuda(), torch.from_numpy(x).cuda(),
                                       weight, True)
        torch.cuda.synchronize()
        ri, rw, rb = R.linear_backward(g.astype(np.float64), x.astype(np.float64), wdeq)
        for name, got, want in (("grad_input", gi, ri), ("grad_weight", gw, rw),
                                ("grad_bias", gb, rb)):
            assert TLB.normwise(got.cpu().numpy(), want) <= TOL, (name, Nb, D_in, D_out, wdt)


@pytest.mark.parametrize("seed", SEEDS)
def test_pools_random_shapes_bit_exact(seed):
    rng = np.random.default_rng(seed + 400)
    for i in range(25):
        N, C = int(rng.integers(1, 5)), int(rng.integers(1, 20))
        H, W = int(rng.integers(1, 60)), int(rng.integers(1, 60))
        x = (rng.standard_normal((N, C, H, W)) *
             np.exp2(rng.integers(-6, 6, (N, C, H, W)))).astype(np.float32)
        k = (int(rng.integers(1, min(H, 4) + 1)), int(rng.integers(1, min(W, 4) + 1)))
        st = (int(rng.integers(1, 4)), int(rng.integers(1, 4)))
        pd = (int(rng.integers(0, k[0] // 2 + 1)), int(rng.integers(0, k[1] // 2 + 1)))
        print(f"pools seed {seed} case {i}: {(N, C, H, W)} max {k} {st} {pd}", flush=True)
        got = F.avg_pool2d(x)
        assert np.array_equal(got.view(np.uint32), R.avg_pool2d(x).view(np.uint32))
        got = np.asarray(F.max_pool2d(x, k, st, pd, "zeros"))
        want = R.max_pool2d(x, k, st, pd, "zeros")
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


@pytest.mark.parametrize("seed", SEEDS)
def test_fused_epilogues_random_geometries(seed):
    """BN-style per-channel affine + ReLU + amax, and bf16 / f16 / E4M3 /
    E5M2 stores, on random convolutions and Linear shapes."""
    rng = np.random.default_rng(seed + 500)
    for i in range(8):
        N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, mode, wdt = conv_case(rng)
        print(f"conv epilogue seed {seed} case {i}: "
              f"{(N, C, H, W, C_out, KH, KW, sh, sw, ph, pw, mode, wdt)}", flush=True)
        x = rng.standard_normal((N, C, H, W)).astype(np.float32)
        wshape = (C_out, C, KH, KW)
        w = (rng.standard_normal(wshape) * np.sqrt(2.0 / (C * KH * KW))).astype(np.float32)
        bias = rng.standard_normal(C_out).astype(np.float32)
        wd, ws, _ = TE.quantized_codes(w, wdt, rng)
        run = lambda ep: TE.conv_ex(x, wd, wdt, ws, wshape, (sh, sw), (ph, pw), mode, ep,  # noqa: E731
                                    bias)
        TE.check_all_outputs(run, run(None), C_out, rng)
    for i in range(6):
        M, D_in, D_out = int(rng.integers(1, 300)), int(rng.integers(1, 600)), int(rng.integers(1, 500))
        if rng.random() < 0.5:
            M, D_in, D_out = (128 * int(rng.integers(1, 3)), 64 * int(rng.integers(1, 5)),
                              256 * int(rng.integers(1, 3)))
        wdt = str(rng.choice(["e4m3", "e5m2", "bf16"]))
        print(f"linear epilogue seed {seed} case {i}: {(M, D_in, D_out, wdt)}", flush=True)
        x = rng.standard_normal((M, D_in)).astype(np.float32)
        w = (rng.standard_normal((D_out, D_in)) * np.sqrt(2.0 / D_in)).astype(np.float32)
        bias = rng.standard_normal(D_out).astype(np.float32)
        wd, ws, _ = TE.quantized_codes(w, wdt, rng)
        run = lambda ep: TE.linear_ex(x, wd, wdt, ws, D_out, ep, bias)  # noqa: E731
        TE.check_all_outputs(run, run(None), D_out, rng)


def extras_case(rng):
    while True:
        N = int(rng.integers(1, 4))
        C = int(rng.integers(1, 9))
        H, W = int(rng.integers(1, 33)), int(rng.integers(1, 33))
        KH, KW = int(rng.integers(1, 6)), int(rng.integers(1, 6))
        sh, sw = int(rng.integers(1, 4)), int(rng.integers(1, 4))
        ph, pw = int(rng.integers(0, 6)), int(rng.integers(0, 6))
        mode = str(rng.choice(MODES))
        if H + 2 * ph < KH or W + 2 * pw < KW:
            continue
        xt = str(rng.choice(["f32", "f32", "bf16", "e4m3"]))
        return N, C, H, W, KH, KW, sh, sw, ph, pw, mode, xt


@pytest.mark.parametrize("seed", SEEDS)
def test_extras_random_geometries(seed):
    """The column matrix and the pooling window view (extras=True) over random
    geometries, padding wider than the image included (numpy.pad's rules),
    for fp32, bf16 and scaled E4M3 inputs: bit-equal to the oracle's
    restatement of the reference's as_strided windows on the decoded input."""
    from novann_amd import quant
    rng = np.random.default_rng(seed + 100)
    for i in range(40):
        case = extras_case(rng)
        N, C, H, W, KH, KW, sh, sw, ph, pw, mode, xt = case
        print(f"extras seed {seed} case {i}: {case}", flush=True)
        x = rng.standard_normal((N, C, H, W)).astype(np.float32)
        xd = torch.from_numpy(x).cuda()
        if xt == "bf16":
            arg = xd.to(torch.bfloat16)
            dec = arg.float().cpu().numpy()
        elif xt == "e4m3":
            arg = quant.quantize(xd, "e4m3")
            dec = quant.dequantize(arg).cpu().numpy()
        else:
            arg, dec = xd, x
        col = F.im2col(arg, (KH, KW), (sh, sw), (ph, pw), mode)
        want, OH, OW = R.im2col(dec, KH, KW, (sh, sw), (ph, pw), mode)
        assert np.array_equal(col.cpu().numpy().view(np.uint32), want.view(np.uint32)), case
        _, win, OH2, OW2, pshape = F.max_pool2d(arg, (KH, KW), (sh, sw), (ph, pw),
                                                padding_mode=mode, extras=True)
        assert (OH2, OW2, tuple(pshape)) == (OH, OW, (N, C, H + 2 * ph, W + 2 * pw)), case
        wv = win.float() if xt == "bf16" else win
        if xt == "e4m3":  # the view holds codes: decode them with the scale
            flat = quant.dequantize(quant.Quantized(win.contiguous().reshape(-1), win.shape, "e4m3",
                                                    arg.scale))
            wv = flat.reshape(win.shape)
        wwant, _, _, _ = R.pool_windows(dec, (KH, KW), (sh, sw), (ph, pw), mode)
        got = wv.contiguous().cpu().numpy()
        assert np.array_equal(got.view(np.uint32), np.ascontiguousarray(wwant).view(np.uint32)), case


@pytest.mark.parametrize("seed", SEEDS)
def test_pool_backward_random_shapes_bit_exact(seed):
    """MaxPool2d and GlobalAvgPool2d backward on random maps, windows, strides,
    paddings and padding modes (every third case on a coarse value grid, so
    windows hold ties; 2x2 stride-2 cases on even maps take the tile path),
    bit for bit against the restatements (NaN compared as NaN)."""
    rng = np.random.default_rng(seed + 700)
    for i in range(20):
        N, C = int(rng.integers(1, 4)), int(rng.integers(1, 12))
        if i % 4 == 0:
            H, W = 2 * int(rng.integers(1, 20)), 2 * int(rng.integers(1, 20))
            k, st, pd, mode = (2, 2), (2, 2), (0, 0), "zeros"
        else:
            H, W = int(rng.integers(1, 40)), int(rng.integers(1, 40))
            k = (int(rng.integers(1, min(H, 4) + 1)), int(rng.integers(1, min(W, 4) + 1)))
            st = (int(rng.integers(1, 4)), int(rng.integers(1, 4)))
            mode = str(rng.choice(MODES))
            # reflect pads at most size - 1 (numpy.pad's rule)
            pd = (int(rng.integers(0, min(k[0] // 2, H - 1) + 1)),
                  int(rng.integers(0, min(k[1] // 2, W - 1) + 1)))
        if i % 3 == 0:
            x = rng.choice(np.array([-0.0, 0.0, 0.5, 1.0, 1.0, -2.0], np.float32), (N, C, H, W))
        else:
            x = rng.standard_normal((N, C, H, W)).astype(np.float32)
        OH = (H + 2 * pd[0] - k[0]) // st[0] + 1
        OW = (W + 2 * pd[1] - k[1]) // st[1] + 1
        g = rng.standard_normal((N, C, OH, OW)).astype(np.float32)
        print(f"pool backward seed {seed} case {i}: {(N, C, H, W)} max {k} {st} {pd} {mode}",
              flush=True)
        got = F.max_pool2d_backward(g, x, k, st, pd, mode)
        want = R.max_pool2d_backward(g, x, k, st, pd, mode)
        nan = np.isnan(want)
        assert np.array_equal(np.isnan(got), nan)
        assert np.array_equal(got[~nan].view(np.uint32), want[~nan].view(np.uint32))
        gp = rng.standard_normal((N, C, 1, 1)).astype(np.float32)
        got = F.avg_pool2d_backward(gp, (N, C, H, W))
        want = R.global_avg_pool2d_backward(gp, (N, C, H, W))
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
