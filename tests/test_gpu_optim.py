"""AdamW on the GPU (through the C ABI) vs the float32 restatement of
novann's AdamW.step (oracle/optim_ref.py, adamw.py:41-65): bit-exact, since
both evaluate the same float32 operations; re-quantization bit-exact against
the oracle's amax-scaled cast of the updated weights."""
import ctypes

import numpy as np
import pytest
import torch

import oracle as O
from oracle import optim_ref as OR
from novann_amd import _lib
from novann_amd.module import Linear, Parameters, QuantizedParameters
from novann_amd.optim import AdamW
from tests.gpu_util import to_host

pytestmark = pytest.mark.gpu
QT = {"e4m3": O.E4M3, "e5m2": O.E5M2, "e2m1": O.E2M1}


def stream():
    return torch.cuda.current_stream().cuda_stream


def dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


@pytest.mark.parametrize("n", [1, 3, 4, 1000, 4097, (1 << 20) + 3])
@pytest.mark.parametrize("lr,wd,decay", [(1e-3, 0.0, 1), (1e-3, 1e-2, 1), (3e-2, 0.1, 0),
                                         (1e-4, 0.5, 1)])
def test_adamw_step_bit_exact(n, lr, wd, decay):
    print(f"adamw n={n} lr={lr} wd={wd} decay={decay}", flush=True)
    rng = np.random.default_rng(n + int(lr * 1e5))
    w = rng.standard_normal(n).astype(np.float32)
    m, v = np.zeros_like(w), np.zeros_like(w)
    wd_, md, vd = dev(w), dev(m), dev(v)
    amax = torch.zeros(1, device="cuda")
    for t in range(1, 6):
        g = (rng.standard_normal(n) * 10.0 ** rng.integers(-3, 2)).astype(np.float32)
        g[: min(n, 2)] = [0.0, -0.0][: min(n, 2)]
        w, m, v = OR.adamw_step(w, g, m, v, t, lr, 0.9, 0.999, 1e-8, wd, bool(decay))
        hp = _lib.AdamW(lr, 0.9, 0.999, 1e-8, wd, t, decay)
        _lib.check(_lib.load().novaq_adamw_step(wd_.data_ptr(), dev(g).data_ptr(), md.data_ptr(),
                                                vd.data_ptr(), n, ctypes.byref(hp),
                                                amax.data_ptr(), stream()), "adamw")
        torch.cuda.synchronize()
        for name, got, want in (("w", wd_, w), ("m", md, m), ("v", vd, v)):
            gb = got.cpu().numpy()
            assert np.array_equal(gb.view(np.uint32), want.view(np.uint32)), \
                f"step {t} {name}: {np.count_nonzero(gb != want)} mismatches"
        assert float(amax.cpu()[0]) == float(np.abs(w).max())


@pytest.mark.parametrize("qt", ["e4m3", "e5m2", "e2m1"])
@pytest.mark.parametrize("n", [6, 4096 * 64 + 2])
def test_adamw_requantize_bit_exact(qt, n):
    rng = np.random.default_rng(n)
    w = rng.standard_normal(n).astype(np.float32) * 0.05
    g = rng.standard_normal(n).astype(np.float32)
    m = rng.standard_normal(n).astype(np.float32) * 0.01
    v = np.abs(rng.standard_normal(n).astype(np.float32)) * 1e-4
    w1, m1, v1 = OR.adamw_step(w, g, m, v, 7, 1e-3, 0.9, 0.999, 1e-8, 0.01, True)
    wd_, md, vd = dev(w), dev(m), dev(v)
    codes = torch.empty((n + 1) // 2 if qt == "e2m1" else n, dtype=torch.uint8, device="cuda")
    st = torch.empty(2, device="cuda")
    hp = _lib.AdamW(1e-3, 0.9, 0.999, 1e-8, 0.01, 7, 1)
    _lib.check(_lib.load().novaq_adamw_requantize(
        wd_.data_ptr(), dev(g).data_ptr(), md.data_ptr(), vd.data_ptr(), n, ctypes.byref(hp),
        codes.data_ptr(), _lib.DTYPES[qt], st.data_ptr(), stream()), "requantize")
    torch.cuda.synchronize()
    assert np.array_equal(wd_.cpu().numpy().view(np.uint32), w1.view(np.uint32))
    amax = O.amax(w1)
    s = O.scale_from_amax(amax, QT[qt])
    assert float(st.cpu()[0]) == float(amax) and float(st.cpu()[1]) == float(s)
    assert np.array_equal(to_host(codes), O.cast(w1, O.F32, QT[qt], scale=s))


def test_optimizer_class_like_reference():
    """AdamW(params).step() over a quantized Linear (master + re-quantized
    codes) and a numpy bias: the bias array and the master weights follow the
    oracle bit for bit given the same gradients; BatchNorm-named parameters
    are not decayed; zero_grad clears."""
    rng = np.random.default_rng(5)
    layer = Linear(64, 32, bias=True, weight_dtype="e4m3")
    gamma = Parameters(np.ones((1, 32, 1, 1), np.float32))
    gamma.name = "gamma"
    opt = AdamW(layer.parameters() + [gamma], lr=1e-2, weight_decay=0.1)
    w = layer.weight.master.cpu().numpy().copy()
    b = layer.bias.data.copy()
    gm = gamma.data.copy()
    states = {k: (np.zeros_like(a), np.zeros_like(a)) for k, a in (("w", w), ("b", b), ("g", gm))}
    for t in range(1, 4):
        gw = rng.standard_normal(w.shape).astype(np.float32)
        gb = rng.standard_normal(b.shape).astype(np.float32)
        gg = rng.standard_normal(gm.shape).astype(np.float32)
        layer.weight.grad = torch.from_numpy(gw).cuda()
        layer.bias.grad = gb
        gamma.grad = gg
        opt.step()
        w, *states["w"] = OR.adamw_step(w, gw, *states["w"], t, 1e-2, wd=0.1)
        b, *states["b"] = OR.adamw_step(b, gb, *states["b"], t, 1e-2, wd=0.1)
        gm, *states["g"] = OR.adamw_step(gm, gg, *states["g"], t, 1e-2, wd=0.1, decay=False)
    torch.cuda.synchronize()
    assert np.array_equal(layer.weight.master.cpu().numpy(), w)
    assert np.array_equal(layer.bias.data, b) and isinstance(layer.bias.data, np.ndarray)
    assert np.array_equal(gamma.data, gm)
    s = O.scale_from_amax(O.amax(w.reshape(-1)), O.E4M3)
    assert float(layer.weight.scale.cpu()[0]) == float(s)
    assert np.array_equal(to_host(layer.weight.codes.view(torch.uint8)),
                          O.cast(w.reshape(-1), O.F32, O.E4M3, scale=s))
    opt.zero_grad()
    assert not layer.bias.grad.any() and not gamma.grad.any()


def test_training_steps_reduce_the_loss():
    """A quantized Linear trained on a linear regression target through the
    GPU forward, backward and AdamW with re-quantization: the loss falls."""
    rng = np.random.default_rng(6)
    layer = Linear(128, 64, bias=True, weight_dtype="e4m3")
    target = rng.standard_normal((64, 128)).astype(np.float32) * 0.1
    opt = AdamW(layer.parameters(), lr=1e-2)
    losses = []
    for _ in range(30):
        x = rng.standard_normal((256, 128)).astype(np.float32)
        y = layer(x)
        err = y - x @ target.T
        losses.append(float((err ** 2).mean()))
        layer.backward(2.0 * err / err.size)
        opt.step()
        opt.zero_grad()
    assert losses[-1] < 0.5 * losses[0], losses


@pytest.mark.parametrize("gdt", [np.float32, np.float64])
@pytest.mark.parametrize("n", [1, 37, 4096 + 5])
def test_float64_entry_point_bit_exact(gdt, n):
    """novaq_adamw_step_f64 against the oracle's float64 statements (numpy's
    promotion of a float32 gradient included), 4 steps, with and without
    decay."""
    print(f"adamw f64 n={n} grad {np.dtype(gdt).name}", flush=True)
    rng = np.random.default_rng(n)
    lib = _lib.load()
    for decay in (1, 0):
        w = rng.standard_normal(n)
        m, v = np.zeros(n), np.zeros(n)
        wd_, md, vd = (torch.from_numpy(a.copy()).cuda() for a in (w, m, v))
        for t in range(1, 5):
            g = rng.standard_normal(n).astype(gdt)
            gd = torch.from_numpy(g).cuda()
            hp = _lib.AdamW(3e-2, 0.9, 0.999, 1e-8, 0.1, t, decay)
            assert lib.novaq_adamw_step_f64(wd_.data_ptr(), gd.data_ptr(), int(gdt == np.float32),
                                            md.data_ptr(), vd.data_ptr(), n, ctypes.byref(hp),
                                            stream()) == _lib.OK
            w, m, v = OR.adamw_step_f64(w, g, m, v, t, 3e-2, wd=0.1, decay=bool(decay))
        torch.cuda.synchronize()
        for got, want in ((wd_, w), (md, m), (vd, v)):
            assert np.array_equal(got.cpu().numpy().view(np.uint64), want.view(np.uint64))


def test_batchnorm_parameters_as_constructed():
    """BatchNorm2d's gamma / beta are float64 (as in the reference) and step in
    float64 with float64 moments; a float32 gradient is promoted as numpy
    does.  Changing .data between steps counts, as with the reference."""
    from novann_amd.module import BatchNorm2d
    bn = BatchNorm2d(16)
    assert bn.gamma.data.dtype == np.float64
    opt = AdamW(bn.parameters(), lr=1e-2, weight_decay=0.1)
    rng = np.random.default_rng(8)
    ref = {k: [p.data.copy(), np.zeros_like(p.data), np.zeros_like(p.data)]
           for k, p in (("g", bn.gamma), ("b", bn.beta))}
    for t in range(1, 4):
        gg = rng.standard_normal(bn.gamma.data.shape).astype(np.float32)
        gb = rng.standard_normal(bn.beta.data.shape)
        bn.gamma.grad, bn.beta.grad = gg, gb
        opt.step()
        for k, g in (("g", gg), ("b", gb)):
            ref[k] = list(OR.adamw_step_f64(*ref[k][:1], g, *ref[k][1:], t, 1e-2, wd=0.1,
                                            decay=False))
        if t == 2:  # the caller rewrites a parameter between steps
            bn.beta.data[...] = 0.25
            ref["b"][0] = np.full_like(ref["b"][0], 0.25)
    assert bn.gamma.data.dtype == bn.beta.data.dtype == np.float64
    assert np.array_equal(bn.gamma.data.view(np.uint64), ref["g"][0].view(np.uint64))
    assert np.array_equal(bn.beta.data.view(np.uint64), ref["b"][0].view(np.uint64))
