"""Writes tests/golden/*.npz: inputs and expected outputs from sources that
are independent of the build's own oracle and kernels.

  - fp16: numpy's float32 -> float16 astype (numpy is NovaNN's numeric
    backend, so this is the conversion a NovaNN user gets);
  - bf16: torch CPU ``.to(torch.bfloat16)`` on non-NaN inputs;
  - E4M3 / E5M2: torch CPU float8_e4m3fn / float8_e5m2 where torch's
    non-saturating cast agrees with the saturating rule (|x| <= 464 for
    E4M3, |x| < 61440 for E5M2, and NaN); beyond that the saturated code
    +-0x7E / +-0x7B is written directly (the rule itself);
  - E2M1: nearest value of the MX spec's table {0, .5, 1, 1.5, 2, 3, 4, 6}
    by a vectorised numpy search, ties to the even code, |x| > 6 -> 6;
  - decode tables: torch float8 -> float32, the E2M1 spec table;
  - small Linear / Conv2d cases: fp64 numpy / torch CPU conv2d on the
    decoded weights.
The reference (NovaNN) has no golden vectors for this path.
Run:  python tests/golden/make_golden.py   (CPU only, a few seconds).
"""
from __future__ import annotations

import os

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
E2M1_VALUES = np.array([0.0, 0.5, 1.0, 1.5, 2.0, 3.0, 4.0, 6.0])


def u32(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def crafted_inputs(rng: np.random.RandomState) -> np.ndarray:
    vals = []
    # specials
    vals += [0x00000000, 0x80000000, 0x7F800000, 0xFF800000, 0x7FC00000, 0xFFC00000,
             0x7F800001, 0xFF800001, 0x7FBFFFFF, 0x7FFFFFFF, 0xFFFFFFFF, 0x7FC00001,
             0x7F802000, 0x7F801FFF, 0x00000001, 0x80000001, 0x007FFFFF, 0x00800000,
             0x7F7FFFFF, 0xFF7FFFFF]
    f = []
    # boundaries of every target format, with fp32 neighbours
    for v in [448.0, 464.0, 480.0, 57344.0, 61440.0, 65504.0, 65520.0, 6.0, 5.0, 7.0,
              2.0 ** -6, 2.0 ** -9, 2.0 ** -10, 1.5 * 2.0 ** -9, 2.0 ** -14, 2.0 ** -16,
              2.0 ** -17, 2.0 ** -24, 2.0 ** -25, 1.5 * 2.0 ** -24, 3.3895313892515355e38,
              0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 1.0, 1e-30, 1e30]:
        f += [v, -v]
    base = u32(f)
    for d in (-2, -1, 0, 1, 2):
        vals += list((base.astype(np.int64) + d).astype(np.uint32))
    # midpoints between consecutive codes (ties) of E4M3 / E5M2 / E2M1 / fp16
    e4 = torch.arange(0, 0x7F, dtype=torch.int32).to(torch.uint8).view(
        torch.float8_e4m3fn).float().numpy().astype(np.float64)
    e5 = torch.arange(0, 0x7C, dtype=torch.int32).to(torch.uint8).view(
        torch.float8_e5m2).float().numpy().astype(np.float64)
    h = np.arange(0, 0x7C00, 97, dtype=np.uint16).view(np.float16).astype(np.float64)
    for table in (e4, e5, E2M1_VALUES, np.sort(h)):
        mids = (table[:-1] + table[1:]) / 2
        m32 = u32(mids.astype(np.float32))
        for d in (-1, 0, 1):
            vals += list((m32.astype(np.int64) + d).astype(np.uint32))
            vals += list(((m32.astype(np.int64) + d).astype(np.uint32)) | 0x80000000)
    # random normal, log-uniform and raw bit patterns
    vals += list(u32(rng.standard_normal(1024).astype(np.float32)))
    mag = np.exp2(rng.uniform(-30, 30, 1024)) * np.where(rng.rand(1024) < 0.5, -1, 1)
    vals += list(u32(mag.astype(np.float32)))
    vals += list(rng.randint(0, 2 ** 32, size=1024, dtype=np.uint64).astype(np.uint32))
    return np.unique(np.array(vals, dtype=np.uint32))


def f16_expected(bits):
    return bits.view(np.float32).astype(np.float16).view(np.uint16)


def bf16_expected(bits):
    out = torch.from_numpy(bits.view(np.float32).copy()).to(torch.bfloat16).view(
        torch.int16).numpy().view(np.uint16).copy()
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    out[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint16)  # D3 NaN rule
    return out


def fp8_expected(bits, kind):
    tdt, lim, maxc = ((torch.float8_e4m3fn, 464.0, 0x7E) if kind == "e4m3"
                      else (torch.float8_e5m2, 61440.0, 0x7B))
    x = bits.view(np.float32)
    out = torch.from_numpy(x.copy()).to(tdt).view(torch.uint8).numpy().copy()
    big = ~np.isnan(x) & (np.abs(x.astype(np.float64)) >= lim)
    if kind == "e4m3":
        big = ~np.isnan(x) & (np.abs(x.astype(np.float64)) > lim)
    sign = ((bits >> 24) & 0x80).astype(np.uint8)
    out[big] = sign[big] | maxc
    return out


def e2m1_expected(bits):
    x = bits.view(np.float32).astype(np.float64)
    a = np.abs(x)
    d = np.abs(a[:, None] - E2M1_VALUES[None, :])
    best = d.min(axis=1, keepdims=True)
    cand = d == best
    # ties -> even code (codes 0..7 are the table indices)
    even = cand & (np.arange(8)[None, :] % 2 == 0)
    code = np.where(even.any(axis=1), even.argmax(axis=1), cand.argmax(axis=1))
    code = np.where(a > 6.0, 7, code)
    code = np.where(np.isinf(x), 7, code)
    sign = (bits >> 31).astype(np.int64) << 3
    out = (code | sign).astype(np.uint8)
    out[np.isnan(x)] = 0
    return out


def main():
    rng = np.random.RandomState(20251201)
    bits = crafted_inputs(rng)
    dec_e4m3 = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(
        torch.float8_e4m3fn).float().numpy().view(np.uint32).copy()
    dec_e5m2 = torch.arange(256, dtype=torch.int32).to(torch.uint8).view(
        torch.float8_e5m2).float().numpy().view(np.uint32).copy()
    dec_e2m1 = u32(np.concatenate([E2M1_VALUES, -E2M1_VALUES]).astype(np.float32))
    np.savez_compressed(
        os.path.join(HERE, "cast_vectors.npz"),
        inputs=bits, f16=f16_expected(bits), bf16=bf16_expected(bits),
        e4m3=fp8_expected(bits, "e4m3"), e5m2=fp8_expected(bits, "e5m2"),
        e2m1=e2m1_expected(bits), dec_e4m3=dec_e4m3, dec_e5m2=dec_e5m2, dec_e2m1=dec_e2m1)

    # small products on already-decoded weights (fp64 closed forms)
    rng = np.random.RandomState(7)
    x = rng.standard_normal((8, 64)).astype(np.float32)
    codes = rng.randint(0, 256, size=(24, 64)).astype(np.uint8)
    codes[(codes & 0x7F) == 0x7F] = 0x3C  # no NaN weights
    s = np.float32(0.0123)
    wdec = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    w = (wdec * s).astype(np.float32)
    b = rng.standard_normal(24).astype(np.float32)
    y = (x.astype(np.float64) @ w.astype(np.float64).T + b.astype(np.float64)).astype(
        np.float32)
    cx = rng.uniform(0, 1, (2, 3, 9, 7)).astype(np.float32)
    ccodes = rng.randint(0, 256, size=(5, 3, 3, 3)).astype(np.uint8)  # E2M1 byte pairs
    nib = np.stack([ccodes & 0xF, ccodes >> 4], axis=-1).reshape(-1)[: 5 * 3 * 3 * 3]
    cs = np.float32(0.37)
    table = np.concatenate([E2M1_VALUES, -E2M1_VALUES]).astype(np.float32)
    cw = (table[nib] * cs).astype(np.float32).reshape(5, 3, 3, 3)
    cb = rng.standard_normal(5).astype(np.float32)
    padded = np.concatenate([nib, np.zeros(len(nib) % 2, dtype=nib.dtype)])
    packed = (padded[0::2] | (padded[1::2] << 4)).astype(np.uint8)
    conv = {}
    for mode, tmode in [("zeros", "constant"), ("reflect", "reflect"),
                        ("replicate", "replicate"), ("circular", "circular")]:
        xt = torch.from_numpy(cx).double()
        xt = torch.nn.functional.pad(xt, (1, 1, 2, 2), mode=tmode)
        conv[mode] = torch.nn.functional.conv2d(
            xt, torch.from_numpy(cw).double(), torch.from_numpy(cb).double(),
            stride=(2, 1)).float().numpy()
    np.savez_compressed(
        os.path.join(HERE, "product_vectors.npz"),
        lin_x=x, lin_codes=codes, lin_scale=np.array([s]), lin_bias=b, lin_y=y,
        conv_x=cx, conv_packed=packed, conv_scale=np.array([cs]), conv_bias=cb,
        **{f"conv_y_{k}": v for k, v in conv.items()})
    print("inputs:", bits.size)


if __name__ == "__main__":
    with np.errstate(all="ignore"):
        main()
