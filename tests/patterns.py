"""Input generators shared by the CPU and GPU tests (seeded, numpy only)."""
from __future__ import annotations

import numpy as np

# mantissa bits of each narrowing format (f32 -> dtype), by dtype code
MBITS = {1: 10, 2: 7, 3: 3, 4: 2, 5: 1}


def structured_f32(mbits: int) -> np.ndarray:
    """Every sign and fp32 exponent, with the top mbits+2 mantissa bits
    exhaustive (every kept mantissa, the round bit and one more) and the low
    bits set to the patterns that decide rounding: 0, 1, a middle bit, all
    ones.  Covers each RNE decision (below / at / above the tie, odd and even
    kept mantissa) at every exponent, plus Inf / NaN payloads."""
    top = mbits + 2
    low_bits = 23 - top
    lows = np.unique(np.array([0, 1, 1 << max(low_bits - 1, 0), (1 << low_bits) - 1],
                              dtype=np.uint32))
    sign = np.array([0, 1], dtype=np.uint32)[:, None, None, None] << 31
    exp = np.arange(256, dtype=np.uint32)[None, :, None, None] << 23
    man = np.arange(1 << top, dtype=np.uint32)[None, None, :, None] << low_bits
    low = lows[None, None, None, :]
    return (sign | exp | man | low).reshape(-1)


def random_f32_bits(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    return rng.integers(0, 2 ** 32, size=n, dtype=np.uint64).astype(np.uint32)


def config1_tensor(seed: int = 1, shape=(4096, 4096)) -> np.ndarray:
    """BASELINE config [1]: 90% N(0,1), 10% specials (+-0, +-Inf, NaNs,
    subnormal-E4M3 neighbourhood k*2^-9 +- ulp and ties, and an overflow band
    448 .. fp32 max including 464 and 480)."""
    rng = np.random.default_rng(seed)
    n = int(np.prod(shape))
    x = rng.standard_normal(n, dtype=np.float32)
    special = rng.random(n) < 0.10
    k = int(special.sum())
    kind = rng.integers(0, 6, size=k)
    vals = np.empty(k, dtype=np.float32)
    neg = rng.random(k) < 0.5
    # 0: signed zeros
    vals[kind == 0] = 0.0
    # 1: infinities
    vals[kind == 1] = np.inf
    # 2: NaNs with random payloads (quiet and signalling)
    m2 = kind == 2
    payload = rng.integers(1, 1 << 23, size=int(m2.sum()), dtype=np.uint32)
    vals[m2] = (np.uint32(0x7F800000) | payload).view(np.float32)
    # 3: E4M3 subnormal neighbourhood: k*2^-9 and (k+1/2)*2^-9, +- 1 fp32 ulp
    m3 = kind == 3
    c = rng.integers(0, 16, size=int(m3.sum())).astype(np.float32)
    half = (rng.random(int(m3.sum())) < 0.5).astype(np.float32) * 0.5
    base = ((c + half) * np.float32(2.0 ** -9)).astype(np.float32)
    nudge = rng.integers(-1, 2, size=base.size).astype(np.int64)
    vals[m3] = (base.view(np.uint32).astype(np.int64) + nudge).astype(np.uint32).view(
        np.float32)
    # 4: overflow band 448 .. 3.4e38 (log-uniform), with 464 / 480 exactly
    m4 = kind == 4
    band = np.exp2(rng.uniform(np.log2(448.0), 127.9, size=int(m4.sum()))).astype(np.float32)
    pick = rng.random(band.size)
    band[pick < 0.1] = 464.0
    band[(pick >= 0.1) & (pick < 0.2)] = 480.0
    vals[m4] = band
    # 5: fp32 subnormals and tiny values
    m5 = kind == 5
    vals[m5] = rng.integers(1, 1 << 23, size=int(m5.sum()), dtype=np.uint32).view(np.float32)
    # the sign goes in as a bit: a float multiply would quiet the signalling
    # NaNs and, on x86, keep a NaN operand's own sign
    bits = vals.view(np.uint32) | np.where(neg, np.uint32(0x80000000), np.uint32(0))
    x[special] = bits.astype(np.uint32).view(np.float32)
    return x.reshape(shape)


def config2_tensor(n: int, seed: int = 2) -> np.ndarray:
    """BASELINE config [2]: random sign, |x| log-uniform in [2^-20, 2^20]."""
    rng = np.random.default_rng(seed)
    mag = np.exp2(rng.uniform(-20.0, 20.0, size=n)).astype(np.float32)
    sgn = np.where(rng.random(n) < 0.5, -1.0, 1.0).astype(np.float32)
    return mag * sgn


def config3_tensor(n: int, seed: int = 3) -> np.ndarray:
    """BASELINE config [3]: N(0,1) divided by amax/6 (so the tensor spans the
    E2M1 range), with 5% of the entries replaced by exact E2M1 RNE ties."""
    rng = np.random.default_rng(seed)
    x = rng.standard_normal(n, dtype=np.float32)
    x = (x / (np.abs(x).max() / np.float32(6.0))).astype(np.float32)
    ties = np.array([0.25, 0.75, 1.25, 1.75, 2.5, 3.5, 5.0], dtype=np.float32)
    m = rng.random(n) < 0.05
    x[m] = ties[rng.integers(0, ties.size, size=int(m.sum()))] * np.where(
        rng.random(int(m.sum())) < 0.5, -1, 1).astype(np.float32)
    return x
