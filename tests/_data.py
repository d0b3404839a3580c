"""Seeded synthetic inputs shared by the tests (numpy only, CPU-reproducible)."""
import numpy as np

from oracle import bf16_round

INT_MAX = np.iinfo(np.int32).max
INT_MIN = np.iinfo(np.int32).min


def labels(n, pattern, b=2, h=3, seed=20261014):
    """The reference's five label patterns (dism_v3/tests/test_hard_summary.py:14-34)."""
    rng = np.random.default_rng(seed)
    q = rng.integers(-3, 4, (b, h, n), dtype=np.int32)
    k = rng.integers(-3, 4, (b, h, n), dtype=np.int32)
    if pattern == "equal":
        q.fill(INT_MAX)
        k[:] = q
    elif pattern == "disjoint":
        q.fill(INT_MIN)
        k.fill(INT_MAX)
    elif pattern == "periodic":
        q[:] = np.arange(n, dtype=np.int32) % 7
        k[:] = (np.arange(n, dtype=np.int32) + 2) % 7
    elif pattern == "boundary":
        q.fill(1)
        k.fill(1)
        for i in (0, 30, 31, 32, 62, 63, 64, 254, 255, 256, 510, 511, 512):
            if i < n:
                q[:, ::2, i] = -100
                k[:, 1::2, i] = 100
    elif pattern == "alphabet256":
        q = rng.integers(0, 256, (b, h, n), dtype=np.int32)
        k = rng.integers(0, 256, (b, h, n), dtype=np.int32)
    elif pattern == "alphabet4":
        q = rng.integers(0, 4, (b, h, n), dtype=np.int32)
        k = rng.integers(0, 4, (b, h, n), dtype=np.int32)
    elif pattern == "collide":  # distinct labels equal modulo 256: prefilter false positives
        q = rng.integers(0, 4, (b, h, n), dtype=np.int32) * 256 + 7
        k = rng.integers(0, 4, (b, h, n), dtype=np.int32) * 256 + 7
    elif pattern != "random":
        raise ValueError(pattern)
    return q, k


def vectors(n, b=2, h=3, r=8, dv=64, seed=417):
    """sq, sk = silu(N(0,1)) * .4 and v = N(0,1), rounded to bf16 (as float32 arrays).
    Mirrors the reference fixture dism_v3/tests/test_hard_forward.py:15-26 with numpy RNG."""
    rng = np.random.default_rng(seed)

    def silu(x):
        return x / (1.0 + np.exp(-x))

    sq = bf16_round(silu(rng.standard_normal((b, n, h, r))) * 0.4)
    sk = bf16_round(silu(rng.standard_normal((b, n, h, r))) * 0.4)
    v = bf16_round(rng.standard_normal((b, n, h, dv)))
    return sq, sk, v


def flags(b, h):
    hard = np.ones((b, h), dtype=bool)
    if b > 1 and h > 1:
        hard[0, 1] = False
        hard[1, 0] = False
    return hard


def taus(h):
    return np.linspace(-0.5, 0.5, h).astype(np.float32)


def copied_spans(q, k, frac=0.10, lo=32, hi=512, seed=20261204):
    """BASELINE configs[3] generator: starting at t=0 and stepping forward, copy spans of length
    U[lo, hi] from an earlier source s0 (s0 + len <= t0) until `frac` of the positions are
    covered: q[:, t0:t0+len] := k[:, s0:s0+len] (all batch rows and heads alike), so queries
    match earlier keys with long suffixes.  q, k: [B, T, H, d] float arrays, modified in place."""
    rng = np.random.default_rng(seed)
    T = q.shape[1]
    covered, t0 = 0, 0
    while covered < frac * T:
        ln = int(rng.integers(lo, hi + 1))
        t0 = int(rng.integers(t0 + ln, min(T - ln, t0 + 4 * hi) + 1)) if t0 + ln <= T - ln else T
        if t0 + ln > T:
            break
        s0 = int(rng.integers(0, t0 - ln + 1))
        q[:, t0:t0 + ln] = k[:, s0:s0 + ln]
        covered += ln
        t0 += ln
    return covered
