"""Activation rows that pin the int8 activation quantizer's rounding rules.

The reference quantizes with `scale = amax / 127` and
`q = clamp(nearbyint(a * (1.0f / scale)), -128, 127)` in fp32
(src/backends/amd_xdna/amd_xdna.cpp:598-603, 633-639, 762-766).  Two
plausible mistakes give different codes only on special inputs:

* rounding half away from zero instead of nearbyint's half-to-even: rows
  with amax 127 (scale exactly 1) holding +-0.5, +-1.5, +-2.5;
* dividing by the scale instead of multiplying by its fp32 reciprocal: rows
  where fl(a / s) and fl(a * fl(1 / s)) fall on different sides of a
  half-integer, found by a seeded search.

`expected_codes` computes the reference's codes with exact rational
arithmetic and an explicit round-to-nearest-even to fp32 after every
operation (IEEE 754 binary32), independent of numpy's and C's float code.
"""
from fractions import Fraction

import numpy as np


def f32(x: Fraction) -> Fraction:
    """x rounded to the nearest fp32 value, ties to even (normal range)."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    m = abs(x)
    e = m.numerator.bit_length() - m.denominator.bit_length()
    # scale so that 2^23 <= m / 2^e < 2^24
    e -= 23
    while m / Fraction(2) ** e >= 2 ** 24:
        e += 1
    while m / Fraction(2) ** e < 2 ** 23:
        e -= 1
    v = m / Fraction(2) ** e
    r = round(v)  # Python rounds a Fraction half to even
    return sign * r * Fraction(2) ** e


def rint_half_even(x: Fraction) -> int:
    return round(x)


def expected_codes(row: np.ndarray):
    """(codes, scale) of one row (or block) under the reference's rule."""
    vals = [Fraction(float(v)) for v in row]
    amax = max(abs(v) for v in vals)
    s = f32(amax / 127) if amax > 0 else Fraction(1)
    inv = f32(1 / s)
    q = [max(-128, min(127, rint_half_even(f32(v * inv)))) for v in vals]
    return np.array(q, np.int8), np.float32(float(s))


def tie_row(K: int) -> np.ndarray:
    """amax 127 (scale 1.0) with exact half-integers: half-to-even gives
    0, 2, 2, 4 where half-away gives 1, 2, 3, 5."""
    r = np.zeros(K, np.float32)
    vals = [127.0, 0.5, -0.5, 1.5, -1.5, 2.5, -2.5, 3.5, -3.5, 4.5, 126.5, -126.5, -127.0]
    r[: len(vals)] = vals
    return r


def reciprocal_rows(n_rows: int, K: int, seed: int) -> np.ndarray:
    """Rows whose values sit next to a half-integer multiple of the scale,
    kept only when the divide variant rounds differently from the
    reciprocal-multiply rule in at least a quarter of the positions."""
    rng = np.random.default_rng(seed)
    rows = []
    while len(rows) < n_rows:
        amax = np.float32(rng.uniform(0.5, 8.0))
        s = np.float32(amax / np.float32(127.0))
        inv = np.float32(np.float32(1.0) / s)
        h = rng.integers(-126, 126, size=8 * K).astype(np.float32) + np.float32(0.5)
        a = (h * s).astype(np.float32)
        # nudge each candidate by up to 3 ulps either way
        steps = rng.integers(-3, 4, size=a.size)
        a = np.array([np.nextafter(x, np.float32(np.sign(d)) * np.float32(np.inf)) if d else x
                      for x, d in zip(a, steps)], np.float32)
        for _ in range(2):
            more = rng.integers(-1, 2, size=a.size)
            a = np.array([np.nextafter(x, np.float32(np.sign(d)) * np.float32(np.inf)) if d else x
                          for x, d in zip(a, more)], np.float32)
        a = a[np.abs(a) < amax]
        q_mul = np.rint((a * inv).astype(np.float32))
        q_div = np.rint((a / s).astype(np.float32))
        diff = a[q_mul != q_div]
        same = a[q_mul == q_div]
        if diff.size < K // 4:
            continue
        take = min(diff.size, K // 2)
        row = np.concatenate([[amax], diff[:take], same[: K - 1 - take]]).astype(np.float32)
        if row.size < K:
            continue
        rows.append(row[:K])
    return np.stack(rows)


def half_away(x: np.ndarray) -> np.ndarray:
    return np.sign(x) * np.floor(np.abs(x) + 0.5)


def variant_codes(A: np.ndarray, divide: bool, away: bool, block: int = 0) -> np.ndarray:
    """Codes under a deliberately wrong rule (numpy fp32), per row or per
    block of `block` values."""
    A = np.asarray(A, np.float32)
    M, K = A.shape
    g = A.reshape(M, -1, block) if block else A.reshape(M, 1, K)
    amax = np.abs(g).max(axis=2, keepdims=True)
    s = np.where(amax > 0, (amax / np.float32(127.0)).astype(np.float32), np.float32(1.0)).astype(np.float32)
    if divide:
        v = (g / s).astype(np.float32)
    else:
        v = (g * (np.float32(1.0) / s).astype(np.float32)).astype(np.float32)
    r = half_away(v) if away else np.rint(v)
    return np.clip(r, -128, 127).astype(np.int8).reshape(M, K)
