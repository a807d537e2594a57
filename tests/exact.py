"""Exact reference arithmetic for pinning the oracle's folds (pure Python).

fma32(a, b, c) rounds the exact rational a*b + c to the nearest binary32
(ties to even), independently of any C library or FPU: it is built from
Fraction arithmetic and integer rounding only.  Folds written with it are the
textbook definition of the reference's single-expression C fold after
contraction (one rounding per block).
"""
from __future__ import annotations

from fractions import Fraction

import numpy as np


def round_f32(x: Fraction) -> np.float32:
    """Nearest binary32 to the exact rational x, ties to even (no overflow handling
    beyond returning +-inf)."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    a = -x if x < 0 else x
    # find e with 2^e <= a < 2^(e+1)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    elif Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)  # subnormal range shares the 2^-149 quantum
    quantum = Fraction(2) ** (e - 23)
    q, r = divmod(a, quantum)  # q integer, 0 <= r < quantum
    q = int(q)
    half = quantum / 2
    if r > half or (r == half and q % 2 == 1):
        q += 1
    val = Fraction(q) * quantum
    if val >= Fraction(2) ** 128:
        return np.float32(sign * np.inf)
    # q * 2^(e-23) is exactly representable; build it through float64 (exact).
    return np.float32(sign * float(val))


def fma32(a, b, c) -> np.float32:
    return round_f32(Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c)))


def mul32(a, b) -> np.float32:
    return round_f32(Fraction(float(a)) * Fraction(float(b)))
