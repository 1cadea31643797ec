"""Exact rational arithmetic for pinning float32 results independently of the
oracle: correctly rounded float32 of a Fraction, and fma / products built on it."""
from __future__ import annotations

import struct
from fractions import Fraction

import numpy as np


def f32_round(a: Fraction) -> float:
    """The float32 nearest to a (ties to even), as a Python float."""
    if a == 0:
        return 0.0
    sign = -1.0 if a < 0 else 1.0
    a = abs(a)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, -126)
    q = Fraction(2) ** (e - 23)
    n = a / q
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    v = fl * q
    if v >= Fraction(2) ** 128:
        return sign * float("inf")
    return sign * float(v)


def f32(x) -> Fraction:
    return Fraction(float(np.float32(x)))


def fma32(a, b, c) -> float:
    return f32_round(f32(a) * f32(b) + f32(c))


def mul32(a, b) -> float:
    return f32_round(f32(a) * f32(b))


def bits(x: float) -> int:
    return struct.unpack("<I", struct.pack("<f", np.float32(x)))[0]
