"""Exact-rational emulation of IEEE binary32 round-to-nearest-even.

Used to pin the oracle independently of numpy and of the C compiler: every
operation of the reference quantizer (my_int4/rtn_int4.py:22-55) and of the
fused transform's sequential matvec (tests/test_sw2.py:12-24) is evaluated
exactly with Fractions and then rounded by ``rn`` -- a separate implementation
of the same specification, not a retyped formula.
"""
from __future__ import annotations

import math
import struct
from fractions import Fraction

EMIN = -126          # binary32 minimum normal exponent
P = 24               # binary32 significand bits


def f32(x: float) -> Fraction:
    """Fraction equal to the binary32 value nearest to Python float x."""
    return Fraction(struct.unpack("<f", struct.pack("<f", x))[0])


def rn(q: Fraction, p: int = P, emin: int = EMIN) -> Fraction:
    """Round q to the nearest binary float with p significand bits, ties to even."""
    if q == 0:
        return Fraction(0)
    sign = -1 if q < 0 else 1
    a = abs(q)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    # now 2^e <= a < 2^(e+1)
    e = max(e, emin)
    ulp = Fraction(2) ** (e - (p - 1))
    n = a / ulp
    fl = n.numerator // n.denominator
    rem = n - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return sign * fl * ulp


def rn_sqrt(v: Fraction) -> Fraction:
    """Correctly rounded binary32 square root of a non-negative binary32 value."""
    if v == 0:
        return Fraction(0)
    k = 200
    scaled = v * (Fraction(4) ** k)
    n = scaled.numerator // scaled.denominator
    s = math.isqrt(n)
    if s * s == scaled:            # exact square (scaled is then an integer)
        return rn(Fraction(s, 2 ** k))
    # sqrt(v) lies strictly inside (s, s+1) / 2^k; a binary32 midpoint cannot
    # equal sqrt(v), so the interval's midpoint rounds the same way.
    return rn(Fraction(2 * s + 1, 2 ** (k + 1)))


def rhe(q: Fraction) -> int:
    """Round half to even to an integer."""
    fl = q.numerator // q.denominator
    rem = q - fl
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and fl % 2 == 1):
        fl += 1
    return fl


def quant_group(values) -> tuple[int, list[int]]:
    """(bf16 scale bits, codes) of one 32-value group of binary32 inputs."""
    x = [Fraction(float(v)) for v in values]
    s1 = Fraction(0)
    s2 = Fraction(0)
    for v in x:
        s1 = rn(s1 + v)
        s2 = rn(s2 + rn(v * v))
    mean = rn(s1 / 32)
    var = rn(rn(s2 / 32) - rn(mean * mean))
    if var >= 0:
        scale = rn(rn(rn_sqrt(var) * f32(0.35337862372398376)) + f32(1e-8))
    else:
        scale = Fraction(1)
    sb = rn(scale, p=8)                      # bf16: 8 significand bits, same exponent range
    codes = [max(-7, min(7, rhe(rn(v / sb)))) for v in x]
    bits = struct.unpack("<I", struct.pack("<f", float(sb)))[0] >> 16
    return bits, codes


def transform_block(x, T, order=None, fused=False) -> list[Fraction]:
    """x'_j = sum_i x_i * T[j][i] for one 32-wide block of binary32 values x and
    a 32 x 32 matrix T, with the reference's rounding (tests/test_sw2.py:18-22):
    the accumulator starts at +0 and for i ascending takes RN(acc + RN(x_i *
    T[j][i])).  `order` permutes the i sequence and `fused` rounds x_i*T+acc
    once (an fma) -- both only to show that a check built on this function
    notices a different order or contraction."""
    xs = [Fraction(float(v)) for v in x]
    idx = list(range(32)) if order is None else list(order)
    out = []
    for j in range(32):
        acc = Fraction(0)
        for i in idx:
            prod = xs[i] * Fraction(float(T[j][i]))
            acc = rn(acc + prod) if fused else rn(acc + rn(prod))
        out.append(acc)
    return out
