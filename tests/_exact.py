"""Exact rational arithmetic used to pin the oracle independently of numpy's
floating-point behaviour (test helper, not product code)."""

from fractions import Fraction
import math
import struct


def round_to_format(x: Fraction, mant_bits: int, emin: int, emax: int) -> Fraction:
    """Round a rational to the nearest value of a binary float format with
    `mant_bits` fraction bits, minimum normal exponent emin and maximum
    exponent emax, ties to even; overflow returns +-inf as float('inf')."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    # fix floor(log2) exactly
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - mant_bits)
    q = a / ulp
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    v = n * ulp
    if v >= Fraction(2) ** (emax + 1):
        return sign * Fraction(10) ** 400  # sentinel for overflow
    return sign * v


def to_bf16(x: Fraction) -> Fraction:
    return round_to_format(x, 7, -126, 127)


def to_fp16(x: Fraction) -> Fraction:
    return round_to_format(x, 10, -14, 15)


def to_fp32(x: Fraction) -> Fraction:
    return round_to_format(x, 23, -126, 127)


def fp16_bits(v: Fraction) -> int:
    if abs(v) >= Fraction(10) ** 300:
        return 0x7C00 | (0x8000 if v < 0 else 0)
    return struct.unpack("<H", struct.pack("<e", float(v)))[0]


def rint_half_even(x: Fraction) -> int:
    n = math.floor(x)
    r = x - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return n
