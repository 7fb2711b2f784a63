"""Exact IEEE-754 rounding written from the standard, independent of numpy.

Used to pin the oracle: binary16 comes from Python's ``struct`` packer (format
``'e'``, round-half-to-even), binary32 from exact rationals rounded by hand.
Neither shares code with numpy's casts, so a slip in the oracle's numpy
expressions (wrong operand order, dropped rounding, wrong dtype promotion)
shows up as a mismatch here.
"""

from __future__ import annotations

import math
import struct
from fractions import Fraction

F32_MIN_EXP = -126
F32_MANT = 23
F32_MAX_EXP = 127


def f16_bits(x: float) -> int:
    """binary16 bits of the double ``x`` rounded to nearest-even (inf on overflow)."""
    if math.isnan(x):
        return 0x7E00
    try:
        return struct.unpack("<H", struct.pack("<e", x))[0]
    except OverflowError:
        return 0x7C00 if x > 0 else 0xFC00


def f16_value(bits: int) -> float:
    return struct.unpack("<e", struct.pack("<H", bits & 0xFFFF))[0]


def _round_half_even_int(fr: Fraction) -> int:
    return round(fr)  # Fraction.__round__ rounds half to even


def round_f32(x: Fraction) -> Fraction:
    """Nearest binary32 value to the rational ``x`` (ties to even); returns a
    Fraction, or +-inf as a float when it overflows."""
    if x == 0:
        return Fraction(0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    e = max(e, F32_MIN_EXP)
    quantum = Fraction(2) ** (e - F32_MANT)
    m = _round_half_even_int(a / quantum)
    r = m * quantum
    if r >= Fraction(2) ** (F32_MAX_EXP + 1):
        return sign * math.inf
    return sign * r


def quantize_group_exact(ws, fp16_scale_first: bool):
    """One group quantized with exact arithmetic.

    ``ws`` are the group's values as binary32-representable floats.
    ``fp16_scale_first=False`` is the float32-scale quantizer, ``True`` the one
    that rounds the scale to binary16 before dividing.  Returns (q list, scale
    as binary16 bits).
    """
    alpha = max(abs(Fraction(w)) for w in ws)
    if alpha == 0:
        s = Fraction(1)
    else:
        s = round_f32(alpha / 7)
    s16_bits = f16_bits(float(s))
    divisor = Fraction(f16_value(s16_bits)) if fp16_scale_first else s
    qs = []
    for w in ws:
        quo = round_f32(Fraction(w) / divisor)
        qs.append(max(-8, min(7, _round_half_even_int(quo))))
    return qs, s16_bits
