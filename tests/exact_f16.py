"""Exact-rational restatement of the encoder's scalar rules (test helper).

An independent second implementation used to pin the NumPy oracle: every
value is a ``fractions.Fraction`` and each fp16 / fp32 operation is rounded by
the explicit IEEE round-to-nearest-even routine below, so a slip in the
oracle's dtype handling (an op done in the wrong precision, a missing
rounding, a wrong tie rule) shows up as a mismatch.
"""

from __future__ import annotations

import math
import struct
from fractions import Fraction

import numpy as np

INF = float("inf")


def _round_float(x: Fraction, mant_bits: int, emin: int, emax: int):
    """Round a rational to the binary format with ``mant_bits`` fraction bits,
    min normal exponent ``emin`` and max exponent ``emax`` (RNE).  Returns a
    Python float (exact) or +-inf."""
    if x == 0:
        return 0.0
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, emin)
    q = Fraction(2) ** (e - mant_bits)
    m = a / q
    n = round(m)  # Fraction.__round__ is round-half-even
    val = n * q
    if val >= Fraction(2) ** (emax + 1):
        return sign * INF
    return sign * float(val)


def r16(x) -> float:
    """Round to IEEE binary16."""
    return _round_float(Fraction(x), 10, -14, 15)


def r32(x) -> float:
    """Round to IEEE binary32."""
    return _round_float(Fraction(x), 23, -126, 127)


def sqrt_r16(s: float) -> float:
    """Correctly rounded binary16 sqrt of a non-negative binary16 value."""
    if s == INF:
        return INF
    if s == 0:
        return 0.0
    fs = Fraction(s)
    h = r16(math.sqrt(s))
    # adjust by exact comparison with the neighbouring midpoints
    for _ in range(3):
        hb = np.float16(h).view(np.uint16)
        up = float(np.uint16(hb + 1).view(np.float16))
        dn = float(np.uint16(hb - 1).view(np.float16)) if hb > 0 else 0.0
        if (Fraction(h) + Fraction(up)) ** 2 / 4 < fs:
            h = up
        elif hb > 0 and (Fraction(h) + Fraction(dn)) ** 2 / 4 > fs:
            h = dn
        else:
            break
    return h


def sqrt_r32(s: Fraction) -> float:
    if s == 0:
        return 0.0
    h = r32(math.sqrt(float(s)))
    for _ in range(3):
        b = struct.unpack("<I", struct.pack("<f", h))[0]
        up = struct.unpack("<f", struct.pack("<I", b + 1))[0]
        dn = struct.unpack("<f", struct.pack("<I", b - 1))[0]
        if (Fraction(h) + Fraction(up)) ** 2 / 4 < s:
            h = up
        elif (Fraction(h) + Fraction(dn)) ** 2 / 4 > s:
            h = dn
        else:
            break
    return h


F16_PI = r16(math.pi)
F16_TWO_PI = r16(2 * math.pi)
F32_PI = r32(math.pi)
F32_TWO_PI = r32(2 * math.pi)


def pair_codes_f16(x: float, y: float, bits: int):
    """(radius, angle code) of one fp16 pair under encoder.py:33,46-55."""
    xx = r16(Fraction(x) * Fraction(x))
    yy = r16(Fraction(y) * Fraction(y))
    s = r16(Fraction(xx) + Fraction(yy)) if INF not in (xx, yy) else INF
    r = sqrt_r16(s)
    a = r16(math.atan2(y, x))  # float64 atan2 rounded once: the oracle's policy
    sh = r16(Fraction(a) + Fraction(F16_PI))
    n = r16(Fraction(sh) / Fraction(F16_TWO_PI))
    n = min(max(n, 0.0), 1.0)
    lv = 2 ** bits - 1
    c = round(Fraction(n) * lv)  # exact in fp32 (<= 19 significant bits), half-even
    return r, min(max(c, 0), lv)


def pair_codes_f32(x: float, y: float, bits: int):
    """(radius, angle code) of one fp32 pair (fp32 arithmetic, encoder.py:33,46-55)."""
    xx = r32(Fraction(x) * Fraction(x))
    yy = r32(Fraction(y) * Fraction(y))
    s = r32(Fraction(xx) + Fraction(yy))
    r = r16(sqrt_r32(Fraction(s)))
    a = r32(math.atan2(y, x))
    sh = r32(Fraction(a) + Fraction(F32_PI))
    n = r32(Fraction(sh) / Fraction(F32_TWO_PI))
    n = min(max(n, 0.0), 1.0)
    if n > r32(1 - 1e-6):
        n = 0.0
    lv = 2 ** bits - 1
    c = round(r32(Fraction(n) * lv))
    return r, min(max(c, 0), lv)


def log_radius_f16(r: float) -> float:
    """f16(log(max(r, fp16(1e-6)))) (encoder.py:37), float64 log rounded once."""
    rr = max(r, r16(1e-6))
    if rr == INF:
        return INF
    return r16(math.log(rr))


def v_group_f16(vals):
    """(scale, codes) of one 32-value fp16 group (v_quant/encoder.py:21-25)."""
    m = max(abs(v) for v in vals)
    s = r16(Fraction(m) / 127)
    if s == 0:
        s = r16(1e-4)
    codes = []
    for v in vals:
        q = r16(Fraction(v) / Fraction(s))
        codes.append(int(min(max(round(Fraction(q)), -128), 127)))
    return s, codes


def v_group_f32(vals):
    m = max(abs(v) for v in vals)
    s = r16(r32(Fraction(m) / 127))
    if s == 0:
        s = r16(1e-4)
    codes = []
    for v in vals:
        q = r32(Fraction(v) / Fraction(s))
        codes.append(int(min(max(round(Fraction(q)), -128), 127)))
    return s, codes
