"""Exact rational rounding used by the oracle pins: round-to-nearest-even of a
Fraction to an IEEE binary format, with no floating-point arithmetic in the
loop.  Independent of numpy's ufuncs, so a check built on it pins what the
oracle's float16/float32 numpy operations compute."""
from fractions import Fraction

import numpy as np

F16_MANT, F16_EMIN, F16_EMAX = 10, -14, 15
F32_MANT, F32_EMIN, F32_EMAX = 23, -126, 127


def rne(x: Fraction, mant: int, emin: int, emax: int = None) -> Fraction:
    """x rounded to `mant` fraction bits (ties to even), subnormals below
    2**emin; values past the largest finite one return +-inf (as float)."""
    if x == 0:
        return Fraction(0)
    s = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, emin)
    ulp = Fraction(2) ** (e - mant)
    q = a / ulp
    n = q.numerator // q.denominator
    r = q - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2):
        n += 1
    v = n * ulp
    if emax is not None and v >= Fraction(2) ** (emax + 1):
        return s * float("inf")
    return s * v


def f16(x: Fraction) -> Fraction:
    return rne(x, F16_MANT, F16_EMIN, F16_EMAX)


def f32(x: Fraction) -> Fraction:
    return rne(x, F32_MANT, F32_EMIN, F32_EMAX)


def frac(v) -> Fraction:
    return Fraction(float(v))


def nearest_level(q, maxv: int) -> int:
    """The integer level in [0, maxv] nearest to q (ties to the even level),
    found by enumerating every level; NaN gives 0, q past the top gives maxv."""
    if isinstance(q, float):
        if q != q:
            return 0
        if q == float("inf"):
            return maxv
        if q == float("-inf"):
            return 0
    best = None
    for lev in range(maxv + 1):
        d = abs(Fraction(q) - lev)
        if best is None or d < best[0] or (d == best[0] and lev % 2 == 0):
            best = (d, lev)
    return best[1]


def pack_bits_msb(codes, bits: int, unit: int):
    """Concatenate `bits`-bit codes MSB first into bytes, zero-padding the code
    list to a multiple of `unit` codes (independent of any shift formula)."""
    n = -(-len(codes) // unit) * unit
    c = list(codes) + [0] * (n - len(codes))
    out_bits = []
    for v in c:
        for k in range(bits - 1, -1, -1):
            out_bits.append((int(v) >> k) & 1)
    return np.array([int("".join(map(str, out_bits[i:i + 8])), 2) for i in range(0, len(out_bits), 8)], np.uint8)
