"""Exact binary32 arithmetic on rationals, for closed-form known answers.

Every operation is evaluated exactly with ``fractions.Fraction`` and then
rounded once to the nearest binary32 value (ties to even), which is what an
IEEE-754 binary32 multiply or divide returns.  Nothing here calls numpy or
torch arithmetic, so the known answers do not depend on the libraries the
oracle or the kernels are checked against.

The two int8 per-token quantizer forms they separate:

* reciprocal multiply (vLLM ``dynamic_scaled_int8_quant``, the activation
  quantizer the reference calls at ``H3/inference/w8a8.py:178``):
  ``q = sat8(rne(fl(x * fl(127 / amax))))``, scale ``fl(amax / 127)``;
* division: ``q = rne(fl(x / fl(amax / 127)))``.

They round differently exactly where ``x * 127 / amax`` lies on a half-integer
(``x = amax / 2`` and its odd multiples): the rounded reciprocal or rounded
scale pushes the binary32 product or quotient to one side of the tie.
"""

from __future__ import annotations

from fractions import Fraction


def rn32(v: Fraction) -> Fraction:
    """Round a rational to the nearest binary32 value, ties to even (normal
    and subnormal range; the callers stay far from overflow)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    e = max(e, -126)                     # subnormals share the 2^-149 grid
    ulp = Fraction(2) ** (e - 23)
    m = a / ulp
    n = m.numerator // m.denominator
    rem = m - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sign * n * ulp


def rne_int(v: Fraction) -> int:
    """Round a rational to the nearest integer, ties to even (nearbyint)."""
    n = v.numerator // v.denominator
    rem = v - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return n


def sat8(q: int) -> int:
    return max(-128, min(127, q))


def int8_rcp_mul(x: float, amax: float) -> int:
    """vLLM form: sat8(rne(fl(x * fl(127 / amax)))); zero row -> 0."""
    if amax == 0:
        return 0
    inv = rn32(Fraction(127) / Fraction(amax))
    return sat8(rne_int(rn32(Fraction(x) * inv)))


def int8_div(x: float, amax: float) -> int:
    """Division form: sat8(rne(fl(x / fl(amax / 127))))."""
    if amax == 0:
        return 0
    s = rn32(Fraction(amax) / Fraction(127))
    return sat8(rne_int(rn32(Fraction(x) / s)))


def int8_scale(amax: float) -> Fraction:
    """The per-token scale both forms store: fl(amax / 127)."""
    return rn32(Fraction(amax) / Fraction(127))


def bf16_values(lo_bits: int, hi_bits: int, step: int = 1) -> list[float]:
    """Positive bf16 values with bit patterns in [lo_bits, hi_bits), as floats
    (exact: every bf16 value is a binary64 value)."""
    out = []
    for b in range(lo_bits, hi_bits, step):
        mant = b & 0x7F
        exp = (b >> 7) & 0xFF
        if exp == 0 or exp == 0xFF:
            continue
        out.append(float((Fraction(128 + mant, 128)) * Fraction(2) ** (exp - 127)))
    return out


def separating_cases(limit: int = 64) -> list[tuple[float, float, int, int]]:
    """(x, amax, q_rcp, q_div) with bf16 x <= amax where the two forms give
    different codes: the ties x * 127 / amax = n + 1/2 with x = (2n + 1) amax / 254
    representable in bf16."""
    cases = []
    for amax in bf16_values(0x3C00, 0x4300, 13):
        for odd in (1, 3, 5, 7, 127):
            x = Fraction(amax) * odd / 254     # x * 127 / amax = odd / 2
            xf = float(x)
            if Fraction(xf) != x or not _is_bf16(xf) or xf > amax:
                continue
            qr, qd = int8_rcp_mul(xf, amax), int8_div(xf, amax)
            if qr != qd:
                cases.append((xf, amax, qr, qd))
        if len(cases) >= limit:
            break
    return cases


def _is_bf16(v: float) -> bool:
    f = Fraction(v)
    if f == 0:
        return True
    a = abs(f)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    if Fraction(2) ** e > a:
        e -= 1
    m = a / Fraction(2) ** (e - 7)
    return m.denominator == 1 and -126 <= e <= 127
