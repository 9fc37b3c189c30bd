"""Writes fp8_e4m3_from_fp16.bin: the E4M3 code the reference encoder
(int4_decode_step.hip:47-68) gives for every fp16 bit pattern 0..65535.

The table is derived in the value domain with exact rationals, independently
of the oracle's bit manipulation:
  * NaN -> +448; values clamp to [-448, 448];
  * |v| is rounded to 4 significant bits (1 implicit + 3 stored) at its own
    binade, half-way cases away from zero (the encoder adds fp32 mantissa
    bit 19 to the top three bits);
  * a biased E4M3 exponent <= 0 flushes to a signed zero, >= 15 saturates to
    the code 0x7E (+-448).

Usage: python tests/golden/make_fp8_table.py   (rewrites the .bin beside it)
"""
import math
import os
from fractions import Fraction

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "fp8_e4m3_from_fp16.bin")


def fp16_value(bits):
    """Exact value of an fp16 bit pattern (Fraction, or 'nan'/±inf floats)."""
    s = -1 if bits & 0x8000 else 1
    e = (bits >> 10) & 0x1F
    m = bits & 0x3FF
    if e == 0x1F:
        return float("nan") if m else s * float("inf")
    if e == 0:
        return s * Fraction(m, 1 << 24)
    return s * (1 + Fraction(m, 1024)) * Fraction(2) ** (e - 15)


def encode(bits):
    v = fp16_value(bits)
    if isinstance(v, float) and math.isnan(v):
        return 0x7E
    sign = 0x80 if bits & 0x8000 else 0
    if isinstance(v, float):  # +-inf
        v = Fraction(448) if v > 0 else Fraction(-448)
    a = min(abs(v), Fraction(448))
    if a == 0:
        return sign
    k = math.floor(math.log2(a))
    while Fraction(2) ** k > a:  # exact floor(log2 a)
        k -= 1
    while Fraction(2) ** (k + 1) <= a:
        k += 1
    q = a / Fraction(2) ** (k - 3)  # in [8, 16)
    n = math.floor(q + Fraction(1, 2))  # ties away from zero
    if n == 16:
        k, n = k + 1, 8
    E = k + 7
    if E <= 0:
        return sign
    if E >= 15:
        return sign | 0x7E
    return sign | (E << 3) | (n - 8)


def main():
    table = np.array([encode(b) for b in range(1 << 16)], dtype=np.uint8)
    table.tofile(OUT)
    print(f"wrote {OUT} ({table.size} bytes)")


if __name__ == "__main__":
    main()
