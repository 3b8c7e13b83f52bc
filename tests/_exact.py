"""Exact-rational helpers: IEEE binary32 rounding of rationals, fused
multiply-add and the reference's accumulation chains, computed without
relying on any C code.  Used to pin the oracle's floating-point order."""
from fractions import Fraction

import numpy as np


def round_f32(x: Fraction) -> np.float32:
    """Round a rational to the nearest binary32 (ties to even); normal range only."""
    if x == 0:
        return np.float32(0.0)
    sign = -1 if x < 0 else 1
    a = abs(x)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    q = Fraction(2) ** (e - 23)
    m = a / q
    n = m.numerator // m.denominator
    r = m - n
    if r > Fraction(1, 2) or (r == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return np.float32(sign * float(n * q))


def fr(v) -> Fraction:
    return Fraction(float(np.float32(v)))


def fma32(a, b, c) -> np.float32:
    return round_f32(fr(a) * fr(b) + fr(c))


def l2_fma_chain(a, b) -> np.float32:
    """acc = fma(diff, diff, acc) over dimensions (the reference's device L2)."""
    acc = np.float32(0.0)
    for x, y in zip(np.asarray(a, np.float32), np.asarray(b, np.float32)):
        d = np.float32(x - y)
        acc = fma32(d, d, acc)
    return acc


def lut_entry_chain(r, p) -> np.float32:
    """One LUT entry in the op order of gpu_global.cu:115-158."""
    r = np.asarray(r, np.float32)
    p = np.asarray(p, np.float32)
    d = (r - p).astype(np.float32)
    s = len(d)
    if s == 4:
        return fma32(d[0], d[0], fma32(d[1], d[1], fma32(d[2], d[2], np.float32(d[3] * d[3]))))
    if s == 8:
        t = fma32(d[0], d[0], fma32(d[1], d[1], fma32(d[2], d[2], np.float32(d[3] * d[3]))))
        return fma32(d[4], d[4], fma32(d[5], d[5], fma32(d[6], d[6], fma32(d[7], d[7], t))))
    acc = np.float32(0.0)
    for x in d:
        acc = fma32(x, x, acc)
    return acc


def seq_sum_f32(terms) -> np.float32:
    acc = np.float32(0.0)
    for t in terms:
        acc = np.float32(acc + np.float32(t))
    return acc
