"""The int8-x GEMM's quantize-on-load (csrc/gemm.hip, x8_quantize) takes the piece scale m / 127 without a divide:
q0 = fl(m * r), r = fl(1 / 127), corrected by one residual step, s = fl(q0 + fl(m - q0 * 127) * r) (two fused
multiply-adds). The reference takes the IEEE quotient (kernels/dspark.hip:883-904, x_fill). This checks, in exact
rational arithmetic, that the two agree for every positive finite fp16 m (the GEMM input is fp16, so m is one)."""
from fractions import Fraction

import numpy as np


def f32(x):
    """x (a Fraction) rounded to the nearest float32, ties to even."""
    c = np.float32(float(x))
    cands = (np.nextafter(c, np.float32(-np.inf)), c, np.nextafter(c, np.float32(np.inf)))
    return min(cands, key=lambda y: (abs(Fraction(float(y)) - x), int(np.float32(y).view(np.uint32)) & 1))


def test_residual_quotient_equals_ieee_division_for_every_fp16():
    r = np.float32(1) / np.float32(127)
    assert Fraction(float(r)) != Fraction(1, 127)  # r is inexact: the correction step matters
    R = Fraction(float(r))
    bad = []
    first_guess_wrong = 0
    for u in range(1, 0x7C00):
        M = Fraction(float(np.uint16(u).view(np.float16)))
        want = f32(M / 127)
        q0 = f32(M * R)
        e = f32(M - Fraction(float(q0)) * 127)
        s = f32(Fraction(float(q0)) + Fraction(float(e)) * R)
        first_guess_wrong += q0 != want
        if s != want:
            bad.append(u)
    assert not bad, f"{len(bad)} fp16 values differ, first {bad[:4]}"
    # the uncorrected product alone is not the quotient for some m (so the test would catch a dropped step)
    assert first_guess_wrong > 0
