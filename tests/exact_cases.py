"""Inputs with exactly known answers, shared by the oracle and package tests."""

from __future__ import annotations

from fractions import Fraction

import numpy as np


def crafted_error_case():
    """A weight whose quantization errors are known exactly (kernelforge/quantize.py:117-126).

    Four groups of 64 (G=64, N=2, K=128).  Each group holds +-absmax with absmax / 7 an exact fp16
    value, so the scale is absmax / 7 exactly, and every other value is chosen so fl32(w / s) is
    exact and rint gives a known q (ties to even at .5).  Returns (w fp32, err as Fractions per
    element), err = q*s - w.  The largest error is negative, so a max without abs() fails; the
    errors are not all equal in size, so rmse != max and a missing sqrt or a sum instead of a
    mean fails.
    """
    g = 64
    groups = [
        (7.0, [1.25, 2.5, 3.5, -0.375, -6.75, 0.5]),   # s = 1: q 1, 2 (tie), 4 (tie), 0, -7, 0 (tie)
        (14.0, [-3.0, 5.0, 9.5, 0.25]),              # s = 2: w/s -1.5 -> -2, 2.5 -> 2, 4.75 -> 5, 0.125 -> 0
        (3.5, [-1.3125, 0.75, 2.0]),                  # s = 0.5: w/s -2.625 -> -3, 1.5 -> 2, 4 -> 4
        (0.0, []),                                    # all zero: scale 1, q 0, no error
    ]
    w = np.zeros((2, 128), dtype=np.float32)
    errs = []
    for gi, (amax, vals) in enumerate(groups):
        row, col0 = divmod(gi * g, 128)
        s = Fraction(amax) / 7 if amax else Fraction(1)
        block = [0.0] * g
        if amax:
            block[0], block[1] = amax, -amax
        for i, v in enumerate(vals):
            block[2 + i] = v
        w[row, col0:col0 + g] = block
        for v in block:
            r = Fraction(v) / s
            q = max(-8, min(7, round(r)))  # Python's round is ties-to-even on Fractions
            errs.append(q * s - Fraction(v))
    return w, errs
