#!/usr/bin/env python3
"""Derives the double-precision erf of the GELU (kernels.hip `derf`, and the oracle's `ref_erf`
which must stay identical to it): two Chebyshev interpolants of erf evaluated at 40-digit
precision (mpmath), converted to monomials in the interval variable and printed as exact
hexadecimal C doubles.

  |x| < 1:      erf(x) = x * P(2 x^2 - 1),    P of degree 11 (erf(sqrt s) / sqrt s on s in [0, 1])
  1 <= |x| < 4: erf(x) = 1 - Q((2|x| - 5) / 3), Q of degree 20 (erfc on [1, 4])
  |x| >= 4:     +-1 (erfc(4) = 1.5e-8 is below half an f32 ulp of 1)

Run: python3 erf_coeffs.py  (prints the two tables and their measured errors)."""
import mpmath
import numpy as np
from numpy.polynomial import chebyshev as Ch

mpmath.mp.dps = 40


def cheb_monomial(func, a, b, deg):
    k = np.arange(deg + 1)
    t = np.cos(np.pi * (k + 0.5) / (deg + 1))
    ys = np.array([float(func(mpmath.mpf(a) + (mpmath.mpf(b) - a) * (mpmath.mpf(float(tt)) + 1) / 2)) for tt in t])
    return Ch.cheb2poly(Ch.chebfit(t, ys, deg))


def small(s):
    if s == 0:
        return 2 / mpmath.sqrt(mpmath.pi)
    r = mpmath.sqrt(s)
    return mpmath.erf(r) / r


P = cheb_monomial(small, 0, 1, 11)
Q = cheb_monomial(mpmath.erfc, 1, 4, 20)


def horner(c, t):
    p = c[-1]
    for v in c[-2::-1]:
        p = p * t + v
    return p


if __name__ == "__main__":
    for name, c in (("ERF_P", P), ("ERF_Q", Q)):
        print(f"{name}[{len(c)}] = {{")
        print(",\n".join("    " + ", ".join(float(v).hex() for v in c[i:i + 3]) for i in range(0, len(c), 3)))
        print("};")
    xs = np.linspace(0, 1, 4001)
    ea = max(abs(float(mpmath.erf(x)) - x * horner(P, 2 * x * x - 1)) for x in xs)
    xs = np.linspace(1, 4, 4001)
    eb = max(abs(float(mpmath.erf(x)) - (1 - horner(Q, (2 * x - 5) / 3))) for x in xs)
    print(f"max abs error: |x|<1 {ea:.2e}, 1<=|x|<4 {eb:.2e}")
