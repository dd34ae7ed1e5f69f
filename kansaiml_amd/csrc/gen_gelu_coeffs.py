"""Derives the constants of kh::gelu (kh_act.h).

GELU(x) = x * Phi(x).  With a = |x| and u = Phi(-a) = erfc(a / sqrt(2)) / 2,
GELU(x) = x * (1 - u) for x >= 0 and x * u for x < 0.  erfc is taken in the
form of Numerical Recipes (Press et al., 2nd ed., section 6.2, erfcc):

    erfc(z) = t * exp(-z^2 + P(t)),   t = 1 / (1 + z / 2),

where P is smooth on t in (0, 1].  Here P is fitted anew, by Chebyshev
interpolation of degree 8 on z in [0, ZMAX] only (beyond it u < 1e-9, below
the rounding of 1 - u and negligible against |x| * u), and rewritten for the
kernel: in h = t / 2 = 1 / (2 + z), so that u = h * exp(-z^2 + P(2h)); as a
polynomial in h - H_MID (well-conditioned coefficients); with log2(e) folded
in, so that

    u = h * 2^(Q(h - H_MID) - a^2 * log2(e) / 2).

Prints the binary32 coefficients of Q (highest degree first, as kh_act.h
evaluates them) and the maximum relative error of the fitted erfc.  numpy
and scipy only; run from anywhere:  python3 gen_gelu_coeffs.py
"""

import numpy as np
from scipy.special import erfc

ZMAX = 4.4
DEGREE = 8
H_MID = 0.328125  # about the middle of h in [1 / (2 + ZMAX), 1 / 2], exact in binary32
LOG2E = 1.4426950408889634


def coefficients():
    h_lo, h_hi = 1.0 / (2.0 + ZMAX), 0.5

    def target(h):  # Q(h - H_MID) without the approximation: log2(erfc(z) / (2h)) + z^2 log2(e)
        z = 1.0 / h - 2.0
        return (np.log(erfc(z) / (2.0 * h)) + z * z) * LOG2E

    nodes = np.cos(np.linspace(0.0, np.pi, 4001)) * (h_hi - h_lo) / 2 + (h_hi + h_lo) / 2
    cheb = np.polynomial.chebyshev.chebfit(2 * (nodes - h_lo) / (h_hi - h_lo) - 1, target(nodes), DEGREE)
    poly = np.polynomial.Polynomial(np.polynomial.chebyshev.cheb2poly(cheb))
    # the Chebyshev variable as a function of s = h - H_MID
    shifted = poly(np.polynomial.Polynomial([2 * (H_MID - h_lo) / (h_hi - h_lo) - 1, 2 / (h_hi - h_lo)]))
    q = shifted.coef.astype(np.float32)
    h = np.linspace(h_lo, h_hi, 200001)
    err = np.abs(np.polynomial.polynomial.polyval(h - H_MID, shifted.coef) - target(h)).max() / LOG2E
    return q, err


if __name__ == "__main__":
    q, err = coefficients()
    print(f"max relative error of the fitted erfc on z in [0, {ZMAX}]: {err:.2e}")
    for i in range(DEGREE, -1, -1):
        print(f"  s^{i}: {float(q[i])!r}f")
