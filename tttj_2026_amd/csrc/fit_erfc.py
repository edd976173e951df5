#!/usr/bin/env python3
"""Derive the erfc coefficients used by gelu_erf() in common.hpp.

erfc(z) for z >= 0 is written as  t * exp(-z^2 + P(t)),  t = 1 / (1 + z/2),  the Chebyshev-fit
form of Press et al., Numerical Recipes (2nd ed., section 6.2).  f(t) = ln(erfc(z) / t) + z^2 is
smooth on (0, 1] (it tends to -ln(2 sqrt(pi)) as z -> inf), so a degree-9 polynomial fitted at
Chebyshev nodes gives erfc with a relative error below 1e-7 for every z (checked here in float64
against scipy.special.erfc, printed on exit).  Relative accuracy in the tail is what keeps
GELU(v) = v * erfc(-v / sqrt 2) / 2 correctly rounded in fp16 for negative v.

Run:  python tttj_2026_amd/csrc/fit_erfc.py
"""

import numpy as np
from numpy.polynomial import chebyshev as C
from numpy.polynomial import polynomial as P
from scipy.special import erfc

DEG, T_MIN, NODES = 9, 0.07, 4000


def main() -> None:
    k = np.arange(NODES)
    tt = 0.5 * (1 + np.cos(np.pi * (k + 0.5) / NODES)) * (1 - T_MIN) + T_MIN
    z = 2 * (1 / tt - 1)
    f = np.log(erfc(z) / tt) + z * z
    x = 2 * (tt - T_MIN) / (1 - T_MIN) - 1
    cheb = C.chebfit(x, f, DEG)
    a, b = 2 / (1 - T_MIN), -2 * T_MIN / (1 - T_MIN) - 1
    coef = np.zeros(DEG + 1)
    for i, ci in enumerate(C.cheb2poly(cheb)):
        coef[: i + 1] += ci * P.polypow([b, a], i)
    zs = np.linspace(0, 12, 400001)
    ts = 1 / (1 + zs / 2)
    rel = np.abs(ts * np.exp(-zs * zs + P.polyval(ts, coef)) / erfc(zs) - 1).max()
    print("coefficients c0..c9 (P(t) = sum c_i t^i):")
    print(", ".join("%.9ef" % c for c in coef))
    print(f"max relative error of erfc on [0, 12]: {rel:.2e}")


if __name__ == "__main__":
    main()
