#!/usr/bin/env python3
"""Derive the erfc coefficients used by gelu_erf() in common.hpp.

erfc(z) for z >= 0 is written as  t * exp(-z^2 + P(t)),  t = 1 / (1 + z/2),  the Chebyshev-fit
form of Press et al., Numerical Recipes (2nd ed., section 6.2).  f(t) = ln(erfc(z) / t) + z^2 is
smooth on (0, 1] (it tends to -ln(2 sqrt(pi)) as z -> inf), so a degree-9 polynomial fitted at
Chebyshev nodes gives erfc with a relative error below 1e-7 for every z (checked here in float64
against scipy.special.erfc, printed on exit).  Relative accuracy in the tail is what keeps
GELU(v) = v * erfc(-v / sqrt 2) / 2 correctly rounded in fp16 for negative v.

The kernel evaluates the exp2 form: with w = |v| * sqrt(log2(e) / 2) (so that w^2 = log2(e) z^2),
q = erfc(z) / 2 = t * exp2(Q(t) - w^2), t = 1 / (1 + w / (2 sqrt(log2 e))), Q = log2(e) P - 1, and
GELU(v) = max(v, 0) - |v| q for either sign of v.  The script prints Q's coefficients and the two
scale constants, and checks that form in float32 against float64 on every fp16 value in [-12, 12].

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
    log2e = np.log2(np.e)
    q_coef = coef * log2e
    q_coef[0] -= 1.0
    k_w, k_t = np.sqrt(log2e / 2), 1 / (2 * np.sqrt(log2e))
    print("exp2 form: Q coefficients c0..c9:")
    print(", ".join("%.9ef" % c for c in q_coef))
    print("w = |v| * %.9ef,  t = 1 / (1 + w * %.9ef)" % (k_w, k_t))
    # float32 evaluation of the kernel's sequence against float64, on every fp16 value in [-12, 12]
    f32 = np.float32
    v16 = np.arange(0, 65536, dtype=np.uint16).view(np.float16)
    v16 = v16[np.isfinite(v16) & (np.abs(v16) <= 12)]
    v = v16.astype(f32)
    w = np.abs(v) * f32(k_w)
    t = f32(1) / (w * f32(k_t) + f32(1))
    pq = np.full_like(v, f32(q_coef[9]))
    for c in q_coef[8::-1]:
        pq = pq * t + f32(c)
    q = t * np.exp2(pq - w * w)
    g32 = (np.maximum(v, f32(0)) - np.abs(v) * q).astype(np.float16)
    v64 = v16.astype(np.float64)
    from scipy.special import erf
    g64 = v64 * 0.5 * (1 + erf(v64 / np.sqrt(2)))
    exact16 = g64.astype(np.float16)
    mism = np.sum(g32.view(np.uint16) != exact16.view(np.uint16))
    print(f"fp16 GELU results differing from the correctly rounded value: {mism} of {v.size}")


if __name__ == "__main__":
    main()
