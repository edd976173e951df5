#!/usr/bin/env python3
"""Derive the erfc coefficients used by gelu_erf() in common.hpp.

erfc(z) for z >= 0 is written as  t * exp(-z^2 + P(t)),  t = 1 / (1 + z/2),  the Chebyshev-fit
form of Press et al., Numerical Recipes (2nd ed., section 6.2).  f(t) = ln(erfc(z) / t) + z^2 is
smooth on (0, 1] (it tends to -ln(2 sqrt(pi)) as z -> inf).  The fit covers t in [0.4, 1], i.e.
z <= 3 (|v| <= 4.24), where fp16 GELU needs erfc to ~2e-7 relative; beyond it the polynomial
extrapolates smoothly (bounded as t -> 0) and exp(-z^2) carries the result: for v > 4.24 the
correction |v| q is below 0.1 fp16 ulp of v, and for v < -4.24 the result is within the fp16
subnormal range, where the absolute error is what counts.  Degree 6 is the lowest that keeps the
float32 evaluation correctly rounded on all but ~3e-4 of the fp16 inputs in [-12, 12] (degree 9 over
all z, the form's classic use, reaches ~1.6e-4 at three more FMAs per value); the script prints the
largest relative error of erfc on the fitted range and that count.

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

DEG, T_MIN, NODES = 6, 0.4, 4000


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
    zs = np.linspace(0, 2 * (1 / T_MIN - 1), 400001)
    ts = 1 / (1 + zs / 2)
    rel = np.abs(ts * np.exp(-zs * zs + P.polyval(ts, coef)) / erfc(zs) - 1).max()
    print(f"coefficients c0..c{DEG} (P(t) = sum c_i t^i):")
    print(", ".join("%.9ef" % c for c in coef))
    print(f"max relative error of erfc on [0, {zs[-1]:.2f}]: {rel:.2e}")
    log2e = np.log2(np.e)
    q_coef = coef * log2e
    q_coef[0] -= 1.0
    k_w, k_t = np.sqrt(log2e / 2), 1 / (2 * np.sqrt(log2e))
    print(f"exp2 form: Q coefficients c0..c{DEG}:")
    print(", ".join("%.9ef" % c for c in q_coef))
    print("w = |v| * %.9ef,  t = 1 / (1 + w * %.9ef)" % (k_w, k_t))
    # float32 evaluation of the kernel's sequence against float64, on every fp16 value in [-12, 12]
    f32 = np.float32
    v16 = np.arange(0, 65536, dtype=np.uint16).view(np.float16)
    v16 = v16[np.isfinite(v16) & (np.abs(v16) <= 12)]
    v = v16.astype(f32)
    w = np.abs(v) * f32(k_w)
    t = f32(1) / (w * f32(k_t) + f32(1))
    pq = np.full_like(v, f32(q_coef[DEG]))
    for c in q_coef[DEG - 1::-1]:
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
