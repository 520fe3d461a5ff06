"""Fit of the polynomial inside portable_expf (gsplat_amd/csrc/common.h) and
its host restatement oracle_portable_expf (oracle/exact_ref.c).

Test infrastructure, not imported by anything: it records where the four
coefficients c3..c6 come from.  e^r on [-ln2/2, ln2/2] (the Cody-Waite
reduced range) is approximated by 1 + r + r^2/2 + c3 r^3 + c4 r^4 + c5 r^5 +
c6 r^6, whose first three coefficients are those of e^r and exact in float32.
c3..c6 minimise the maximum relative error |p(r)/e^r - 1| over a dense grid:
a linear program in (c3, c4, c5, c6, t) with the constraints
-t <= p(r_i)/e^{r_i} - 1 <= t (scipy's HiGHS solver).  The float32
roundings of the solution are the device constants; evaluated in float32
Horner form with fused multiply-adds they keep e^x within 0.9 ulp of the
double exp for every float x in [-87, 88] (an exhaustive check, run once).

Run: python oracle/exp_poly_fit.py
"""
from math import log

import numpy as np
from scipy.optimize import linprog


def fit(n_grid: int = 4001):
    a = log(2.0) / 2.0
    x = np.linspace(-a, a, n_grid)
    e = np.exp(x)
    powers = (3, 4, 5, 6)
    base = (1.0 + x + 0.5 * x * x) / e - 1.0
    m = np.stack([x ** j / e for j in powers], axis=1)
    scale = np.abs(m).max(axis=0)  # conditioning
    ms = m / scale
    ones = np.ones((n_grid, 1))
    a_ub = np.vstack([np.hstack([ms, -ones]), np.hstack([-ms, -ones])])
    b_ub = np.concatenate([-base, base])
    cost = np.zeros(len(powers) + 1)
    cost[-1] = 1.0
    res = linprog(cost, A_ub=a_ub, b_ub=b_ub,
                  bounds=[(None, None)] * len(powers) + [(0.0, None)], method="highs")
    assert res.status == 0, res.message
    return res.x[:-1] / scale


if __name__ == "__main__":
    c = fit()
    a = log(2.0) / 2.0
    r = np.linspace(-a, a, 200001)
    p = 1.0 + r + 0.5 * r * r + sum(cj * r ** j for cj, j in zip(c, (3, 4, 5, 6)))
    print("max relative error %.3e" % np.abs(p / np.exp(r) - 1.0).max())
    for j, cj in zip((3, 4, 5, 6), c):
        print("c%d = %s" % (j, float.hex(float(np.float32(cj)))))
