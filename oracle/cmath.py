"""The reference runtime's own exp / erf / GELU in fp32 numpy arithmetic (TEST INFRASTRUCTURE ONLY).

Follows runtime/vault3.c:104-129 (v3_expf, v3_erff, v3_geluf) operation by operation.  numpy evaluates
each float32 operation with one IEEE rounding and never fuses a multiply with an add, which is how the
runtime's C is compiled (a standard C mode does not contract), so the results are the runtime's bit
for bit.  v3_expf: round-half-away k = [x / ln 2], r = x - k ln2_hi - k ln2_lo, a degree-7 Taylor
polynomial in Horner form, scaled by 2^k built in the exponent bits (two steps below 2^-126).
v3_erff: Abramowitz & Stegun 7.1.26.  v3_geluf: 0.5 x (1 + erf(x / sqrt 2)).
"""
from __future__ import annotations

import numpy as np

F = np.float32


def _bits(u) -> np.ndarray:
    return np.asarray(u, dtype=np.uint32).view(np.float32)


def expf(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    with np.errstate(over="ignore", under="ignore", invalid="ignore"):
        kf = x * F(1.44269504088896341)
        k = np.where(np.isfinite(kf), kf + np.where(kf >= F(0), F(0.5), F(-0.5)), F(0)).astype(np.int32)
        kfl = k.astype(np.float32)
        r = (x - kfl * F(0.693145751953125)) - kfl * F(1.428606765330187e-06)
        p = F(1.3888889e-3) + r * F(1.9841270e-4)
        p = F(8.3333338e-3) + r * p
        p = F(4.1666668e-2) + r * p
        p = F(1.6666667e-1) + r * p
        p = F(0.5) + r * p
        p = F(1.0) + r * p
        p = F(1.0) + r * p
        hi = p * _bits(np.full(x.shape, 254 << 23, np.uint32)) * F(2.0)
        lo = p * _bits(((np.clip(k, -150, 127) + 126 + 127).astype(np.int64) & 0xFF).astype(np.uint32) << 23) * \
            _bits(np.full(x.shape, 1 << 23, np.uint32))
        mid = p * _bits(((np.clip(k, -126, 127) + 127).astype(np.uint32)) << 23)
        y = np.where(k > 127, hi, np.where(k < -126, lo, mid))
        y = np.where(x > F(88.72), F(np.inf), y)
        y = np.where(x < F(-103.9), F(0.0), y)
    return y.astype(np.float32)


def erff(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    z = np.abs(x)
    t = F(1.0) / (F(1.0) + F(0.3275911) * z)
    p = (((((F(1.061405429) * t - F(1.453152027)) * t) + F(1.421413741)) * t - F(0.284496736)) * t +
         F(0.254829592)) * t
    y = F(1.0) - p * expf(-z * z)
    y = np.where(z > F(4.0), F(1.0), y)
    return np.where(x < F(0), -y, y).astype(np.float32)


def geluf(x) -> np.ndarray:
    x = np.asarray(x, dtype=np.float32)
    return (F(0.5) * x * (F(1.0) + erff(x * F(0.70710678118654752)))).astype(np.float32)
