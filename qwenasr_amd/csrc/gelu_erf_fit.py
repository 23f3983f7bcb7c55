"""Derives the coefficients of the erf-GELU kernel (act.hip, gelu_erf) and
checks the float32 evaluation the kernel performs.

Method. Exact GELU is x * Phi(x) with Phi the normal CDF, and
Phi(x) = sigmoid(Q(x)) with Q(x) = 2 artanh(erf(x/sqrt2)) = ln(erfc(-t)/erfc(t)),
t = x/sqrt2. Q is odd and smooth, so on |x| <= X0 it is approximated by an odd
polynomial x * P(x^2), P of degree n-1. The coefficients come from a weighted
minimax fit (Lawson's iteratively reweighted least squares) of Q, weighted by
the sensitivity of GELU to Q, |x| * sigma(Q) * (1 - sigma(Q)), so the fit spends
its accuracy where GELU feels it. The float64 target uses scipy.special.erfc.

Evaluation in float32 (what the kernel does):
    xc = clamp(x, -X0, X0); q = xc * P(xc^2)          (Horner, fused multiply-adds)
    e  = exp(-|q|)                                     (<= 1: no overflow)
    t  = (x * e) * (1 / (1 + e))                       (= x * sigmoid(-|q|))
    gelu = x >= 0 ? x - t : t ;  gelu = 0 for x < -X0
Both branches avoid cancellation; beyond X0 the tails are exact to f32
rounding (exp(-Q(X0)) is below half an ulp of 1).

Run:  python qwenasr_amd/csrc/gelu_erf_fit.py     (prints the coefficients and
the worst absolute error against float64 over [-12, 12] plus N(0, 2^2) samples,
with the hardware exp2/rcp perturbed by +-1 ulp)
"""
from __future__ import annotations

import numpy as np
from scipy import special

N_TERMS = 7
X0 = 6.0          # clamp of the polynomial argument
FIT_RANGE = 5.5   # fit interval [0, FIT_RANGE]


def fit(n: int = N_TERMS, x_max: float = FIT_RANGE) -> np.ndarray:
    x = np.linspace(0, x_max, 400001)[1:]
    t = x / np.sqrt(2)
    q_target = np.log(special.erfc(-t) / special.erfc(t))
    sig = 1 / (1 + np.exp(-q_target))
    sens = x * sig * (1 - sig)
    u = (x / x_max) ** 2
    a = np.stack([x * u ** k for k in range(n)], 1)
    w = sens + 1e-3 * sens.max() * (x < 0.05)
    for _ in range(400):
        ww = w / w.max()
        c, *_ = np.linalg.lstsq(a * ww[:, None], q_target * ww, rcond=None)
        err = np.abs(a @ c - q_target) * sens
        w = w * (err / err.max()) ** 0.3 + 1e-30
    return np.array([c[k] / x_max ** (2 * k) for k in range(n)])


def _fma32(a, b, c):
    return (np.asarray(a, np.float64) * np.asarray(b, np.float64) + np.asarray(c, np.float64)).astype(np.float32)


def gelu_f32(x: np.ndarray, c32: np.ndarray, rcp_err: float = 0.0, exp_err: float = 0.0) -> np.ndarray:
    x = x.astype(np.float32)
    xc = np.clip(x, np.float32(-X0), np.float32(X0))
    x2 = (xc * xc).astype(np.float32)
    p = np.full_like(x2, c32[-1])
    for k in range(len(c32) - 2, -1, -1):
        p = _fma32(p, x2, np.full_like(x2, c32[k]))
    q = (xc * p).astype(np.float32)
    arg = (np.abs(q) * np.float32(-1.4426950408889634)).astype(np.float32)
    e = (np.exp2(arg.astype(np.float64)) * (1 + exp_err)).astype(np.float32)
    d = (np.float32(1) + e).astype(np.float32)
    r = ((1.0 / d.astype(np.float64)) * (1 + rcp_err)).astype(np.float32)
    t = ((x * e).astype(np.float32) * r).astype(np.float32)
    out = np.where(x >= 0, (x - t).astype(np.float32), t)
    return np.where(x < -X0, np.float32(0), out)


def main() -> None:
    c32 = fit().astype(np.float32)
    print("coefficients (float32, x^0 .. x^12 of P):")
    for k, v in enumerate(c32):
        print(f"  c{k} = {float(v)!r}  (bits 0x{np.float32(v).view(np.uint32):08x})")
    xs = np.concatenate([np.linspace(-12, 12, 2_400_001),
                         np.random.default_rng(0).standard_normal(2_000_000) * 2,
                         np.linspace(-1e-3, 1e-3, 20001), [-1e30, 1e30, -100, 100, 0.0]]).astype(np.float32)
    ref = 0.5 * xs.astype(np.float64) * special.erfc(-xs.astype(np.float64) / np.sqrt(2))
    worst = 0.0
    for re_, ee in [(0, 0), (1.2e-7, 1.2e-7), (-1.2e-7, -1.2e-7), (1.2e-7, -1.2e-7), (-1.2e-7, 1.2e-7)]:
        got = gelu_f32(xs, c32, re_, ee).astype(np.float64)
        worst = max(worst, float(np.nanmax(np.abs(got - ref))))
    print(f"worst |gelu_f32 - gelu_f64| = {worst:.3e}")


if __name__ == "__main__":
    main()
