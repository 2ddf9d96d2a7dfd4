"""Fit the erf polynomial behind the kernels' GELU (prints the C constants).

erf(z) is odd and saturates, so it is approximated on [0, Z] as
    erf(z) ~= z * P(z^2),   P a degree-D polynomial,
and clamped beyond Z.  P is the weighted least-squares fit (weight z, so the
error of erf itself is levelled) on a dense grid, computed in a Chebyshev
basis of t = z^2 for conditioning and converted to monomial coefficients for
Horner evaluation, under one equality constraint: Z * P(Z^2) = 1, so that the
clamped value is exactly erf's limit.  Without it the clamped value is the
fit's value at Z (about erf(3) = 1 - 2.2e-5), and GELU(x) = x Phi(x) carries
that residue times |x| for every x beyond the clamp (x = -12: -1.3e-4 where
GELU is 0).

The kernel evaluates the normal CDF directly, Phi(x) = 0.5 + xc * Q(xc^2) with
xc = clamp(x, +-Z sqrt 2), Q_k = P_k / (2 sqrt 2 * 2^k) (``phi_coeffs``), which
folds the 1/sqrt 2 argument scaling and the 1/2 into the coefficients.
``kernel_coeffs`` rounds Q to float32 and then moves Q_0 by whole ulps until
the kernel's float32 evaluation (fused multiply-adds) of c Q(c^2) at the clamp
c = Z sqrt 2 is as close to 1/2 as float32 allows, so Phi is 0 and 1 there.

    python fuseml_amd/csrc/fit_erf.py
"""

import numpy as np
from numpy.polynomial import chebyshev as C
from numpy.polynomial import polynomial as P
from scipy.special import erf

Z = 3.0
D = 8


def fit(Z=Z, D=D):
    """Monomial coefficients of P (in t = z^2), least squares with Z P(Z^2) = 1."""
    z = np.linspace(1e-8, Z, 200001)
    t = z * z
    y = erf(z) / z
    s = 2 * t / (Z * Z) - 1                    # t in [0, Z^2] -> s in [-1, 1]
    A = C.chebvander(s, D) * z[:, None]        # weight z
    b = y * z
    g = np.ones(D + 1)                         # T_k(1) = 1: P(Z^2) = sum of the Chebyshev coefficients
    # KKT system of  min |A c - b|^2  subject to  g . c = 1 / Z
    kkt = np.zeros((D + 2, D + 2))
    kkt[: D + 1, : D + 1] = 2 * A.T @ A
    kkt[: D + 1, D + 1] = g
    kkt[D + 1, : D + 1] = g
    rhs = np.concatenate([2 * A.T @ b, [1.0 / Z]])
    ch = np.linalg.solve(kkt, rhs)[: D + 1]
    mono_s = C.cheb2poly(ch)                   # in s = a t + b
    a_, b_ = 2 / (Z * Z), -1.0
    mono = np.zeros(D + 1)
    for k, c in enumerate(mono_s):
        mono[: k + 1] += c * P.polypow([b_, a_], k)[: k + 1]
    return mono


def phi_coeffs(mono):
    """Coefficients of Q in Phi(x) = 0.5 + x * Q(x^2), from erf's P."""
    return [c / (2.0 * np.sqrt(2.0) * 2.0 ** k) for k, c in enumerate(mono)]


def _fma32(a, b, c):
    """float32 fused multiply-add: the float64 product of two float32 values is
    exact, so one rounding of the float64 sum to float32 (the sum's own
    float64 rounding aside) is the fma's."""
    return np.float32(np.float64(a) * np.float64(b) + np.float64(c))


def kernel_q_at(x, q):
    """The kernel's float32 Horner evaluation of Q(x^2) at one float32 x."""
    x = np.float32(x)
    t = np.float32(x * x)
    p = _fma32(q[-1], t, q[-2])
    for qk in q[-3::-1]:
        p = _fma32(p, t, qk)
    return p


def kernel_coeffs(Z=Z, D=D):
    """float32 Q_0..Q_D as the kernels hold them (Q_0 tuned at the clamp)."""
    q = [np.float32(c) for c in phi_coeffs(fit(Z, D))]
    c = np.float32(Z * np.sqrt(2.0))
    best = None
    for k in range(-64, 65):
        q0 = np.float32(q[0] * (1 + k * 2.0 ** -24))
        trial = [q0] + q[1:]
        hi = _fma32(c, kernel_q_at(c, trial), np.float32(0.5))
        lo = _fma32(-c, kernel_q_at(c, trial), np.float32(0.5))
        score = abs(float(hi) - 1.0) + abs(float(lo))
        if best is None or score < best[0]:
            best = (score, trial)
    return best[1]


def max_err(q, Z=Z):
    """Max |Phi_kernel(x) - Phi(x)| over |x| <= 12, float32 evaluation as in the kernel."""
    c = np.float32(Z * np.sqrt(2.0))
    x = np.linspace(-12, 12, 480001).astype(np.float32)
    xc = np.clip(x, -c, c)
    t = (xc * xc).astype(np.float32)
    p = np.float32(q[-1]) * t.astype(np.float64) + np.float64(q[-2])
    p = p.astype(np.float32)
    for qk in q[-3::-1]:
        p = (p.astype(np.float64) * t + np.float64(qk)).astype(np.float32)
    phi = (xc.astype(np.float64) * p + 0.5).astype(np.float32)
    ref = 0.5 * (1 + erf(x.astype(np.float64) / np.sqrt(2.0)))
    err = np.abs(phi - ref)
    return err.max(), float(x[err.argmax()])


if __name__ == "__main__":
    q = kernel_coeffs()
    err, at = max_err(q)
    print(f"// Phi(x) = 0.5 + xc Q(xc^2), xc = clamp(x, +-{Z} sqrt 2); max |error| {err:.2e} (at x={at:.3f})")
    print(f"constexpr float kPhiClamp = {Z * np.sqrt(2.0):.17g}f;")
    for k, c in enumerate(q):
        print(f"constexpr float kPhiQ{k} = {float(c):.9e}f;")
