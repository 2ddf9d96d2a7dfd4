"""Fit the erf polynomial behind the kernels' GELU (prints the C constants).

erf(z) is odd and saturates, so it is approximated on [0, Z] as
    erf(z) ~= z * P(z^2),   P a degree-D polynomial,
and clamped to 1 (in magnitude) beyond Z.  P is the weighted least-squares
fit (weight z, so the error of erf itself is levelled) on a dense grid,
computed in a Chebyshev basis of t = z^2 for conditioning and converted to
monomial coefficients for Horner evaluation.  The script also reports the
maximum absolute error of the float32 Horner evaluation against scipy's erf.

The kernel evaluates the normal CDF directly, Phi(x) = 0.5 + x * Q(x^2) for
|x| <= Z sqrt 2, with Q_k = P_k / (2 sqrt 2 * 2^k) (``phi_coeffs``), which
folds the 1/sqrt 2 argument scaling and the 1/2 into the coefficients.

    python fuseml_amd/csrc/fit_erf.py
"""

import numpy as np
from numpy.polynomial import chebyshev as C
from numpy.polynomial import polynomial as P
from scipy.special import erf

Z = 3.0
D = 8


def fit(Z=Z, D=D):
    z = np.linspace(1e-8, Z, 200001)
    t = z * z
    y = erf(z) / z
    # Chebyshev least squares on t in [0, Z^2], weight z
    ch = C.chebfit(2 * t / (Z * Z) - 1, y, D, w=z)
    # convert to monomials in t
    mono_s = C.cheb2poly(ch)  # in s = 2t/Z^2 - 1
    # substitute s = a t + b
    a, b = 2 / (Z * Z), -1.0
    mono = np.zeros(D + 1)
    for k, c in enumerate(mono_s):
        mono[: k + 1] += c * P.polypow([b, a], k)[: k + 1]
    return mono


def phi_coeffs(mono):
    """Coefficients of Q in Phi(x) = 0.5 + x * Q(x^2), from erf's P."""
    return [c / (2.0 * np.sqrt(2.0) * 2.0 ** k) for k, c in enumerate(mono)]


def max_err(mono, Z=Z):
    zt = np.linspace(0, 6, 400001).astype(np.float32)
    t32 = zt * zt
    p = np.float32(mono[-1])
    for c in mono[-2::-1]:
        p = p * t32 + np.float32(c)
    e = np.minimum(zt * p, np.float32(1.0))
    e = np.where(zt > Z, np.float32(1.0), e)
    err = np.abs(e.astype(np.float64) - erf(zt.astype(np.float64)))
    return err.max(), float(zt[err.argmax()])


if __name__ == "__main__":
    mono = fit()
    err, at = max_err(mono)
    print(f"// erf(z) = z * P(z^2) on [0, {Z}], clamped beyond; max |error| {err:.2e} (at z={at:.3f})")
    print(f"constexpr float kPhiClamp = {Z * np.sqrt(2.0):.17g}f;")
    for k, c in enumerate(phi_coeffs(mono)):
        print(f"constexpr float kPhiQ{k} = {c:.9e}f;")
