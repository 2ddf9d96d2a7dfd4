"""Host-side checks of the kernels' closed-form math.

The erf polynomial constants are read from the HIP source and evaluated in
float32 exactly as the kernel's Horner scheme does, then compared with
scipy's erf (the library routine) and with the closed-form GELU identities.
The fit itself is reproduced from fuseml_amd/csrc/fit_erf.py.
"""

import math
import os
import re
import sys

import numpy as np
from scipy.special import erf

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(REPO, "fuseml_amd", "csrc", "gemm_epilogue.hip")


def _coeffs():
    text = open(SRC).read()
    found = dict(re.findall(r"constexpr float kErfP(\d) = ([-+0-9.eE]+)f;", text))
    return [np.float32(float(found[str(k)])) for k in range(len(found))]


def erf_poly32(z):
    c = _coeffs()
    z = np.asarray(z, dtype=np.float32)
    zc = np.clip(z, np.float32(-3.0), np.float32(3.0))
    t = zc * zc
    p = c[-1]
    for ck in c[-2::-1]:
        p = p * t + ck  # the kernel uses fma; float32 rounding differs by < 1 ulp
    return np.clip(zc * p, np.float32(-1.0), np.float32(1.0))


def test_erf_polynomial_error_bound():
    z = np.linspace(-8, 8, 400001, dtype=np.float32)
    err = np.abs(erf_poly32(z).astype(np.float64) - erf(z.astype(np.float64)))
    assert err.max() < 4e-5, err.max()


def test_erf_polynomial_is_odd_and_saturates():
    z = np.linspace(0, 8, 10001, dtype=np.float32)
    assert np.array_equal(erf_poly32(-z), -erf_poly32(z))
    assert erf_poly32(np.float32(0.0)) == 0.0
    assert np.all(np.abs(erf_poly32(np.float32([3.5, 6.0, 1e30]))) == 1.0)


def test_gelu_from_poly_matches_closed_form():
    x = np.linspace(-8, 8, 200001, dtype=np.float32)
    h = np.float32(0.5) * x
    g = h * erf_poly32(x * np.float32(1 / math.sqrt(2))) + h
    ref = 0.5 * x.astype(np.float64) * (1 + erf(x.astype(np.float64) / math.sqrt(2)))
    assert np.abs(g - ref).max() < 2e-4
    # GELU(x) - GELU(-x) = x holds for the exact function and for the odd erf approximation
    gm = (np.float32(-0.5) * x) * erf_poly32(-x * np.float32(1 / math.sqrt(2))) + np.float32(-0.5) * x
    assert np.allclose(g - gm, x, atol=1e-5)


def test_fit_script_reproduces_constants():
    sys.path.insert(0, os.path.join(REPO, "fuseml_amd", "csrc"))
    import fit_erf

    mono = fit_erf.fit()
    assert np.allclose(np.float32(mono), np.array(_coeffs()), rtol=1e-6, atol=1e-12)
    err, _ = fit_erf.max_err(mono)
    assert err < 4e-5


def test_gelu_tanh_as_sigmoid_identity():
    # 0.5 (1 + tanh(u)) == sigmoid(2u): the kernel computes GELU(tanh) as x * sigmoid(2u)
    u = np.linspace(-20, 20, 2001)
    assert np.allclose(0.5 * (1 + np.tanh(u)), 1 / (1 + np.exp(-2 * u)), atol=1e-15)
