"""Host-side checks of the kernels' closed-form math.

The GELU constants (the normal-CDF polynomial) are read from the HIP source
and evaluated in float32 exactly as the kernel's Horner scheme does, then
compared with scipy's erf (the library routine), with the closed-form GELU and
its identities, and with the fit script that produced them.
"""

import math
import os
import re
import sys

import numpy as np
from scipy.special import erf

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
SRC = os.path.join(REPO, "fuseml_amd", "csrc", "gemm_epilogue.hip")


def _consts():
    text = open(SRC).read()
    q = dict(re.findall(r"constexpr float kPhiQ(\d) = ([-+0-9.eE]+)f;", text))
    clamp = float(re.search(r"constexpr float kPhiClamp = ([-+0-9.eE]+)f;", text).group(1))
    return [np.float32(float(q[str(k)])) for k in range(len(q))], np.float32(clamp)


def phi32(x):
    """The kernel's Phi(x) = 0.5 + xc * Q(xc^2), xc = clamp(x), in float32."""
    q, c = _consts()
    x = np.asarray(x, dtype=np.float32)
    xc = np.clip(x, -c, c)
    t = xc * xc
    p = q[-1]
    for qk in q[-2::-1]:
        p = p * t + qk  # the kernel uses fma; float32 rounding differs by < 1 ulp
    return xc * p + np.float32(0.5)


def gelu32(x):
    x = np.asarray(x, dtype=np.float32)
    return x * phi32(x)


def test_phi_error_bound():
    x = np.linspace(-12, 12, 600001, dtype=np.float32)
    ref = 0.5 * (1 + erf(x.astype(np.float64) / math.sqrt(2)))
    assert np.abs(phi32(x) - ref).max() < 4e-5


def test_phi_symmetry_and_range():
    x = np.linspace(0, 12, 10001, dtype=np.float32)
    assert np.allclose(phi32(x) + phi32(-x), 1.0, atol=1e-6)       # Phi(x) + Phi(-x) = 1
    assert phi32(np.float32(0.0)) == np.float32(0.5)
    assert np.all((phi32(x) > 0.49) & (phi32(x) < 1.0 + 5e-5))


def test_gelu_matches_closed_form():
    x = np.linspace(-10, 10, 200001, dtype=np.float32)
    ref = 0.5 * x.astype(np.float64) * (1 + erf(x.astype(np.float64) / math.sqrt(2)))
    err = np.abs(gelu32(x) - ref)
    assert err.max() < 2e-4                       # absolute, over |x| <= 10
    big = np.abs(x) > 0.5
    assert (err[big] / np.abs(ref[big] + 1e-30)).max() < 1e-3 or err[big].max() < 2e-4
    assert np.allclose(gelu32(x) - gelu32(-x), x, atol=2e-5)   # GELU(x) - GELU(-x) = x


def test_fit_script_reproduces_constants():
    sys.path.insert(0, os.path.join(REPO, "fuseml_amd", "csrc"))
    import fit_erf

    mono = fit_erf.fit()
    q, clamp = _consts()
    assert np.allclose(np.float32(fit_erf.phi_coeffs(mono)), np.array(q), rtol=1e-6, atol=1e-14)
    assert math.isclose(float(clamp), fit_erf.Z * math.sqrt(2), rel_tol=1e-7)
    err, _ = fit_erf.max_err(mono)
    assert err < 4e-5


def test_gelu_tanh_as_sigmoid_identity():
    # 0.5 (1 + tanh(u)) == sigmoid(2u): the kernel computes GELU(tanh) as x * sigmoid(2u)
    u = np.linspace(-20, 20, 2001)
    assert np.allclose(0.5 * (1 + np.tanh(u)), 1 / (1 + np.exp(-2 * u)), atol=1e-15)
