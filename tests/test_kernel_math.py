"""Host-side checks of the kernels' closed-form math.

The fp32 split product is checked against the exact float64 product and
against tf32 rounding (the reference's fp32 path).  The GELU constants (the normal-CDF polynomial) are read from the HIP source
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
SRC = os.path.join(REPO, "fuseml_amd", "csrc", "gelu_phi.h")


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
    # fused multiply-adds as in the kernel: the float64 product of two float32
    # values is exact, then one rounding to float32
    p = (np.float64(q[-1]) * t + np.float64(q[-2])).astype(np.float32)
    for qk in q[-3::-1]:
        p = (p.astype(np.float64) * t + np.float64(qk)).astype(np.float32)
    return (xc.astype(np.float64) * p + 0.5).astype(np.float32)


def gelu32(x):
    x = np.asarray(x, dtype=np.float32)
    return x * phi32(x)


def test_phi_error_bound():
    x = np.linspace(-12, 12, 600001, dtype=np.float32)
    ref = 0.5 * (1 + erf(x.astype(np.float64) / math.sqrt(2)))
    assert np.abs(phi32(x) - ref).max() < 1.5e-5


def test_phi_reaches_its_limits_at_the_clamp():
    """The constrained fit: Phi = 1 at +3 sqrt 2 and ~0 at -3 sqrt 2 in float32,
    so GELU beyond the clamp is x (above) and at most 3e-7 (below, |x| <= 14)."""
    _, c = _consts()
    assert phi32(c) == np.float32(1.0) and 0.0 <= phi32(-c) < 3e-8
    x = np.linspace(-14, -float(c), 20001, dtype=np.float32)
    assert np.abs(gelu32(x)).max() < 3e-7
    x = np.linspace(float(c), 14, 20001, dtype=np.float32)
    assert np.array_equal(gelu32(x), x)


def test_phi_symmetry_and_range():
    x = np.linspace(0, 12, 10001, dtype=np.float32)
    assert np.allclose(phi32(x) + phi32(-x), 1.0, atol=1e-6)       # Phi(x) + Phi(-x) = 1
    assert phi32(np.float32(0.0)) == np.float32(0.5)
    assert np.all((phi32(x) > 0.49) & (phi32(x) < 1.0 + 5e-5))


def test_gelu_matches_closed_form():
    x = np.linspace(-10, 10, 200001, dtype=np.float32)
    ref = 0.5 * x.astype(np.float64) * (1 + erf(x.astype(np.float64) / math.sqrt(2)))
    err = np.abs(gelu32(x) - ref)
    assert err.max() < 7e-5                       # absolute, over |x| <= 10
    big = x > 0.5
    assert (err[big] / np.abs(ref[big])).max() < 2e-5
    assert np.allclose(gelu32(x) - gelu32(-x), x, atol=2e-5)   # GELU(x) - GELU(-x) = x


def test_fit_script_reproduces_constants():
    sys.path.insert(0, os.path.join(REPO, "fuseml_amd", "csrc"))
    import fit_erf

    q, clamp = _consts()
    assert [float(v) for v in fit_erf.kernel_coeffs()] == [float(v) for v in q]
    assert np.float32(clamp) == np.float32(fit_erf.Z * math.sqrt(2))
    err, _ = fit_erf.max_err(q)
    assert err < 1.5e-5


def test_gelu_tanh_as_sigmoid_identity():
    # 0.5 (1 + tanh(u)) == sigmoid(2u): the kernel computes GELU(tanh) as x * sigmoid(2u)
    u = np.linspace(-20, 20, 2001)
    assert np.allclose(0.5 * (1 + np.tanh(u)), 1 / (1 + np.exp(-2 * u)), atol=1e-15)


# ---------------------------------------------------------------------------
# The fp32 split product (fuseml_amd/csrc/split_f32.hip): x = hi + lo with
# hi = bf16(x), lo = bf16(x - hi); a.b ~= hi.hi + hi.lo + lo.hi.
# ---------------------------------------------------------------------------


def _split(x):
    import torch

    t = torch.as_tensor(np.asarray(x, dtype=np.float32))
    hi = t.to(torch.bfloat16)
    lo = (t - hi.float()).to(torch.bfloat16)
    return hi.double().numpy(), lo.double().numpy()


def _tf32(x):
    """Round-to-nearest to 10 explicit mantissa bits (the tf32 input format)."""
    b = np.asarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    b = ((b + 0xFFF + ((b >> 13) & 1)) >> 13) << 13
    return b.astype(np.uint32).view(np.float32).astype(np.float64)


def test_split_represents_x_to_2_pow_minus_17():
    rng = np.random.default_rng(0)
    x = (rng.standard_normal(200000) * np.exp2(rng.integers(-60, 60, 200000))).astype(np.float32)
    hi, lo = _split(x)
    err = np.abs(x.astype(np.float64) - hi - lo)
    assert (err <= 2.0 ** -17 * np.abs(x)).all()
    assert (np.abs(lo) <= 2.0 ** -8 * np.abs(x)).all()      # lo is the rounding residue of hi


def test_split_segments_give_the_three_term_product():
    """A3 = [hi|hi|lo], B3 = [hi|lo|hi] along K: A3 . B3^T is exactly
    hi.hi + hi.lo + lo.hi (float64 sums of exact bf16 products)."""
    rng = np.random.default_rng(1)
    a, w = rng.standard_normal((5, 24)).astype(np.float32), rng.standard_normal((7, 24)).astype(np.float32)
    ah, al = _split(a)
    wh, wl = _split(w)
    a3, w3 = np.concatenate([ah, ah, al], 1), np.concatenate([wh, wl, wh], 1)
    assert np.allclose(a3 @ w3.T, ah @ wh.T + ah @ wl.T + al @ wh.T, rtol=1e-14, atol=0)


def test_split_product_is_far_closer_than_tf32():
    """Against the exact product of the fp32 inputs, the split product's error
    is below 2^-16 of sum |a||b| per output, and over 30x below tf32's."""
    rng = np.random.default_rng(2)
    K = 1024
    a = rng.standard_normal((64, K)).astype(np.float32)
    w = (rng.standard_normal((96, K)) / math.sqrt(K)).astype(np.float32)
    exact = a.astype(np.float64) @ w.astype(np.float64).T
    scale = np.abs(a.astype(np.float64)) @ np.abs(w.astype(np.float64)).T
    ah, al = _split(a)
    wh, wl = _split(w)
    split = ah @ wh.T + ah @ wl.T + al @ wh.T
    tf32 = _tf32(a) @ _tf32(w).T
    e_split, e_tf32 = np.abs(split - exact), np.abs(tf32 - exact)
    assert (e_split <= 2.0 ** -16 * scale).all()
    assert e_tf32.max() > 30 * e_split.max()
