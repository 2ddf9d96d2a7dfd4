"""The fused amax's integer-atomic dispatch, compiled from the kernel's own header.

``fuseml_amd/csrc/amax_order.h`` decides, for each partial maximum, whether the
device folds it into the fp32 output with a signed ``atomicMax`` or an unsigned
``atomicMin`` on its bits.  This test compiles that header with g++ on the host,
applies the two hardware atomics' semantics (signed max / unsigned min of 32-bit
words) to sequences of partials starting from the kernel's ``-inf`` fill, and
checks every result against ``numpy.maximum.reduce`` (NaN-propagating, like
``torch.amax``).  The cases that matter are signed zeros: ``-0.0`` compares
equal to ``+0.0`` but its bits are ``INT_MIN`` as a signed int, so a
``v >= 0`` dispatch loses it (``[-1.0, -0.0]`` would give ``-1.0``).
"""

from __future__ import annotations

import ctypes
import itertools
import pathlib
import shutil
import subprocess

import numpy as np
import pytest

HEADER_DIR = pathlib.Path(__file__).resolve().parents[1] / "fuseml_amd" / "csrc"

_SHIM = r"""
#include "amax_order.h"
extern "C" uint32_t fold(uint32_t stored, uint32_t vbits) {
  uint32_t x;
  if (fuseml_amax::atomic_for(vbits, &x) == fuseml_amax::kSignedMax)
    return (int32_t)stored > (int32_t)x ? stored : x;   // atomicMax on int
  return stored < x ? stored : x;                        // atomicMin on unsigned
}
"""


@pytest.fixture(scope="module")
def fold(tmp_path_factory):
    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    d = tmp_path_factory.mktemp("amax")
    src = d / "shim.cpp"
    src.write_text(_SHIM)
    lib = d / "libamax.so"
    subprocess.run(["g++", "-O1", "-shared", "-fPIC", "-D__host__=", "-D__device__=",
                    f"-I{HEADER_DIR}", str(src), "-o", str(lib)], check=True)
    so = ctypes.CDLL(str(lib))
    so.fold.restype = ctypes.c_uint32
    so.fold.argtypes = [ctypes.c_uint32, ctypes.c_uint32]
    return so.fold


NEG_INF_BITS = 0xFF800000


def _bits(x: float) -> int:
    return int(np.array([x], dtype=np.float32).view(np.uint32)[0])


def _float(b: int) -> float:
    return float(np.array([b], dtype=np.uint32).view(np.float32)[0])


def _device_amax(fold, partials):
    stored = NEG_INF_BITS
    for p in partials:
        stored = fold(stored, _bits(p))
    return _float(stored)


def _same(got: float, want: float) -> bool:
    if np.isnan(want):
        return bool(np.isnan(got))
    return got == want  # -0.0 == +0.0: torch.amax over a mix of zeros may return either


VALUES = [-0.0, 0.0, -1.0, 1.0, -2.5, 3.0, -np.inf, np.inf, np.nan, -1e-30, 1e-30,
          -3.4e38, 3.4e38, -1.4e-45]


def test_signed_zero_cases_from_review(fold):
    assert _same(_device_amax(fold, [-0.0]), -0.0)
    assert np.signbit(_device_amax(fold, [-0.0]))  # exactly -0.0, not -inf
    assert _same(_device_amax(fold, [-1.0, -0.0]), -0.0)
    assert _same(_device_amax(fold, [-2.5, -0.0, -3.0]), -0.0)
    assert _same(_device_amax(fold, [-0.0, -2.5]), -0.0)


def test_every_pair_and_triple_in_every_order(fold):
    for n in (1, 2, 3):
        for parts in itertools.product(VALUES, repeat=n):
            want = float(np.maximum.reduce(np.array(parts, dtype=np.float32)))
            got = _device_amax(fold, parts)
            assert _same(got, want), (parts, got, want)


def test_nan_is_sticky_in_both_orders(fold):
    for x in VALUES:
        assert np.isnan(_device_amax(fold, [np.nan, x]))
        assert np.isnan(_device_amax(fold, [x, np.nan]))
        assert np.isnan(_device_amax(fold, [x, -np.nan]))  # sign bit set NaN too


def test_random_partials_match_numpy(fold):
    rng = np.random.default_rng(0)
    for _ in range(300):
        n = int(rng.integers(1, 9))
        parts = rng.standard_normal(n).astype(np.float32)
        parts[rng.random(n) < 0.3] = -0.0
        parts[rng.random(n) < 0.1] = 0.0
        want = float(np.maximum.reduce(parts))
        assert _same(_device_amax(fold, [float(p) for p in parts]), want), parts
