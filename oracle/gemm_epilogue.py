"""CPU oracle of the fused GEMM+epilogue path (numpy, float64 by default).

TEST INFRASTRUCTURE ONLY.  This module is the checker: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only to compute expected values or a CPU reference timing.  The
product path (``fuseml_amd``) never imports it and has no CPU fallback.

It restates what the reference's fused kernel computes for one fusion group
(fuseml/codegen/kernel_generator.py) as plain array arithmetic:

* GEMM: ``acc = A @ B`` accumulated in ``dtype``
  (kernel_generator.py:1454-1542, ``tl.dot(a, b, acc=acc)``).
* Epilogue, applied to the accumulator in chain order
  (kernel_generator.py:912-1065, emitters 1599-1903):
    add        v + s * operand      operand broadcast to [M,N]   (1745-1828)
    mul        v * operand                                       (1830-1903)
    relu       where(v > 0, v, 0)                                (1599-1605)
    gelu_erf   0.5 v (1 + erf(v / sqrt 2))                       (1607-1642)
    gelu_tanh  0.5 v (1 + tanh(sqrt(2/pi) (v + 0.044715 v^3)))   (torch semantics
               of approximate='tanh'; the reference ignores it — a defect)
    sigmoid    1 / (1 + exp(-v))                                 (1644-1656)
    scale      v * s ;  add_scalar  v + s ;  add_self  v + s v ;  mul_self  v * v
    store      copy of v into escape output k                    (2020-2039)
  The addmm bias is the first ``add`` of the chain, bound by role; the
  reference's rank-based bias (881-901) is a defect and is NOT restated.
* Reductions of the final value along axis 1 (over N -> [M]) or axis 0
  (over M -> [N]): sum, amax, mean = sum / len (1909-2018), over exactly the
  [M,N] elements (no padded tile elements, unlike 1959-1960, 1983-1984).
* Output cast: bf16 round-to-nearest-even; fp16 saturated to +-65504 before
  rounding (1544-1593).

Parity status of each function is stated in ``PINS`` below; every entry is
checked by ``tests/test_oracle.py``.
"""

from __future__ import annotations

import math
from typing import Dict, List, Sequence, Tuple

import numpy as np
from scipy.special import erf as _erf

SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
GELU_TANH_CUBIC = 0.044715
FP16_MAX = 65504.0

# function -> how tests/test_oracle.py pins it (nothing here is "unpinned").
PINS: Dict[str, str] = {
    "gemm": "brute-force float64 triple loop; K=1 outer product; W=0; W=I; torch.mm fp64",
    "gelu_erf": "math.erf closed form; x - (-x) identity; Phi(1); torch gelu",
    "gelu_tanh": "math.tanh closed form; odd identity; distinct from erf at x=1; torch gelu(tanh)",
    "sigmoid": "sigmoid(0)=1/2; s(x)+s(-x)=1; torch.sigmoid",
    "relu": "sign invariant; torch.relu",
    "apply_chain": "explicit-loop broadcasting on tiny inputs; torch eager chains; golden fixtures",
    "reduce": "mean == sum/len; amax >= every element; torch sum/amax/mean",
    "round_bf16": "torch .to(bfloat16) bit patterns incl. ties",
    "round_f16_saturating": "torch .to(float16) after clamp; +-65504 saturation",
    "gemm_epilogue": "golden fixtures from torch eager fp32 modules (tests/golden)",
    "workloads": "torch eager fp32 nn.Module forward of each config on small shapes",
}


def gemm(a: np.ndarray, b: np.ndarray, dtype=np.float64) -> np.ndarray:
    """acc[M,N] = A[M,K] @ B[K,N] (kernel_generator.py:1454-1542)."""
    return np.asarray(a, dtype=dtype) @ np.asarray(b, dtype=dtype)


def gelu_erf(v: np.ndarray) -> np.ndarray:
    return 0.5 * v * (1.0 + _erf(v / math.sqrt(2.0)))


def gelu_tanh(v: np.ndarray) -> np.ndarray:
    return 0.5 * v * (1.0 + np.tanh(SQRT_2_OVER_PI * (v + GELU_TANH_CUBIC * v * v * v)))


def sigmoid(v: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        return 1.0 / (1.0 + np.exp(-v))


def relu(v: np.ndarray) -> np.ndarray:
    return np.where(v > 0, v, 0.0).astype(v.dtype, copy=False)


def _broadcast(x: np.ndarray, shape: Tuple[int, int], dtype) -> np.ndarray:
    return np.broadcast_to(np.asarray(x, dtype=dtype), shape)


def apply_chain(
    acc: np.ndarray,
    chain: Sequence[Tuple[str, int, float]],
    operands: Sequence[np.ndarray],
    n_extra: int = 0,
) -> Tuple[np.ndarray, List[np.ndarray]]:
    """Run an epilogue chain on ``acc``; return (final value, escape outputs).

    ``chain`` holds ``(kind, index, scalar)`` triples; ``index`` selects from
    ``operands`` (add/mul) or the escape slot (store).
    """
    v = acc
    shape = v.shape
    extras: List[np.ndarray] = [None] * n_extra  # type: ignore[list-item]
    for kind, idx, s in chain:
        if kind == "add":
            v = v + s * _broadcast(operands[idx], shape, v.dtype)
        elif kind == "mul":
            v = v * _broadcast(operands[idx], shape, v.dtype)
        elif kind == "relu":
            v = relu(v)
        elif kind == "gelu_erf":
            v = gelu_erf(v)
        elif kind == "gelu_tanh":
            v = gelu_tanh(v)
        elif kind == "sigmoid":
            v = sigmoid(v)
        elif kind == "scale":
            v = v * s
        elif kind == "add_scalar":
            v = v + s
        elif kind == "add_self":
            v = v + s * v
        elif kind == "mul_self":
            v = v * v
        elif kind == "store":
            extras[idx] = v.copy()
        else:
            raise ValueError(f"unknown epilogue op {kind!r}")
    return v, extras


def reduce(v: np.ndarray, kind: str, axis: int) -> np.ndarray:
    """Row (axis=1) or column (axis=0) reduction (kernel_generator.py:1933-2018)."""
    if kind == "sum":
        return v.sum(axis=axis)
    if kind == "amax":
        return v.max(axis=axis)
    if kind == "mean":
        return v.sum(axis=axis) * (1.0 / v.shape[axis])
    raise ValueError(f"unknown reduction {kind!r}")


def gemm_epilogue(
    inputs: Sequence[np.ndarray],
    left: int,
    right: int,
    chain: Sequence[Tuple[str, int, float]],
    reductions: Sequence[str] = (),
    reduce_axis: int = 1,
    n_extra: int = 0,
    dtype=np.float64,
) -> Dict[str, object]:
    """Everything one fused launch produces, in ``dtype``.

    ``inputs`` are the group's external tensors in launcher order (A [M,K],
    B [K,N], epilogue operands broadcastable to [M,N]).  Returns
    ``{"tile": v, "extra": [...], "sum"/"amax"/"mean": [...]}``.
    """
    acc = gemm(inputs[left], inputs[right], dtype)
    v, extras = apply_chain(acc, chain, [np.asarray(x, dtype=dtype) for x in inputs], n_extra)
    out: Dict[str, object] = {"tile": v, "extra": extras}
    for r in reductions:
        out[r] = reduce(v, r, reduce_axis)
    return out


# ---------------------------------------------------------------------------
# Output casts
# ---------------------------------------------------------------------------


def round_bf16(x: np.ndarray) -> np.ndarray:
    """float32 -> bfloat16 (round to nearest, ties to even) -> float32."""
    f = np.ascontiguousarray(x, dtype=np.float32)
    u = f.view(np.uint32).astype(np.uint64)
    rounded = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
    nan = np.isnan(f)
    out = rounded.astype(np.uint32).view(np.float32).copy()
    out[nan] = np.nan
    return out


def round_f16_saturating(x: np.ndarray) -> np.ndarray:
    """Clamp to +-65504 then round to float16 (kernel_generator.py:1575-1581)."""
    return np.clip(np.asarray(x, dtype=np.float32), -FP16_MAX, FP16_MAX).astype(np.float16).astype(np.float32)
