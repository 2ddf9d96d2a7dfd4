"""CPU oracle of the five benchmark workloads (numpy).

TEST INFRASTRUCTURE ONLY (see ``oracle/gemm_epilogue.py``): used by tests/,
``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg.

Each function is the eager module of one benchmark config written as array
arithmetic on weights in ``nn.Linear`` layout ``W[out, in]`` (``y = x W^T + b``):

* C1/C2 ``transformer_mlp`` — benchmarks/bench_mlp_block.py:160-182
  (Linear -> GELU -> Linear [+ residual]); C1 uses GELU(tanh) and no residual.
* C3 ``activation_heavy`` — sigmoid(relu(x W^T + b) * g) + r.
* C4 ``gemm_row_reductions`` — h = relu(x W^T); sum, amax, mean of h over N.
* C5 ``stacked_mlp`` — bench_mlp_block.py:210-220, four C2-style blocks.

Rows are independent in every workload, so ``rows=`` evaluates a subset of
rows exactly (used to check full-size GPU results at sampled rows).
"""

from __future__ import annotations

from typing import Dict, Optional, Sequence, Tuple

import numpy as np

from .gemm_epilogue import gelu_erf, gelu_tanh, relu, sigmoid


def _f(x, dtype):
    return np.asarray(x, dtype=dtype)


def _rows(x, rows):
    return x if rows is None else x[rows]


def linear(x, w, b=None, dtype=np.float64):
    y = _f(x, dtype) @ _f(w, dtype).T
    if b is not None:
        y = y + _f(b, dtype)
    return y


def transformer_mlp(x, w1, b1, w2, b2, approximate="none", residual=True, rows=None, dtype=np.float64):
    xr = _f(_rows(x, rows), dtype)
    h = linear(xr, w1, b1, dtype)
    h = gelu_tanh(h) if approximate == "tanh" else gelu_erf(h)
    y = linear(h, w2, b2, dtype)
    return y + xr if residual else y


def activation_heavy(x, w, b, g, r, rows=None, dtype=np.float64):
    xr = _f(_rows(x, rows), dtype)
    h = relu(linear(xr, w, b, dtype))
    h = sigmoid(h * _f(_rows(g, rows), dtype))
    return h + _f(r, dtype)


def gemm_row_reductions(x, w, rows=None, dtype=np.float64) -> Dict[str, np.ndarray]:
    h = relu(linear(_f(_rows(x, rows), dtype), w, None, dtype))
    return {"tile": h, "sum": h.sum(axis=1), "amax": h.max(axis=1), "mean": h.sum(axis=1) / h.shape[1]}


def stacked_mlp(x, blocks: Sequence[Tuple], rows=None, dtype=np.float64):
    y = _f(_rows(x, rows), dtype)
    for w1, b1, w2, b2 in blocks:
        y = transformer_mlp(y, w1, b1, w2, b2, "none", True, None, dtype)
    return y
