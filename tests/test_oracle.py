"""Pin the CPU oracle before trusting it (CPU only).

Every function of ``oracle/`` is checked against something that does not
restate its own formula: brute-force float64 loops on tiny inputs, special
cases with closed-form answers (K=1 outer product, W=0, W=I), mathematical
identities (odd/even symmetries of GELU and the logistic function), the
standard library (``math.erf``, ``math.tanh``) and torch's own eager kernels
(the reference's eager path).  Each check is chosen so that a plausible slip
(dropped bias, transposed operand, erf vs tanh GELU, wrong reduction axis,
mean over the wrong length) fails it.
"""

import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import gemm_epilogue as ora
from oracle import workloads as ora_w


def _rng(seed=0):
    return np.random.default_rng(seed)


# ---------------------------------------------------------------------------
# GEMM
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("M,N,K", [(1, 1, 1), (3, 5, 7), (7, 2, 17), (4, 9, 1)])
def test_gemm_brute_force(M, N, K):
    r = _rng(1)
    a, b = r.standard_normal((M, K)), r.standard_normal((K, N))
    ref = [[sum(a[m, k] * b[k, n] for k in range(K)) for n in range(N)] for m in range(M)]
    assert np.allclose(ora.gemm(a, b), np.array(ref), rtol=1e-12, atol=1e-12)


def test_gemm_special_cases():
    r = _rng(2)
    x = r.standard_normal((6, 4))
    assert np.allclose(ora.gemm(x, np.eye(4)), x)                          # W = I
    assert np.allclose(ora.gemm(x, np.zeros((4, 3))), 0.0)                 # W = 0
    u, v = r.standard_normal((5, 1)), r.standard_normal((1, 8))
    assert np.allclose(ora.gemm(u, v), np.outer(u[:, 0], v[0]))            # K = 1
    rect = r.standard_normal((2, 3))
    with pytest.raises(ValueError):
        ora.gemm(rect, rect)                                               # shape check, no silent transpose


def test_gemm_matches_torch_fp64():
    r = _rng(3)
    a, b = r.standard_normal((33, 65)), r.standard_normal((65, 17))
    ref = torch.mm(torch.from_numpy(a), torch.from_numpy(b)).numpy()
    assert np.allclose(ora.gemm(a, b), ref, rtol=1e-12, atol=1e-12)


# ---------------------------------------------------------------------------
# Activations
# ---------------------------------------------------------------------------


def test_gelu_erf_closed_form_and_identities():
    xs = [-6.0, -2.5, -1.0, -0.1, 0.0, 0.3, 1.0, 2.0, 7.0]
    for x in xs:
        assert math.isclose(float(ora.gelu_erf(np.float64(x))),
                            0.5 * x * (1 + math.erf(x / math.sqrt(2))), rel_tol=1e-14, abs_tol=1e-15)
    x = np.linspace(-8, 8, 1001)
    assert np.allclose(ora.gelu_erf(x) - ora.gelu_erf(-x), x, atol=1e-13)  # Phi(x)+Phi(-x)=1
    # Phi(1) = 0.8413447460685429
    assert math.isclose(float(ora.gelu_erf(np.float64(1.0))), 0.8413447460685429, rel_tol=1e-13)
    t = torch.from_numpy(x)
    assert np.allclose(ora.gelu_erf(x), F.gelu(t, approximate="none").numpy(), atol=1e-12)


def test_gelu_tanh_closed_form_and_differs_from_erf():
    x = np.linspace(-8, 8, 1001)
    ref = 0.5 * x * (1 + np.tanh(math.sqrt(2 / math.pi) * (x + 0.044715 * x ** 3)))
    assert np.allclose(ora.gelu_tanh(x), ref, atol=1e-14)
    assert np.allclose(ora.gelu_tanh(x) - ora.gelu_tanh(-x), x, atol=1e-13)
    t = torch.from_numpy(x)
    assert np.allclose(ora.gelu_tanh(x), F.gelu(t, approximate="tanh").numpy(), atol=1e-12)
    # the two GELU forms are distinguishable (guards against the reference's erf-always defect)
    one = np.float64(1.0)
    assert abs(float(ora.gelu_tanh(one)) - float(ora.gelu_erf(one))) > 1e-4
    assert math.isclose(float(ora.gelu_tanh(one)),
                        0.5 * (1 + math.tanh(math.sqrt(2 / math.pi) * 1.044715)), rel_tol=1e-14)


def test_sigmoid_and_relu():
    x = np.linspace(-30, 30, 601)
    s = ora.sigmoid(x)
    assert ora.sigmoid(np.float64(0.0)) == 0.5
    assert np.allclose(s + ora.sigmoid(-x), 1.0, atol=1e-15)
    assert np.all((s >= 0) & (s <= 1))
    assert np.allclose(s, torch.sigmoid(torch.from_numpy(x)).numpy(), atol=1e-15)
    r = ora.relu(x)
    assert np.all(r >= 0) and np.array_equal(r[x > 0], x[x > 0]) and np.all(r[x <= 0] == 0)


# ---------------------------------------------------------------------------
# Epilogue chains and operand broadcasting
# ---------------------------------------------------------------------------


def test_apply_chain_broadcast_explicit_loops():
    r = _rng(4)
    M, N = 3, 4
    acc = r.standard_normal((M, N))
    row, col, tile, sc = r.standard_normal(N), r.standard_normal((M, 1)), r.standard_normal((M, N)), 0.5
    ops = [row, col, tile, np.float64(sc)]
    chain = [("add", 0, 1.0), ("mul", 1, 1.0), ("add", 2, -2.0), ("mul", 3, 1.0), ("add_scalar", -1, 0.25)]
    got, _ = ora.apply_chain(acc, chain, ops)
    want = np.empty((M, N))
    for m in range(M):
        for n in range(N):
            v = acc[m, n] + row[n]
            v = v * col[m, 0]
            v = v - 2.0 * tile[m, n]
            v = v * sc
            want[m, n] = v + 0.25
    assert np.allclose(got, want, atol=1e-14)


def test_apply_chain_self_ops_and_store():
    acc = np.array([[1.0, -2.0], [3.0, 0.5]])
    got, extras = ora.apply_chain(acc, [("add_self", -1, 2.0), ("store", 0, 1.0), ("mul_self", -1, 1.0)], [], 1)
    assert np.allclose(extras[0], 3.0 * acc)
    assert np.allclose(got, (3.0 * acc) ** 2)


def test_role_based_bias_not_rank_based():
    """Bias bound by role: bias then a trailing row add are two distinct operands.

    The reference's rank-based binding (kernel_generator.py:884-901) would add
    the trailing row twice; the oracle must not.
    """
    r = _rng(5)
    x, w = r.standard_normal((4, 3)), r.standard_normal((3, 5))
    b, row = r.standard_normal(5), r.standard_normal(5)
    out = ora.gemm_epilogue([b, x, w, row], 1, 2, [("add", 0, 1.0), ("add", 3, 1.0)])["tile"]
    assert np.allclose(out, x @ w + b + row)
    assert not np.allclose(out, x @ w + b + 2 * row)


def test_chain_matches_torch_eager_fp32():
    g = torch.Generator().manual_seed(6)
    x, w = torch.randn(17, 24, generator=g), torch.randn(40, 24, generator=g)
    b, gate, r = torch.randn(40, generator=g), torch.rand(17, 40, generator=g), torch.randn(40, generator=g)
    with torch.no_grad():
        ref = torch.sigmoid(torch.relu(F.linear(x, w, b)) * gate) + r
    chain = [("add", 0, 1.0), ("relu", -1, 1.0), ("mul", 3, 1.0), ("sigmoid", -1, 1.0), ("add", 4, 1.0)]
    inputs = [b.numpy(), x.numpy(), w.t().numpy(), gate.numpy(), r.numpy()]
    got = ora.gemm_epilogue(inputs, 1, 2, chain)["tile"]
    assert np.allclose(got, ref.double().numpy(), rtol=1e-5, atol=1e-5)


# ---------------------------------------------------------------------------
# Reductions
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("axis", [0, 1])
def test_reductions_against_torch_and_invariants(axis):
    v = _rng(7).standard_normal((13, 29))
    t = torch.from_numpy(v)
    assert np.allclose(ora.reduce(v, "sum", axis), t.sum(axis).numpy())
    assert np.allclose(ora.reduce(v, "amax", axis), t.amax(axis).numpy())
    assert np.allclose(ora.reduce(v, "mean", axis), t.mean(axis).numpy())
    assert np.allclose(ora.reduce(v, "mean", axis), ora.reduce(v, "sum", axis) / v.shape[axis])
    mx = ora.reduce(v, "amax", axis)
    assert np.all(mx[:, None] >= v) if axis == 1 else np.all(mx[None, :] >= v)
    assert ora.reduce(v, "sum", axis).shape == (v.shape[1 - axis],)


def test_relu_amax_nonnegative():
    v = ora.relu(_rng(8).standard_normal((9, 31)))
    assert np.all(ora.reduce(v, "amax", 1) >= 0)


# ---------------------------------------------------------------------------
# Output casts
# ---------------------------------------------------------------------------


def test_round_bf16_matches_torch_including_ties():
    r = _rng(9)
    x = np.concatenate([r.standard_normal(10000).astype(np.float32) * 100,
                        np.array([1.00390625, 1.01171875, -1.00390625, 0.0, -0.0, 3e38], np.float32)])
    ref = torch.from_numpy(x).to(torch.bfloat16).float().numpy()
    assert np.array_equal(ora.round_bf16(x), ref)


def test_round_f16_saturates():
    x = np.array([1e6, -1e6, 65504.0, 65519.0, 1.5, -3.25], np.float32)
    got = ora.round_f16_saturating(x)
    assert got[0] == 65504.0 and got[1] == -65504.0
    ref = torch.from_numpy(np.clip(x, -65504, 65504)).to(torch.float16).float().numpy()
    assert np.array_equal(got, ref)


# ---------------------------------------------------------------------------
# Workload forwards against torch eager modules (fp32, small shapes)
# ---------------------------------------------------------------------------


def _f64(t):
    return t.detach().double().numpy()


def test_workloads_match_torch_modules():
    from fuseml_amd.workloads import ActivationHeavy, GemmRowReductions, StackedMLP, TransformerMLP

    torch.manual_seed(0)
    x = torch.randn(9, 16)
    m = TransformerMLP(16, 40).eval()
    with torch.no_grad():
        ref = m(x)
    got = ora_w.transformer_mlp(_f64(x), _f64(m.linear1.weight), _f64(m.linear1.bias),
                                _f64(m.linear2.weight), _f64(m.linear2.bias))
    assert np.allclose(got, ref.double().numpy(), atol=1e-5)

    mt = TransformerMLP(16, 40, approximate="tanh", residual=False).eval()
    with torch.no_grad():
        ref = mt(x)
    got = ora_w.transformer_mlp(_f64(x), _f64(mt.linear1.weight), _f64(mt.linear1.bias),
                                _f64(mt.linear2.weight), _f64(mt.linear2.bias), approximate="tanh", residual=False)
    assert np.allclose(got, ref.double().numpy(), atol=1e-5)

    ma = ActivationHeavy(16, 40).eval()
    with torch.no_grad():
        ma.row.normal_()
        g = torch.rand(9, 40)
        ref = ma(x, g)
    got = ora_w.activation_heavy(_f64(x), _f64(ma.linear.weight), _f64(ma.linear.bias), _f64(g), _f64(ma.row))
    assert np.allclose(got, ref.double().numpy(), atol=1e-5)

    mr = GemmRowReductions(16, 40).eval()
    with torch.no_grad():
        h, s, mx, mean = mr(x)
    got = ora_w.gemm_row_reductions(_f64(x), _f64(mr.linear.weight))
    assert np.allclose(got["tile"], _f64(h), atol=1e-5)
    assert np.allclose(got["sum"], _f64(s), atol=1e-4)
    assert np.allclose(got["amax"], _f64(mx), atol=1e-5)
    assert np.allclose(got["mean"], _f64(mean), atol=1e-5)

    ms = StackedMLP(16, 24, 3).eval()
    with torch.no_grad():
        ref = ms(x)
    blocks = [(_f64(b.linear1.weight), _f64(b.linear1.bias), _f64(b.linear2.weight), _f64(b.linear2.bias))
              for b in ms.blocks]
    assert np.allclose(ora_w.stacked_mlp(_f64(x), blocks), ref.double().numpy(), atol=1e-4)


def test_workload_rows_subset_is_exact():
    r = _rng(10)
    x, w1, b1 = r.standard_normal((20, 8)), r.standard_normal((12, 8)), r.standard_normal(12)
    w2, b2 = r.standard_normal((8, 12)), r.standard_normal(8)
    full = ora_w.transformer_mlp(x, w1, b1, w2, b2)
    rows = np.array([0, 7, 19])
    assert np.allclose(ora_w.transformer_mlp(x, w1, b1, w2, b2, rows=rows), full[rows])


def test_pins_cover_every_oracle_function():
    for name in ("gemm", "gelu_erf", "gelu_tanh", "sigmoid", "relu", "apply_chain", "reduce",
                 "round_bf16", "round_f16_saturating", "gemm_epilogue"):
        assert name in ora.PINS, name
