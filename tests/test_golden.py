"""Golden fixtures (tests/golden/*.npz, from torch eager fp32 — see make_golden.py).

CPU tier: the oracle reproduces every fixture.
GPU tier: the HIP kernel family (one fused launch per group, through the C ABI)
reproduces the bf16 fixtures within the stated tolerances
(tiles rtol/atol 2e-2; fp32 reductions 1e-2 of |ref|, floored at 1e-3 of the
reduction of |v|), and the fp32 fixture through the fp32 split path to
rtol/atol 1e-4.
"""

import os

import numpy as np
import pytest
import torch

from oracle import gemm_epilogue as ora
from oracle import workloads as ora_w

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def load(name):
    with np.load(os.path.join(HERE, name + ".npz"), allow_pickle=False) as z:
        return {k: z[k].astype(np.float64) for k in z.files}


# ---------------------------------------------------------------------------
# CPU: oracle vs fixtures
# ---------------------------------------------------------------------------


def test_oracle_mlp_block():
    d = load("mlp_block")
    assert np.allclose(ora_w.transformer_mlp(d["x"], d["w1"], d["b1"], d["w2"], d["b2"]), d["y"], atol=1e-5)
    assert np.allclose(ora.gelu_erf(ora_w.linear(d["x"], d["w1"], d["b1"])), d["h"], atol=1e-5)


def test_oracle_act_heavy():
    d = load("act_heavy")
    assert np.allclose(ora_w.activation_heavy(d["x"], d["w"], d["b"], d["g"], d["r"]), d["y"], atol=1e-5)


def test_oracle_row_reductions():
    d = load("row_reductions")
    got = ora_w.gemm_row_reductions(d["x"], d["w"])
    for k in ("h", "sum", "amax", "mean"):
        assert np.allclose(got["tile" if k == "h" else k], d[k], atol=1e-4), k


def test_oracle_col_reductions():
    d = load("col_reductions")
    out = ora.gemm_epilogue([d["b"], d["x"], d["w"].T], 1, 2, [("add", 0, 1.0), ("sigmoid", -1, 1.0)],
                           ("sum", "amax", "mean"), reduce_axis=0)
    for k in ("sum", "amax", "mean"):
        assert np.allclose(out[k], d[k], atol=1e-4), k


def test_oracle_transformer_mlp_tanh():
    d = load("transformer_mlp_tanh_fp32")
    got = ora_w.transformer_mlp(d["x"], d["w1"], d["b1"], d["w2"], d["b2"], approximate="tanh", residual=False)
    assert np.allclose(got, d["y"], atol=1e-5)


def test_oracle_stacked():
    d = load("stacked_mlp")
    blocks = [(d[f"w1_{i}"], d[f"b1_{i}"], d[f"w2_{i}"], d[f"b2_{i}"]) for i in range(3)]
    assert np.allclose(ora_w.stacked_mlp(d["x"], blocks), d["y"], atol=1e-4)


# ---------------------------------------------------------------------------
# GPU: HIP launches vs fixtures
# ---------------------------------------------------------------------------

RTOL = ATOL = 2e-2


def _t(a, dtype=torch.bfloat16):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dtype).cuda()


def _launch(ops, left, right, n_inputs, *args, **spec_kw):
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp
    from fuseml_amd.launcher import HipKernelLauncher

    spec = EpilogueSpec(left=left, right=right, ops=tuple(EpiOp(*o) for o in ops),
                        out_dtype=torch.bfloat16, **spec_kw)
    return HipKernelLauncher(spec, n_inputs)(*args)


def _close(got, ref, what):
    g = got.float().cpu().numpy().astype(np.float64)
    assert np.allclose(g, ref, rtol=RTOL, atol=ATOL), f"{what}: max err {np.abs(g - ref).max()}"


def _red_close(got, ref, scale, what):
    g = got.float().cpu().numpy().astype(np.float64)
    # 1e-2 of |ref|, floored at 1e-3 of the reduction of |v| (sums that cancel)
    assert np.all(np.abs(g - ref) <= 1e-2 * np.maximum(np.abs(ref), 1e-3 * scale) + 1e-7), what


@pytest.mark.gpu
def test_hip_mlp_block_golden():
    d = load("mlp_block")
    x = _t(d["x"])
    h = _launch([("add", 0), ("gelu_erf",)], 1, 2, 3, _t(d["b1"]), x, _t(d["w1"]).t())
    y = _launch([("add", 0), ("add", 3)], 1, 2, 4, _t(d["b2"]), h, _t(d["w2"]).t(), x)
    torch.cuda.synchronize()
    _close(h, d["h"], "h")
    _close(y, d["y"], "y")


@pytest.mark.gpu
def test_hip_act_heavy_golden():
    d = load("act_heavy")
    y = _launch([("add", 0), ("relu",), ("mul", 3), ("sigmoid",), ("add", 4)], 1, 2, 5,
                _t(d["b"]), _t(d["x"]), _t(d["w"]).t(), _t(d["g"]), _t(d["r"]))
    torch.cuda.synchronize()
    _close(y, d["y"], "y")


@pytest.mark.gpu
def test_hip_row_reductions_golden():
    d = load("row_reductions")
    h, s, mx, mean = _launch([("relu",)], 0, 1, 2, _t(d["x"]), _t(d["w"]).t(),
                             reductions=("sum", "amax", "mean"), reduce_axis=1,
                             reduce_dtypes=(torch.float32,) * 3,
                             outputs=(("tile",), ("red", "sum"), ("red", "amax"), ("red", "mean")))
    torch.cuda.synchronize()
    _close(h, d["h"], "h")
    a = np.abs(d["h"])
    _red_close(s, d["sum"], a.sum(1), "sum")
    _red_close(mx, d["amax"], a.max(1), "amax")
    _red_close(mean, d["mean"], a.mean(1), "mean")


@pytest.mark.gpu
def test_hip_col_reductions_golden():
    d = load("col_reductions")
    s, mx, mean = _launch([("add", 0), ("sigmoid",)], 1, 2, 3, _t(d["b"]), _t(d["x"]), _t(d["w"]).t(),
                          store_tile=False, reductions=("sum", "amax", "mean"), reduce_axis=0,
                          reduce_dtypes=(torch.float32,) * 3,
                          outputs=(("red", "sum"), ("red", "amax"), ("red", "mean")))
    torch.cuda.synchronize()
    _red_close(s, d["sum"], d["sum"], "sum")
    _red_close(mx, d["amax"], d["amax"], "amax")
    _red_close(mean, d["mean"], d["mean"], "mean")


@pytest.mark.gpu
def test_hip_stacked_golden():
    d = load("stacked_mlp")
    y = _t(d["x"])
    for i in range(3):
        h = _launch([("add", 0), ("gelu_erf",)], 1, 2, 3, _t(d[f"b1_{i}"]), y, _t(d[f"w1_{i}"]).t())
        y = _launch([("add", 0), ("add", 3)], 1, 2, 4, _t(d[f"b2_{i}"]), h, _t(d[f"w2_{i}"]).t(), y)
    torch.cuda.synchronize()
    _close(y, d["y"], "y")


@pytest.mark.gpu
def test_hip_transformer_mlp_tanh_fp32_golden():
    """The fp32 fixture through the fp32 path (both GEMM operands split into
    bf16 parts, fp32 epilogue and output): torch eager fp32's values to 1e-4."""
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp
    from fuseml_amd.launcher import HipKernelLauncher

    d = load("transformer_mlp_tanh_fp32")
    f32 = torch.float32

    def launch(ops, *args):
        spec = EpilogueSpec(left=1, right=2, ops=tuple(EpiOp(*o) for o in ops), out_dtype=f32)
        return HipKernelLauncher(spec, len(args))(*args)

    h = launch([("add", 0), ("gelu_tanh",)], _t(d["b1"], f32), _t(d["x"], f32), _t(d["w1"], f32).t())
    y = launch([("add", 0)], _t(d["b2"], f32), h, _t(d["w2"], f32).t())
    torch.cuda.synchronize()
    assert h.dtype == y.dtype == f32
    g = y.cpu().numpy().astype(np.float64)
    assert np.allclose(g, d["y"], rtol=1e-4, atol=1e-4), f"max err {np.abs(g - d['y']).max()}"
