"""GPU parity: the HIP kernel family (through the C ABI) against the CPU oracle.

Every case builds seeded bf16/f16 inputs on the CPU, runs one fused launch on
``cuda:0`` through :class:`fuseml_amd.launcher.HipKernelLauncher` (which calls
``fuseml_gemm_epilogue``), and compares with ``oracle.gemm_epilogue`` evaluated
in float64 on the same (exactly representable) input values.

Tolerances (stated by the benchmark contract):
  * 16-bit tile outputs: ``allclose(out, ref, rtol=2e-2, atol=2e-2)`` against
    the float64 oracle;
  * fp32 reductions: ``|red - ref| <= 1e-2 * |ref|``, floored at
    ``1e-2 * 1e-3 * ref_abs`` where ``ref_abs`` is the same reduction of
    ``|v|`` (only a sum or mean that cancels to within 0.1% of its scale
    reaches the floor);
  * fp32 groups (GEMM operands split into bf16 parts): fp32 tiles and
    reductions to rtol = atol = 1e-4; the split itself bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemm_epilogue as ora
from oracle import workloads as ora_w

pytestmark = pytest.mark.gpu

RTOL = 2e-2
ATOL = 2e-2
RED_RTOL = 1e-2
RED_FLOOR = 1e-3


def _launcher(spec, n_inputs):
    from fuseml_amd.launcher import HipKernelLauncher

    return HipKernelLauncher(spec, n_inputs)


def _spec(**kw):
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp

    ops = tuple(EpiOp(*o) if isinstance(o, tuple) else EpiOp(o) for o in kw.pop("ops"))
    return EpilogueSpec(ops=ops, **kw)


def _np(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy().astype(np.float64)


def _check_tile(out: torch.Tensor, ref: np.ndarray, what: str = "tile"):
    got = _np(out)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    bad = ~np.isclose(got, ref, rtol=RTOL, atol=ATOL)
    if bad.any():
        idx = np.argwhere(bad)[:5]
        raise AssertionError(
            f"{what}: {bad.sum()} of {bad.size} mismatches, e.g. "
            + ", ".join(f"{tuple(i)} got {got[tuple(i)]:.5f} ref {ref[tuple(i)]:.5f}" for i in idx)
        )


def _check_red(out: torch.Tensor, ref: np.ndarray, ref_abs: np.ndarray, what: str):
    got = _np(out)
    assert got.shape == ref.shape, (what, got.shape, ref.shape)
    tol = RED_RTOL * np.maximum(np.abs(ref), RED_FLOOR * ref_abs) + 1e-7
    err = np.abs(got - ref)
    assert (err <= tol).all(), f"{what}: max err {err.max()} (tol at worst {tol[err.argmax()]})"


def _gen(seed):
    return torch.Generator().manual_seed(seed)


def _gemm_inputs(M, N, K, dtype, seed=0):
    a = torch.randn(M, K, generator=_gen(seed)).to(dtype)
    w = (torch.randn(N, K, generator=_gen(seed + 1)) / max(K, 1) ** 0.5).to(dtype)
    return a, w


# ---------------------------------------------------------------------------
# Single-op and chain cases at small, ragged shapes
# ---------------------------------------------------------------------------

CHAINS = {
    "bias_gelu": [("add", 0, 1.0), ("gelu_erf", -1, 1.0)],
    "bias_gelu_tanh": [("add", 0, 1.0), ("gelu_tanh", -1, 1.0)],
    "bias_relu": [("add", 0, 1.0), ("relu", -1, 1.0)],
    "sigmoid": [("sigmoid", -1, 1.0)],
    "bias_residual": [("add", 0, 1.0), ("add", 1, 1.0)],
    "act_heavy": [("add", 0, 1.0), ("relu", -1, 1.0), ("mul", 1, 1.0), ("sigmoid", -1, 1.0), ("add", 2, 1.0)],
    "scalars": [("scale", -1, 0.5), ("add_scalar", -1, 0.125), ("add_self", -1, 2.0), ("mul_self", -1, 1.0)],
    "col_bias_alpha": [("add", 3, -0.5)],
    "bcast_mul": [("mul", 4, 1.0), ("add", 0, 1.0)],
}


def _operands(M, N, dtype, seed=10):
    """Operand slots: 0 row bias [N], 1 tile [M,N], 2 row [N], 3 column [M,1], 4 stride-0 expand."""
    g = _gen(seed)
    row = (torch.rand(N, generator=g) * 0.2 - 0.1).to(dtype)
    tile = torch.randn(M, N, generator=g).to(dtype)
    row2 = (torch.rand(N, generator=g) * 0.06 - 0.03).to(dtype)
    col = torch.randn(M, 1, generator=g).to(dtype)
    bc = torch.randn(1, N, generator=g).to(dtype).expand(M, N)
    return [row, tile, row2, col, bc]


SHAPES = [
    (256, 256, 64),     # one 256-tile, one K stage
    (512, 512, 1024),   # large-tile variant, several K stages
    (77, 200, 72),      # ragged M, N and K (K % 64 != 0)
    (1, 8, 8),          # minimum
    (300, 1000, 136),   # ragged, N % 4 == 0
    (130, 257, 48),     # N % 4 != 0: element-wise operand/store path
]


@pytest.mark.parametrize("chain", sorted(CHAINS))
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_chain_parity(chain, shape):
    M, N, K = shape
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype)
    ops = _operands(M, N, dtype)
    inputs = ops + [a, w.t()]
    left, right = len(ops), len(ops) + 1
    steps = CHAINS[chain]
    spec = _spec(left=left, right=right, ops=steps, out_dtype=dtype)
    print(f"case chain={chain} shape={shape}", flush=True)
    out = _launcher(spec, len(inputs))(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], left, right, steps)["tile"]
    _check_tile(out, ref, f"{chain} {shape}")


@pytest.mark.parametrize("axis", [1, 0])
@pytest.mark.parametrize("shape", [(256, 512, 128), (77, 200, 72), (600, 1030, 64), (513, 130, 40)],
                         ids=lambda s: "x".join(map(str, s)))
def test_reductions_parity(axis, shape):
    M, N, K = shape
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=3)
    bias = (torch.rand(N, generator=_gen(5)) - 0.5).to(dtype)
    inputs = [bias, a, w.t()]
    steps = [("add", 0, 1.0), ("sigmoid", -1, 1.0)]  # sigmoid(0)=0.5 would expose padded elements
    spec = _spec(left=1, right=2, ops=steps, out_dtype=dtype, store_tile=False,
                 reductions=("sum", "amax", "mean"), reduce_axis=axis,
                 reduce_dtypes=(torch.float32,) * 3,
                 outputs=(("red", "sum"), ("red", "amax"), ("red", "mean")))
    print(f"case reductions axis={axis} shape={shape}", flush=True)
    s, mx, mean = _launcher(spec, 3)(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], 1, 2, steps, ("sum", "amax", "mean"), axis)
    v = ref["tile"]
    _check_red(s, ref["sum"], np.abs(v).sum(axis=axis), "sum")
    _check_red(mx, ref["amax"], np.abs(v).max(axis=axis), "amax")
    _check_red(mean, ref["mean"], np.abs(v).mean(axis=axis), "mean")


# ---------------------------------------------------------------------------
# Every kernel variant (tile size and K-loop schedule), forced through
# _abi.force_variant (FUSEML_HIP_TILE is read once per process).  The automatic choice
# picks the 256x256 variants only at large sizes, so these cases are what pins
# the ping-pong ("large") and one-wave-per-SIMD ("deep", "deep3"; BK=64)
# schedules on every chain, on ragged edges and on K that ends mid-stage.
# ---------------------------------------------------------------------------

VARIANTS = ["large", "deep", "deep3", "deep3-generic", "small", "narrow64", "narrow32", "large128", "small64"]


def _k_for(variant, K):
    """deep3 (the one-wave schedule with whole-stage fragments; with the fixed
    chain kernels where a chain matches, or the generic op loop only under
    "deep3-generic") runs only for K % 64 == 0 (the library falls back to deep
    otherwise), so its cases keep the ragged M and N and round K up to a
    multiple of 64."""
    return -(-K // 64) * 64 if variant.startswith("deep3") else K


VARIANT_SHAPES = [
    (600, 1030, 200),   # ragged M and N, K ends mid-stage (BK=32 and BK=64)
    (257, 512, 72),     # one row past a 256 tile, K = one BK=64 stage + 8
    (512, 520, 2048),   # several tiles, many stages, N % 8 == 0 but not % 256
    (64, 96, 40),       # smaller than one tile, a single stage
]


@pytest.fixture
def forced_variant(request):
    from fuseml_amd import _abi

    _abi.force_variant(request.param)
    yield request.param
    _abi.force_variant(None)


@pytest.mark.parametrize("forced_variant", VARIANTS, indirect=True)
@pytest.mark.parametrize("chain", sorted(CHAINS))
@pytest.mark.parametrize("shape", VARIANT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_variant_chain_parity(forced_variant, chain, shape):
    M, N, K = shape
    K = _k_for(forced_variant, K)
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=21)
    ops = _operands(M, N, dtype, seed=22)
    inputs = ops + [a, w.t()]
    left, right = len(ops), len(ops) + 1
    steps = CHAINS[chain]
    spec = _spec(left=left, right=right, ops=steps, out_dtype=dtype)
    print(f"case variant={forced_variant} chain={chain} shape={shape}", flush=True)
    out = _launcher(spec, len(inputs))(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], left, right, steps)["tile"]
    _check_tile(out, ref, f"{forced_variant} {chain} {shape}")


# The automatic tile choice on the device (its CU count): one shape per tile it
# picks below a full round of 256x256 tiles, and a 64-row output with a full
# round of them (M <= 128 runs on the smaller tiles).  The launched tile is
# asserted through fuseml_gemm_epilogue_config, the output checked against
# the oracle on two chains (one with a 2-D operand).
AUTO_TILES = [
    ((2048, 4096, 256), (256, 128, 8)),   # 256 ping-pong tiles: one round
    ((2048, 1024, 256), (64, 128, 4)),
    ((1000, 1000, 256), (32, 128, 4)),    # ragged M and N
    ((128, 256, 1024), (32, 128, 4)),     # the reference's small preset's second GEMM
    ((64, 65536, 256), (64, 128, 4)),     # 64 rows against a wide weight: one row of 64x128 tiles
    ((100, 33000, 264), (128, 128, 4)),   # 100 rows: one row of 128x128 tiles at BK = 64, ragged N and K
    ((4096, 4096, 256), (256, 256, 8)),   # a full round: the 256x256 ping-pong kernel
]


@pytest.mark.parametrize("chain", ["bias_gelu", "bias_residual"])
@pytest.mark.parametrize("shape,tile", AUTO_TILES, ids=lambda v: "x".join(map(str, v)))
def test_automatic_tile_choice_parity(shape, tile, chain):
    import ctypes

    from fuseml_amd import _abi

    M, N, K = shape
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=31)
    ops = _operands(M, N, dtype, seed=32)[:2]
    inputs = ops + [a, w.t()]
    left, right = len(ops), len(ops) + 1
    steps = CHAINS[chain]
    spec = _spec(left=left, right=right, ops=steps, out_dtype=dtype)
    print(f"case automatic tile shape={shape} chain={chain}", flush=True)
    L = _launcher(spec, len(inputs))
    out = L(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    (plan,) = L._plans.values()
    cfg = (ctypes.c_int32 * 4)()
    lib = _abi.load_library()
    assert lib.fuseml_gemm_epilogue_config(plan.desc_ref, cfg) == 0, _abi.last_error(lib)
    assert tuple(cfg[:3]) == tile, (shape, tuple(cfg[:3]))
    ref = ora.gemm_epilogue([_np(t) for t in inputs], left, right, steps)["tile"]
    _check_tile(out, ref, f"auto {shape} {chain}")


# Fixed-chain kernels (compile-time epilogues of the deep3 variant) against the
# generic op loop of the same variant: the same arithmetic in the same order,
# so the outputs must be bitwise equal (sums and means, accumulated by fp32
# atomics in no fixed order across workgroups, to 1e-6 relative).
FIXED = {
    "none": ([], 1),
    "bias": ([("add", 0, 0.75)], 2),
    "bias_gelu": (CHAINS["bias_gelu"], 3),
    "bias_gelu_tanh": (CHAINS["bias_gelu_tanh"], 4),
    "bias_relu": (CHAINS["bias_relu"], 5),
    "bias_residual": ([("add", 0, 1.0), ("add", 1, -1.5)], 6),
    "act_heavy": (CHAINS["act_heavy"], 7),
    "relu": ([("relu", -1, 1.0)], 8),
}


def _chain_of(L):
    """The chain kernel id the launcher's (single) plan ran on."""
    import ctypes

    from fuseml_amd import _abi

    (plan,) = L._plans.values()
    return _abi.load_library().fuseml_gemm_epilogue_chain(ctypes.byref(plan.desc))


@pytest.mark.parametrize("name", sorted(FIXED))
@pytest.mark.parametrize("shape", [(600, 1024, 192), (4392, 4360, 128), (256, 512, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_fixed_chain_bitwise_equals_generic(name, shape):
    from fuseml_amd import _abi

    M, N, K = shape
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=91)
    ops = _operands(M, N, dtype, seed=92)
    inputs = [t.cuda() for t in ops + [a, w.t()]]
    left, right = len(ops), len(ops) + 1
    steps, want = FIXED[name]
    spec = _spec(left=left, right=right, ops=steps, out_dtype=dtype)
    print(f"case fixed chain={name} shape={shape}", flush=True)
    outs = {}
    try:
        for variant, chain in (("deep3", want), ("deep3-generic", 0)):
            _abi.force_variant(variant)
            L = _launcher(spec, len(inputs))
            outs[variant] = L(*inputs)
            torch.cuda.synchronize()
            assert _chain_of(L) == chain, (variant, _chain_of(L))
    finally:
        _abi.force_variant(None)
    assert torch.equal(outs["deep3"], outs["deep3-generic"]), f"{name}: fixed differs from generic"
    host = [t.cpu() for t in inputs]
    ref = ora.gemm_epilogue([_np(t) for t in host], left, right, steps)["tile"]
    _check_tile(outs["deep3"], ref, f"fixed {name} {shape}")


@pytest.mark.parametrize("axis", [1, 0])
@pytest.mark.parametrize("shape", [(600, 1032, 128), (4392, 4360, 192)], ids=lambda s: "x".join(map(str, s)))
def test_fixed_relu_reductions_equal_generic(axis, shape):
    """The ReLU + sum/amax/mean group (C4's) on its fixed kernel against the
    generic loop: tile and amax bitwise, sum and mean to 1e-6 relative."""
    from fuseml_amd import _abi

    M, N, K = shape
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=93)
    steps = [("relu", -1, 1.0)]
    spec = _spec(left=0, right=1, ops=steps, out_dtype=dtype, store_tile=True,
                 reductions=("sum", "amax", "mean"), reduce_axis=axis, reduce_dtypes=(torch.float32,) * 3,
                 outputs=(("tile",), ("red", "sum"), ("red", "amax"), ("red", "mean")))
    print(f"case fixed relu reductions axis={axis} shape={shape}", flush=True)
    res = {}
    try:
        for variant, chain in (("deep3", 8), ("deep3-generic", 0)):
            _abi.force_variant(variant)
            L = _launcher(spec, 2)
            res[variant] = L(a.cuda(), w.t().cuda())
            torch.cuda.synchronize()
            assert _chain_of(L) == chain
    finally:
        _abi.force_variant(None)
    (ft, fs, fm, fmean), (gt, gs, gm, gmean) = res["deep3"], res["deep3-generic"]
    assert torch.equal(ft, gt) and torch.equal(fm, gm)
    assert torch.allclose(fs, gs, rtol=1e-6, atol=1e-6) and torch.allclose(fmean, gmean, rtol=1e-6, atol=1e-6)
    ref = ora.gemm_epilogue([_np(a), _np(w.t())], 0, 1, steps, ("sum", "amax", "mean"), axis)
    v = ref["tile"]
    _check_tile(ft, v, "fixed relu tile")
    _check_red(fs, ref["sum"], np.abs(v).sum(axis=axis), "sum")
    _check_red(fm, ref["amax"], np.abs(v).max(axis=axis), "amax")
    _check_red(fmean, ref["mean"], np.abs(v).mean(axis=axis), "mean")


@pytest.mark.parametrize("forced_variant", VARIANTS, indirect=True)
@pytest.mark.parametrize("axis", [1, 0])
def test_variant_reductions_parity(forced_variant, axis):
    M, N, K = 600, 1030, _k_for(forced_variant, 200)
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=23)
    bias = (torch.rand(N, generator=_gen(24)) - 0.5).to(dtype)
    inputs = [bias, a, w.t()]
    steps = [("add", 0, 1.0), ("gelu_erf", -1, 1.0)]
    spec = _spec(left=1, right=2, ops=steps, out_dtype=dtype, store_tile=True,
                 reductions=("sum", "amax", "mean"), reduce_axis=axis,
                 reduce_dtypes=(torch.float32,) * 3,
                 outputs=(("tile",), ("red", "sum"), ("red", "amax"), ("red", "mean")))
    print(f"case variant={forced_variant} reductions axis={axis}", flush=True)
    tile, s, mx, mean = _launcher(spec, 3)(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], 1, 2, steps, ("sum", "amax", "mean"), axis)
    v = ref["tile"]
    _check_tile(tile, v, f"{forced_variant} tile")
    _check_red(s, ref["sum"], np.abs(v).sum(axis=axis), "sum")
    _check_red(mx, ref["amax"], np.abs(v).max(axis=axis), "amax")
    _check_red(mean, ref["mean"], np.abs(v).mean(axis=axis), "mean")


@pytest.mark.parametrize("forced_variant", VARIANTS, indirect=True)
@pytest.mark.parametrize("axis", [1, 0])
@pytest.mark.parametrize("shape", [(600, 1030, 200), (257, 512, 72), (64, 96, 40)],
                         ids=lambda s: "x".join(map(str, s)))
def test_variant_amax_of_nonpositive_values(forced_variant, axis, shape):
    """relu -> scale(-1) -> amax: every value is <= 0, and relu's +0 becomes
    -0.0, so most maxima are -0.0.  The fp32 atomic max must fold a -0.0
    partial in (it has the sign bit set: the unsigned-min path); one row of A
    and one row of W are all zero, so a whole output row and a whole column
    hold nothing but -0.0, whose maximum is -0.0, not the -inf fill."""
    M, N, K = shape
    K = _k_for(forced_variant, K)
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=61)
    a[min(3, M - 1)] = 0
    w[min(5, N - 1)] = 0
    steps = [("relu", -1, 1.0), ("scale", -1, -1.0)]
    spec = _spec(left=0, right=1, ops=steps, out_dtype=dtype, store_tile=True,
                 reductions=("amax", "sum"), reduce_axis=axis,
                 reduce_dtypes=(torch.float32,) * 2,
                 outputs=(("tile",), ("red", "amax"), ("red", "sum")))
    print(f"case variant={forced_variant} nonpositive amax axis={axis} shape={shape}", flush=True)
    tile, mx, s = _launcher(spec, 2)(a.cuda(), w.t().cuda())
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(a), _np(w.t())], 0, 1, steps, ("amax", "sum"), axis)
    v = ref["tile"]
    assert (v <= 0).all()
    _check_tile(tile, v, f"{forced_variant} tile")
    got = _np(mx)
    assert np.isfinite(got).all(), f"amax has -inf: {np.argwhere(~np.isfinite(got))[:5].ravel()}"
    _check_red(mx, ref["amax"], np.abs(v).max(axis=axis), "amax")
    _check_red(s, ref["sum"], np.abs(v).sum(axis=axis), "sum")
    zero_line = min(3, M - 1) if axis == 1 else min(5, N - 1)
    assert got[zero_line] == 0.0 and np.signbit(got[zero_line]), "all -0.0 line must give -0.0"


@pytest.mark.parametrize("forced_variant", VARIANTS, indirect=True)
@pytest.mark.parametrize("axis", [1, 0])
@pytest.mark.parametrize("store_tile", [True, False], ids=["tile", "notile"])
@pytest.mark.parametrize("shape", [(600, 1024, 200), (257, 512, 72)], ids=lambda s: "x".join(map(str, s)))
def test_variant_reductions_with_tile_operand(forced_variant, axis, store_tile, shape):
    """Reductions after a 2-D (LDS-staged) residual: the reduction partials reuse
    the staging tile's LDS, with and without a staged output."""
    M, N, K = shape
    K = _k_for(forced_variant, K)
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=25)
    bias = (torch.rand(N, generator=_gen(26)) - 0.5).to(dtype)
    resid = torch.randn(M, N, generator=_gen(27)).to(dtype)
    inputs = [bias, resid, a, w.t()]
    steps = [("add", 0, 1.0), ("add", 1, 1.0), ("sigmoid", -1, 1.0)]
    outputs = ((("tile",),) if store_tile else ()) + (("red", "sum"), ("red", "amax"), ("red", "mean"))
    spec = _spec(left=2, right=3, ops=steps, out_dtype=dtype, store_tile=store_tile,
                 reductions=("sum", "amax", "mean"), reduce_axis=axis,
                 reduce_dtypes=(torch.float32,) * 3, outputs=outputs)
    print(f"case variant={forced_variant} reductions+tile operand axis={axis} "
          f"store_tile={store_tile} shape={shape}", flush=True)
    res = _launcher(spec, len(inputs))(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], 2, 3, steps, ("sum", "amax", "mean"), axis)
    v = ref["tile"]
    if store_tile:
        _check_tile(res[0], v, f"{forced_variant} tile")
        res = res[1:]
    s, mx, mean = res
    _check_red(s, ref["sum"], np.abs(v).sum(axis=axis), "sum")
    _check_red(mx, ref["amax"], np.abs(v).max(axis=axis), "amax")
    _check_red(mean, ref["mean"], np.abs(v).mean(axis=axis), "mean")


@pytest.mark.parametrize("forced_variant", VARIANTS, indirect=True)
@pytest.mark.parametrize("K", [0, 8, 64, 96, 136])
def test_variant_tile_operand_short_k(forced_variant, K):
    """A 2-D operand with K of zero to a few stages: every way the staged
    operand's LDS slots can be left free by a short K loop."""
    M, N = 520, 776
    K = _k_for(forced_variant, K)
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=28)
    ops = _operands(M, N, dtype, seed=29)
    inputs = ops + [a, w.t()]
    left, right = len(ops), len(ops) + 1
    steps = CHAINS["bias_residual"]
    spec = _spec(left=left, right=right, ops=steps, out_dtype=dtype)
    print(f"case variant={forced_variant} tile operand K={K}", flush=True)
    out = _launcher(spec, len(inputs))(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], left, right, steps)["tile"]
    _check_tile(out, ref, f"{forced_variant} K={K}")


@pytest.mark.parametrize("forced_variant", VARIANTS, indirect=True)
@pytest.mark.parametrize("shape", [(600, 1024, 200), (257, 512, 72)], ids=lambda s: "x".join(map(str, s)))
def test_variant_fp16_chain(forced_variant, shape):
    """fp16 GEMM operands (f16 MFMA), an fp16 residual through the staging tile
    and an fp16 staged output, saturated at +-65504, on every variant."""
    M, N, K = shape
    K = _k_for(forced_variant, K)
    dtype = torch.float16
    a, w = _gemm_inputs(M, N, K, dtype, seed=31)
    bias = (torch.rand(N, generator=_gen(32)) - 0.5).to(dtype)
    resid = torch.randn(M, N, generator=_gen(33)).to(dtype)
    inputs = [bias, resid, a, w.t()]
    steps = [("add", 0, 1.0), ("gelu_erf", -1, 1.0), ("add", 1, 1.0), ("scale", -1, 3.0e4)]
    spec = _spec(left=2, right=3, ops=steps, out_dtype=dtype)
    print(f"case variant={forced_variant} fp16 chain shape={shape}", flush=True)
    out = _launcher(spec, len(inputs))(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], 2, 3, steps)["tile"]
    ref_sat = np.clip(ref, -ora.FP16_MAX, ora.FP16_MAX)
    got = _np(out)
    assert np.isfinite(got).all()
    assert np.allclose(got, ref_sat, rtol=RTOL, atol=ATOL * 3.0e4)


@pytest.mark.parametrize("forced_variant", ["large", "deep", "deep3"], indirect=True)
@pytest.mark.parametrize("shape,axis", [((4392, 4360, 136), 1), ((3996, 5112, 72), 0)],
                         ids=["324tiles-rows", "320tiles-cols"])
def test_variant_persistent_rounds(forced_variant, shape, axis):
    """More tiles than workgroups: the 256-wide variants launch one workgroup per
    CU and loop over the tiles in rounds.  324 tiles leave a last round of 68
    (not a multiple of the 8 XCDs: plain order), 320 tiles one of 64 (XCD
    order); ragged M and N, a staged residual and reductions that accumulate
    across the rounds."""
    M, N, K = shape
    K = _k_for(forced_variant, K)
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=41)
    bias = (torch.rand(N, generator=_gen(42)) - 0.5).to(dtype)
    resid = torch.randn(M, N, generator=_gen(43)).to(dtype)
    inputs = [bias, resid, a, w.t()]
    steps = [("add", 0, 1.0), ("add", 1, 1.0), ("gelu_erf", -1, 1.0)]
    spec = _spec(left=2, right=3, ops=steps, out_dtype=dtype, store_tile=True,
                 reductions=("sum", "amax", "mean"), reduce_axis=axis,
                 reduce_dtypes=(torch.float32,) * 3,
                 outputs=(("tile",), ("red", "sum"), ("red", "amax"), ("red", "mean")))
    print(f"case variant={forced_variant} persistent rounds shape={shape} axis={axis}", flush=True)
    tile, s, mx, mean = _launcher(spec, len(inputs))(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], 2, 3, steps, ("sum", "amax", "mean"), axis)
    v = ref["tile"]
    _check_tile(tile, v, f"{forced_variant} tile")
    _check_red(s, ref["sum"], np.abs(v).sum(axis=axis), "sum")
    _check_red(mx, ref["amax"], np.abs(v).max(axis=axis), "amax")
    _check_red(mean, ref["mean"], np.abs(v).mean(axis=axis), "mean")


@pytest.mark.parametrize("forced_variant", ["large"], indirect=True)
@pytest.mark.parametrize("shape,resid", [
    ((4392, 4360, 264), True),    # 324 tiles (plain order), K ends mid-stage: 9 stages
    ((3996, 5112, 256), True),    # 320 tiles (XCD order), exactly 2 x 4 stages
    ((6000, 6100, 512), False),   # 576 tiles: up to three per workgroup, no staged operand
    ((4392, 4360, 224), True),    # 7 stages
], ids=["324tiles-k264", "320tiles-k256", "576tiles-bias-gelu", "324tiles-k224"])
def test_variant_persistent_rounds_staged_output(forced_variant, shape, resid):
    """The ping-pong schedule over more tiles than workgroups with a staged
    output and no reductions: ragged M and N, one to three tiles per
    workgroup, K from 7 to 16 stages, with and without the DMA-staged residual."""
    M, N, K = shape
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=51)
    bias = (torch.rand(N, generator=_gen(52)) - 0.5).to(dtype)
    inputs = [bias]
    steps = [("add", 0, 1.0)]
    if resid:
        inputs.append(torch.randn(M, N, generator=_gen(53)).to(dtype))
        steps.append(("add", 1, 1.0))
    steps.append(("gelu_erf", -1, 1.0))
    inputs += [a, w.t()]
    left, right = len(inputs) - 2, len(inputs) - 1
    spec = _spec(left=left, right=right, ops=steps, out_dtype=dtype)
    print(f"case variant={forced_variant} persistent staged output shape={shape} resid={resid}", flush=True)
    out = _launcher(spec, len(inputs))(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(t) for t in inputs], left, right, steps)["tile"]
    _check_tile(out, ref, f"persistent staged output {shape}")


def test_escape_store_and_tile_with_reductions():
    """mm -> relu (escapes) -> row sum/amax/mean: the C4 group shape, small."""
    M, N, K = 320, 640, 256
    dtype = torch.bfloat16
    a, w = _gemm_inputs(M, N, K, dtype, seed=7)
    steps = [("relu", -1, 1.0), ("store", 0, 1.0)]
    spec = _spec(left=0, right=1, ops=steps, out_dtype=dtype, store_tile=False,
                 reductions=("sum", "amax", "mean"), reduce_axis=1,
                 reduce_dtypes=(torch.float32,) * 3, extra_dtypes=(dtype,),
                 outputs=(("extra", 0), ("red", "sum"), ("red", "amax"), ("red", "mean")))
    h, s, mx, mean = _launcher(spec, 2)(a.cuda(), w.t().cuda())
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(a), _np(w.t())], 0, 1, steps, ("sum", "amax", "mean"), 1, n_extra=1)
    _check_tile(h, ref["extra"][0], "escape tile")
    v = ref["tile"]
    _check_red(s, ref["sum"], np.abs(v).sum(1), "sum")
    _check_red(mx, ref["amax"], np.abs(v).max(1), "amax")
    _check_red(mean, ref["mean"], np.abs(v).mean(1), "mean")


def test_fp16_operands_and_saturation():
    M, N, K = 128, 256, 64
    a, w = _gemm_inputs(M, N, K, torch.float16, seed=11)
    steps = [("scale", -1, 4.0e4)]  # pushes |v| past 65504 -> saturates
    spec = _spec(left=0, right=1, ops=steps, out_dtype=torch.float16)
    out = _launcher(spec, 2)(a.cuda(), w.t().cuda())
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(a), _np(w.t())], 0, 1, steps)["tile"]
    ref_sat = np.clip(ref, -ora.FP16_MAX, ora.FP16_MAX)
    got = _np(out)
    assert np.isfinite(got).all()
    assert (np.abs(got) <= ora.FP16_MAX).all()
    assert np.allclose(got, ref_sat, rtol=RTOL, atol=ATOL * 4.0e4)


def test_k_zero_is_epilogue_of_bias():
    M, N = 64, 96
    a = torch.empty(M, 0, dtype=torch.bfloat16)
    w = torch.empty(N, 0, dtype=torch.bfloat16)
    bias = torch.linspace(-2, 2, N).to(torch.bfloat16)
    steps = [("add", 0, 1.0), ("gelu_erf", -1, 1.0)]
    spec = _spec(left=1, right=2, ops=steps, out_dtype=torch.bfloat16)
    out = _launcher(spec, 3)(bias.cuda(), a.cuda(), w.t().cuda())
    torch.cuda.synchronize()
    ref = np.broadcast_to(ora.gelu_erf(_np(bias)), (M, N))
    _check_tile(out, ref, "K=0")


def test_transposed_and_strided_gemm_operands():
    """A given K-strided and B given N-contiguous: the launcher re-lays them out."""
    M, N, K = 192, 320, 96
    a, w = _gemm_inputs(M, N, K, torch.bfloat16, seed=13)
    a_t = a.t().contiguous().t()          # stride (1, M): not K-contiguous
    b_nmajor = w.t().contiguous()         # [K,N] row-major: N-contiguous
    spec = _spec(left=0, right=1, ops=[("relu",)], out_dtype=torch.bfloat16)
    out = _launcher(spec, 2)(a_t.cuda(), b_nmajor.cuda())
    torch.cuda.synchronize()
    ref = ora.relu(ora.gemm(_np(a), _np(w.t())))
    _check_tile(out, ref, "relayout")


@pytest.mark.parametrize("forced_variant", ["auto", "large", "deep3"], indirect=True)
def test_graph_capture_replays(forced_variant):
    """A fused launch captured in a HIP graph (torch.cuda.CUDAGraph).  The
    launcher only queues work on the current stream: the reduction buffers are
    cleared by a fill kernel, not a memset, and nothing is read back to the
    host.  Each replay, after new values are copied into the captured inputs
    and with eager launches and synchronisations between replays, gives the
    eager launch's tile and amax bit for bit, and the oracle's sum."""
    M, N, K = 600, 1030, 192
    dtype = torch.bfloat16
    steps = [("add", 0, 1.0), ("gelu_erf", -1, 1.0), ("add", 1, 1.0)]
    spec = _spec(left=2, right=3, ops=steps, out_dtype=dtype, store_tile=True,
                 reductions=("sum", "amax"), reduce_axis=1,
                 reduce_dtypes=(torch.float32, torch.float32),
                 outputs=(("tile",), ("red", "sum"), ("red", "amax")))
    L = _launcher(spec, 4)

    def host_inputs(seed):
        a, w = _gemm_inputs(M, N, K, dtype, seed=seed)
        bias = (torch.rand(N, generator=_gen(seed + 2)) - 0.5).to(dtype)
        resid = torch.randn(M, N, generator=_gen(seed + 3)).to(dtype)
        return [bias, resid, a, w.t()]

    print(f"case graph capture variant={forced_variant}", flush=True)
    static = [t.cuda() for t in host_inputs(40)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        L(*static)  # first call builds the launch plan outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_tile, g_sum, g_amax = L(*static)
    for seed in (41, 42, 43):
        host = host_inputs(seed)
        for dst, src in zip(static, host):
            dst.copy_(src)
        e_tile, _, e_amax = L(*static)  # eager launch on the same inputs
        torch.cuda.synchronize()
        g_tile.fill_(float("nan"))  # a replay that wrote nothing would show
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_tile, e_tile), f"replay seed {seed}: tile differs from eager"
        assert torch.equal(g_amax, e_amax), f"replay seed {seed}: amax differs from eager"
        ref = ora.gemm_epilogue([_np(t) for t in host], 2, 3, steps, ("sum", "amax"), 1)
        _check_tile(g_tile, ref["tile"], f"replay seed {seed}")
        _check_red(g_sum, ref["sum"], np.abs(ref["tile"]).sum(axis=1), f"replay seed {seed} sum")
        _check_red(g_amax, ref["amax"], np.abs(ref["tile"]).max(axis=1), f"replay seed {seed} amax")


# ---------------------------------------------------------------------------
# fp32 GEMM groups: both operands split into bf16 parts (fuseml_split_bf16x3),
# one bf16 GEMM over K' = 3 ceil8(K).  The split is integer/bit work and is
# checked bit for bit; the fused fp32 results are checked against the float64
# oracle to rtol = atol = 1e-4 (the reference's tf32 path is ~1e-3 off).
# ---------------------------------------------------------------------------

FP32_RTOL = 1e-4
FP32_ATOL = 1e-4
BF16_MAX = 3.38953139e38


def _split_bits_ref(x: torch.Tensor):
    """hi and lo bits of the split, from torch's own bf16 rounding: hi =
    bf16(x) (RNE), or the truncated bits where that would overflow a finite x;
    lo = bf16(x - hi) for finite x, else 0."""
    fin = torch.isfinite(x)
    big = fin & (x.abs() > BF16_MAX)
    hi = torch.where(big, (x.view(torch.int32) >> 16).to(torch.int16), x.to(torch.bfloat16).view(torch.int16))
    hi_f = (hi.to(torch.int32) << 16).view(torch.float32)
    lo = torch.where(fin, x - hi_f, torch.zeros_like(x)).to(torch.bfloat16).view(torch.int16)
    return hi, lo


def _split_on_device(x: torch.Tensor, seg_codes: int):
    from fuseml_amd import _abi

    lib = _abi.load_library()
    rows, K = x.shape
    kp = -(-K // 8) * 8
    dst = torch.full((rows, 3 * kp), 0x7777, dtype=torch.int16, device=x.device)
    rc = lib.fuseml_split_bf16x3(x.data_ptr(), rows, K, x.stride(0), x.stride(1), dst.data_ptr(), 3 * kp, kp,
                                 seg_codes, torch.cuda.current_stream().cuda_stream)
    assert rc == 0, _abi.last_error(lib)
    torch.cuda.synchronize()
    return dst.cpu(), kp


@pytest.mark.parametrize("layout", ["contig", "ragged_k", "strided_k", "transposed", "one_row"])
@pytest.mark.parametrize("seg_codes", ["A", "B"])
def test_split_bf16x3_bit_exact(layout, seg_codes):
    """Segment s of each row holds hi, lo or hf (hi with inf/NaN written as 0)
    as the 2-bit code says: A3 = hi|hf|lo, B3 = hi|lo|hf."""
    from fuseml_amd import _abi

    codes = {"A": _abi.SPLIT_A, "B": _abi.SPLIT_B}[seg_codes]
    g = _gen(60)
    shapes = {"contig": (300, 64), "ragged_k": (37, 100), "strided_k": (41, 3 * 77), "transposed": (56, 33),
              "one_row": (1, 24)}
    base = torch.randn(*shapes[layout], generator=g)
    base = base * torch.exp2(torch.randint(-40, 40, base.shape, generator=g).float())
    specials = [float("inf"), -float("inf"), float("nan"), -0.0, 1e-40, -3e-39, 3.3e38, -3.39e38,
                3.4028235e38, 3.3895314e38, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -9]
    base.view(-1)[: len(specials)] = torch.tensor(specials)
    x = {"strided_k": lambda t: t[:, ::3], "transposed": lambda t: t.t()}.get(layout, lambda t: t)(base)
    print(f"case split layout={layout} codes={seg_codes} shape={tuple(x.shape)} stride={x.stride()}", flush=True)
    got, kp = _split_on_device(x.cuda(), codes)
    hi, lo = _split_bits_ref(x)
    K = x.shape[1]
    nan = torch.isnan(x)
    fin = torch.isfinite(x)
    for seg in range(3):
        part = got[:, seg * kp: seg * kp + K]
        code = (codes >> (2 * seg)) & 3
        if code == _abi.SEG_LO:
            ok = part == lo                                   # lo of inf/NaN is 0
        elif code == _abi.SEG_HI_FINITE:
            ok = torch.where(fin, part == hi, part == 0)      # hf of inf/NaN is 0
        else:
            as_f = (part.to(torch.int32) << 16).view(torch.float32)
            ok = torch.where(nan, torch.isnan(as_f), part == hi)
        assert ok.all(), f"segment {seg}: {(~ok).sum()} of {ok.numel()} differ, e.g. x={x[~ok][:4].tolist()}"
        assert (got[:, seg * kp + K: (seg + 1) * kp] == 0).all(), f"segment {seg} padding"


def test_fp32_graph_capture_replays():
    """An fp32 group is three launches (two splits, then the GEMM) with its
    split buffers from the caching allocator: captured in a HIP graph, each
    replay with new inputs copied in equals an eager launch bit for bit."""
    M, N, K = 600, 1030, 341
    spec = _spec(left=1, right=2, ops=[("add", 0, 1.0), ("gelu_erf", -1, 1.0)], out_dtype=torch.float32)
    L = _launcher(spec, 3)

    def host_inputs(seed):
        a, w = _gemm_inputs(M, N, K, torch.float32, seed=seed)
        return [torch.rand(N, generator=_gen(seed + 2)) - 0.5, a, w.t()]

    print("case fp32 graph capture", flush=True)
    static = [t.cuda() for t in host_inputs(70)]
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        L(*static)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        g_out = L(*static)
    for seed in (71, 72):
        host = host_inputs(seed)
        for dst, src in zip(static, host):
            dst.copy_(src)
        eager = L(*static)
        torch.cuda.synchronize()
        g_out.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(g_out, eager), f"replay seed {seed} differs from eager"
        ref = ora.gemm_epilogue([_np(t) for t in host], 1, 2, [("add", 0, 1.0), ("gelu_erf", -1, 1.0)])["tile"]
        assert np.isclose(_np(g_out), ref, rtol=FP32_RTOL, atol=FP32_ATOL).all()


@pytest.mark.parametrize("shape", [(77, 200, 72), (300, 520, 13)], ids=lambda s: "x".join(map(str, s)))
def test_fp32_group_with_inf_and_nan_operands(shape):
    """Non-finite fp32 GEMM operands give what fp32 gives: +-inf in A and in W
    next to values exact in bf16 (lo = 0, so hi(inf) . lo(b) would be
    inf * 0 = NaN), a NaN in each.  The NaN / +inf / -inf pattern of the fused
    result equals torch fp32's on the CPU exactly (it depends only on which
    products are infinite, not on the summation order); finite values agree
    to 1e-4."""
    M, N, K = shape
    a, w = _gemm_inputs(M, N, K, torch.float32, seed=81)
    # exact in bf16, so their lo part is 0; no exact zeros (0 * inf is NaN in
    # fp32, and a reference that skipped zero products would hide it)
    a[:, ::2] = torch.round(a[:, ::2] * 4) / 4
    a[a == 0] = 0.5
    w[::2, :] = torch.round(w[::2, :] * 8) / 8
    w[w == 0] = -0.125
    a[0, 1] = float("inf")
    a[3, K - 1] = -float("inf")
    a[5, 0] = float("nan")
    w[2, 3 % K] = float("inf")
    w[7, 5 % K] = -float("inf")
    w[11, (K - 2) % K] = float("nan")
    bias = torch.rand(N, generator=_gen(82)) - 0.5
    steps = [("add", 0, 1.0), ("relu", -1, 1.0)]
    spec = _spec(left=1, right=2, ops=steps, out_dtype=torch.float32)
    print(f"case fp32 inf/nan operands shape={shape}", flush=True)
    out = _launcher(spec, 3)(bias.cuda(), a.cuda(), w.t().cuda())
    torch.cuda.synchronize()
    ref = torch.relu(torch.addmm(bias, a, w.t()))      # torch fp32 on the CPU
    got = out.cpu()
    for what, mask in (("nan", torch.isnan), ("+inf", lambda t: t == float("inf")),
                       ("-inf", lambda t: t == -float("inf"))):
        g, r = mask(got), mask(ref)
        assert torch.equal(g, r), f"{what}: {int((g != r).sum())} positions differ, e.g. {torch.nonzero(g != r)[:4].tolist()}"
    assert int(torch.isinf(ref).sum()) > 0 and int(torch.isnan(ref).sum()) > 0
    fin = torch.isfinite(ref)
    assert torch.allclose(got[fin], ref[fin], rtol=FP32_RTOL, atol=FP32_ATOL)


FP32_CHAINS = ["bias_gelu", "act_heavy", "scalars", "bcast_mul", "bias_residual", "sigmoid"]


@pytest.mark.parametrize("chain", FP32_CHAINS)
@pytest.mark.parametrize("shape", [(77, 200, 72), (300, 1000, 136), (130, 257, 48), (512, 520, 1000),
                                   (64, 96, 13)], ids=lambda s: "x".join(map(str, s)))
def test_fp32_chain_parity(chain, shape):
    M, N, K = shape
    dtype = torch.float32
    a, w = _gemm_inputs(M, N, K, dtype, seed=61)
    ops = _operands(M, N, dtype, seed=62)
    inputs = ops + [a, w.t()]
    left, right = len(ops), len(ops) + 1
    steps = CHAINS[chain]
    spec = _spec(left=left, right=right, ops=steps, out_dtype=dtype)
    print(f"case fp32 chain={chain} shape={shape}", flush=True)
    out = _launcher(spec, len(inputs))(*[t.cuda() for t in inputs])
    torch.cuda.synchronize()
    assert out.dtype == torch.float32
    ref = ora.gemm_epilogue([_np(t) for t in inputs], left, right, steps)["tile"]
    got = _np(out)
    bad = ~np.isclose(got, ref, rtol=FP32_RTOL, atol=FP32_ATOL)
    assert not bad.any(), f"{chain} {shape}: {bad.sum()} mismatches, max err {np.abs(got - ref).max():.3g}"


@pytest.mark.parametrize("forced_variant", ["auto", "large", "deep3"], indirect=True)
def test_fp32_reductions_and_escape(forced_variant):
    """fp32 group with an escape store (bf16) and row reductions, on the
    256-wide variants too (K' = 3 * 344 = 1032 for K = 341)."""
    M, N, K = 600, 1030, 341
    a, w = _gemm_inputs(M, N, K, torch.float32, seed=63)
    bias = torch.rand(N, generator=_gen(64)) - 0.5
    steps = [("add", 0, 1.0), ("store", 0, 1.0), ("gelu_erf", -1, 1.0)]
    spec = _spec(left=1, right=2, ops=steps, out_dtype=torch.float32, store_tile=True,
                 reductions=("sum", "amax", "mean"), reduce_axis=1, reduce_dtypes=(torch.float32,) * 3,
                 extra_dtypes=(torch.bfloat16,),
                 outputs=(("tile",), ("extra", 0), ("red", "sum"), ("red", "amax"), ("red", "mean")))
    print(f"case fp32 reductions variant={forced_variant}", flush=True)
    tile, pre, s, mx, mean = _launcher(spec, 3)(bias.cuda(), a.cuda(), w.t().cuda())
    torch.cuda.synchronize()
    ref = ora.gemm_epilogue([_np(bias), _np(a), _np(w.t())], 1, 2, steps, ("sum", "amax", "mean"), 1, n_extra=1)
    v = ref["tile"]
    assert np.isclose(_np(tile), v, rtol=FP32_RTOL, atol=FP32_ATOL).all()
    _check_tile(pre, ref["extra"][0], "bf16 escape of an fp32 group")
    for got, key, scale in ((s, "sum", np.abs(v).sum(1)), (mx, "amax", np.abs(v).max(1)),
                            (mean, "mean", np.abs(v).mean(1))):
        err = np.abs(_np(got) - ref[key])
        assert (err <= FP32_RTOL * np.maximum(np.abs(ref[key]), 1e-3 * scale) + 1e-6).all(), key


# ---------------------------------------------------------------------------
# Full-size configurations, checked at sampled rows
# ---------------------------------------------------------------------------


def _sample_rows(M, n=48, seed=0):
    rng = np.random.default_rng(seed)
    rows = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, n)]))
    return rows


def test_c2_full_size_sampled_rows():
    """C2 at full size: G1 (K=1024, 1024 tiles) on the ping-pong schedule over
    four rounds, G2 (K=4096, 256 tiles, residual) on the one-wave whole-stage
    schedule, one tile per workgroup."""
    from fuseml_amd.workloads import c2_mlp_block

    wl = c2_mlp_block()
    m = wl.model
    x = wl.inputs[0]
    W1, b1, W2, b2 = m.linear1.weight, m.linear1.bias, m.linear2.weight, m.linear2.bias
    g1 = _launcher(_spec(left=1, right=2, ops=[("add", 0, 1.0), ("gelu_erf",)], out_dtype=x.dtype), 3)
    g2 = _launcher(_spec(left=1, right=2, ops=[("add", 0, 1.0), ("add", 3, 1.0)], out_dtype=x.dtype), 4)
    xd = x.cuda()
    h = g1(b1.cuda(), xd, W1.t().cuda())
    y = g2(b2.cuda(), h, W2.t().cuda(), xd)
    torch.cuda.synchronize()
    rows = _sample_rows(x.shape[0])
    ref = ora_w.transformer_mlp(_np(x), _np(W1), _np(b1), _np(W2), _np(b2), rows=rows)
    _check_tile(y[torch.as_tensor(rows).cuda()], ref, "C2 block")
    # h is an exact bf16 round of G1; check it too
    ref_h = ora.gelu_erf(ora_w.linear(_np(x)[rows], _np(W1), _np(b1)))
    _check_tile(h[torch.as_tensor(rows).cuda()], ref_h, "C2 G1")


def test_c5_block_full_size_sampled_rows():
    """One C5 block at full size: G1 (K=4096, 2048 tiles) and G2 (K=16384, 512
    tiles, residual) both on the one-wave whole-stage schedule, several tiles
    per workgroup."""
    from fuseml_amd.workloads import c5_stacked_mlp

    wl = c5_stacked_mlp(num_blocks=1)
    blk = wl.model.blocks[0]
    x = wl.inputs[0]
    W1, b1, W2, b2 = blk.linear1.weight, blk.linear1.bias, blk.linear2.weight, blk.linear2.bias
    g1 = _launcher(_spec(left=1, right=2, ops=[("add", 0, 1.0), ("gelu_erf",)], out_dtype=x.dtype), 3)
    g2 = _launcher(_spec(left=1, right=2, ops=[("add", 0, 1.0), ("add", 3, 1.0)], out_dtype=x.dtype), 4)
    print("case C5 block full size", flush=True)
    xd = x.cuda()
    h = g1(b1.cuda(), xd, W1.t().cuda())
    y = g2(b2.cuda(), h, W2.t().cuda(), xd)
    torch.cuda.synchronize()
    rows = _sample_rows(x.shape[0], n=24, seed=5)
    ref = ora_w.transformer_mlp(_np(x), _np(W1), _np(b1), _np(W2), _np(b2), rows=rows)
    _check_tile(y[torch.as_tensor(rows).cuda()], ref, "C5 block")
    ref_h = ora.gelu_erf(ora_w.linear(_np(x)[rows], _np(W1), _np(b1)))
    _check_tile(h[torch.as_tensor(rows).cuda()], ref_h, "C5 G1")


def test_same_signature_aligned_then_misaligned_operand():
    """One launch plan serves every call with the same shapes, strides and
    dtypes; the operands' base alignment is checked per call.  The second call
    passes A as a view 2 bytes off a 16-byte boundary (same strides, same
    plan): the launcher copies it to an aligned buffer and the result still
    matches the oracle, as does a W whose view starts 2 bytes in."""
    M, N, K = 300, 520, 136
    dtype = torch.bfloat16
    steps = CHAINS["bias_gelu"]
    spec = _spec(left=1, right=2, ops=steps, out_dtype=dtype)
    L = _launcher(spec, 3)
    bias = (torch.rand(N, generator=_gen(95)) - 0.5).to(dtype)
    print("case aligned then misaligned operands", flush=True)
    for shift in (0, 1):
        big_a = torch.randn(M, K + 8, generator=_gen(96 + shift)).to(dtype)
        big_w = (torch.randn(N, K + 8, generator=_gen(98 + shift)) / K ** 0.5).to(dtype)
        a_dev, w_dev = big_a.cuda()[:, shift:shift + K], big_w.cuda()[:, shift:shift + K]
        assert (a_dev.data_ptr() % 16 == 0) == (shift == 0)
        out = L(bias.cuda(), a_dev, w_dev.t())
        torch.cuda.synchronize()
        host = [bias, big_a[:, shift:shift + K], big_w[:, shift:shift + K].t()]
        ref = ora.gemm_epilogue([_np(t) for t in host], 1, 2, steps)["tile"]
        _check_tile(out, ref, f"shift {shift}")
    assert len(L._plans) == 1 and L.launch_count == 2
