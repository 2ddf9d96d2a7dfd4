"""GPU parity at the benchmark configs' full shapes, and the boundary cases that
need real sizes: the reference's own FusionGroup on the device, NaN
propagation, operands beyond 2 GiB.

Every config runs at exactly its benchmark shape, so the kernel variant and the
number of persistent rounds are the ones the benchmark measures (C3: 1024
tiles of 256x256 on the ping-pong schedule; C4: 1024 tiles, K=2048, the
one-wave whole-stage schedule, a stored tile plus three fp32 row reductions;
C5: four chained blocks).  Rows are independent in every workload, so the
float64 oracle checks tiles at sampled rows; C4's reductions are [8192] and
are all checked.

Tolerances: 16-bit tiles ``allclose(rtol=2e-2, atol=2e-2)`` against the
float64 oracle; fp32 reductions ``|got - ref| <= 1e-2 * |ref|`` with a floor of
1e-2 * 1e-3 * (the same reduction of |v|) for values that cancel to near zero.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from oracle import gemm_epilogue as ora
from oracle import workloads as ora_w

pytestmark = pytest.mark.gpu

RTOL = ATOL = 2e-2
RED_RTOL = 1e-2
RED_FLOOR = 1e-3


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _case(msg):
    print(f"case {msg}", flush=True)


def _close(got, ref, what):
    g = _np(got)
    assert g.shape == ref.shape, (what, g.shape, ref.shape)
    bad = ~np.isclose(g, ref, rtol=RTOL, atol=ATOL)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} mismatches, max err {np.abs(g - ref).max()}"


def _red_close(got, ref, ref_abs, what):
    g = _np(got)
    assert g.shape == ref.shape, (what, g.shape, ref.shape)
    tol = RED_RTOL * np.maximum(np.abs(ref), RED_FLOOR * ref_abs)
    err = np.abs(g - ref)
    assert (err <= tol).all(), f"{what}: max err {err.max()} at {err.argmax()} (tol there {tol[err.argmax()]})"


def _rows(M, n=64, seed=0):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, n)]))


def _launcher(spec, n):
    from fuseml_amd.launcher import HipKernelLauncher

    return HipKernelLauncher(spec, n)


def _launched(L):
    """(BM, BN, waves) and the epilogue chain id of the launcher's (single) plan:
    what its launches ran."""
    from fuseml_amd import _abi

    lib = _abi.load_library()
    (plan,) = L._plans.values()
    cfg = (ctypes.c_int32 * 4)()
    assert lib.fuseml_gemm_epilogue_config(ctypes.byref(plan.desc), cfg) == 0
    return tuple(cfg[:3]), lib.fuseml_gemm_epilogue_chain(ctypes.byref(plan.desc))


def _compile(model, **kw):
    from fuseml_amd.compiler import FuseMLCompiler

    torch._dynamo.reset()
    be = FuseMLCompiler(**kw)
    return torch.compile(model, backend=be), be


# ---------------------------------------------------------------------------
# C3 at 16384 x 1024 -> 4096 with the full [16384, 4096] gate
# ---------------------------------------------------------------------------


def _c3_ref(wl, rows):
    m = wl.model
    x, g = wl.inputs
    return ora_w.activation_heavy(_np(x), _np(m.linear.weight), _np(m.linear.bias), _np(g), _np(m.row), rows=rows)


def test_c3_full_size_launcher():
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp
    from fuseml_amd.workloads import c3_activation_heavy

    _case("C3 full size, launcher")
    wl = c3_activation_heavy()
    m = wl.model
    x, g = wl.inputs
    spec = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("relu"), EpiOp("mul", 3), EpiOp("sigmoid"),
                               EpiOp("add", 4)), torch.bfloat16)
    L = _launcher(spec, 5)
    with torch.no_grad():
        y = L(m.linear.bias.cuda(), x.cuda(), m.linear.weight.t().cuda(), g.cuda(), m.row.cuda())
    torch.cuda.synchronize()
    # one-wave whole-stage variant, 4 rounds of 256 tiles, the act-heavy fixed chain
    assert _launched(L) == ((256, 256, 4), 7)
    rows = _rows(16384)
    _close(y[torch.as_tensor(rows).cuda()], _c3_ref(wl, rows), "C3")


def test_c3_full_size_compiled():
    from fuseml_amd.workloads import c3_activation_heavy

    _case("C3 full size, torch.compile(backend=FuseMLCompiler())")
    wl = c3_activation_heavy()
    rows = _rows(16384, seed=1)
    ref = _c3_ref(wl, rows)
    wl.to("cuda")
    compiled, be = _compile(wl.model)
    with torch.no_grad():
        y = compiled(*wl.inputs)
    torch.cuda.synchronize()
    assert be.fusion_strategy == "hip" and len(be.launchers) == 1
    _close(y[torch.as_tensor(rows).cuda()], ref, "C3 compiled")


# ---------------------------------------------------------------------------
# C4 at 8192 x 8192 x 2048: tile + three fp32 row reductions, all 8192 checked
# ---------------------------------------------------------------------------


@pytest.fixture(scope="module")
def c4_oracle():
    from fuseml_amd.workloads import c4_gemm_row_reductions

    wl = c4_gemm_row_reductions()
    ref = ora_w.gemm_row_reductions(_np(wl.inputs[0]), _np(wl.model.linear.weight))
    a = np.abs(ref["tile"])
    scales = {"sum": a.sum(1), "amax": a.max(1), "mean": a.mean(1)}
    return wl, ref, scales


def _check_c4(h, s, mx, mean, ref, scales, what):
    rows = _rows(8192, seed=2)
    _close(h[torch.as_tensor(rows).cuda()], ref["tile"][rows], f"{what} tile")
    for got, key in ((s, "sum"), (mx, "amax"), (mean, "mean")):
        assert got.dtype == torch.float32 and got.shape == (8192,)
        _red_close(got, ref[key], scales[key], f"{what} {key}")


def test_c4_full_size_launcher(c4_oracle):
    """The bench's spec on its production variant: one-wave whole-stage K loop,
    4 persistent rounds."""
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp

    _case("C4 full size, launcher (deep3, 4 rounds)")
    wl, ref, scales = c4_oracle
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), torch.bfloat16, store_tile=True,
                        reductions=("sum", "amax", "mean"), reduce_axis=1,
                        reduce_dtypes=(torch.float32,) * 3,
                        outputs=(("red", "sum"), ("red", "amax"), ("red", "mean"), ("tile",)))
    L = _launcher(spec, 2)
    with torch.no_grad():
        s, mx, mean, h = L(wl.inputs[0].cuda(), wl.model.linear.weight.t().cuda())
    torch.cuda.synchronize()
    assert _launched(L) == ((256, 256, 4), 8)  # deep3, the ReLU (+ reductions) fixed chain
    _check_c4(h, s, mx, mean, ref, scales, "C4")


def test_c4_full_size_compiled_sibling_reductions(c4_oracle):
    _case("C4 full size, FuseMLCompiler(fuse_sibling_reductions=True)")
    wl, ref, scales = c4_oracle
    model = wl.model.cuda()
    x = wl.inputs[0].cuda()
    compiled, be = _compile(model, fuse_sibling_reductions=True)
    with torch.no_grad():
        h, s, mx, mean = compiled(x)
    torch.cuda.synchronize()
    assert be.fusion_strategy == "hip" and len(be.launchers) == 1
    assert be.launchers[0].spec.reductions == ("sum", "amax", "mean")
    _check_c4(h, s, mx, mean, ref, scales, "C4 compiled")
    wl.model.cpu()


# ---------------------------------------------------------------------------
# C5: all four blocks chained at 8192 x 4096 (16384 hidden)
# ---------------------------------------------------------------------------


def test_c5_four_blocks_chained():
    from fuseml_amd.workloads import c5_stacked_mlp

    _case("C5 full size, 4 blocks chained (compiled)")
    wl = c5_stacked_mlp()
    blocks = [(_np(b.linear1.weight), _np(b.linear1.bias), _np(b.linear2.weight), _np(b.linear2.bias))
              for b in wl.model.blocks]
    rows = _rows(8192, n=24, seed=5)
    ref = ora_w.stacked_mlp(_np(wl.inputs[0]), blocks, rows=rows)
    wl.to("cuda")
    # the fused kernels under test (the default cost model sends these long-K
    # groups to eager, whose GEMM is faster at K >= 4096)
    compiled, be = _compile(wl.model, k_per_epilogue_pass=0)
    with torch.no_grad():
        y = compiled(*wl.inputs)
    torch.cuda.synchronize()
    assert be.fusion_strategy == "hip"
    assert sum(l.launch_count for l in {id(l): l for l in be.launchers}.values()) == 8
    _close(y[torch.as_tensor(rows).cuda()], ref, "C5 4 blocks")


# ---------------------------------------------------------------------------
# The reference's FusionGroup, through the reference's surgery, on the device
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("cublas", [False, True], ids=["triton", "cublas_epilogue"])
def test_reference_route_reference_groups_on_gpu(cublas):
    from torch.fx.experimental.proxy_tensor import make_fx

    from fuseml_amd.compiler import build_hip_launcher
    from fuseml_amd.launcher import HipKernelLauncher
    from fuseml_amd.workloads import c2_mlp_block
    from refsurgery import bind, reference_groups, reference_surgery

    _case(f"reference-route groups cublas={cublas}")
    wl = c2_mlp_block(scale=1 / 8)  # x[2048, 1024]
    m = wl.model
    x = wl.inputs[0]
    ref = ora_w.transformer_mlp(_np(x), _np(m.linear1.weight), _np(m.linear1.bias),
                                _np(m.linear2.weight), _np(m.linear2.bias))
    m = m.cuda()
    xd = x.cuda()
    with torch.no_grad():
        gm = make_fx(m)(xd)
    groups = reference_groups(gm, (xd,), cublas=cublas)
    bound = bind(gm, reference_surgery(gm, groups), build_hip_launcher)
    assert all(isinstance(b, HipKernelLauncher) for b in bound)
    with torch.no_grad():
        y = gm(xd)
    torch.cuda.synchronize()
    assert [b.launch_count for b in bound] == [1, 1] and [b.fallback_count for b in bound] == [0, 0]
    _close(y, ref, "reference-route C2 block")


# ---------------------------------------------------------------------------
# NaN propagation (torch semantics: relu, amax, fp16 saturation keep NaN)
# ---------------------------------------------------------------------------


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16], ids=["bf16", "fp16"])
def test_nan_propagates_like_eager(out_dtype):
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp

    _case(f"NaN propagation {out_dtype}")
    M, N, K = 600, 1024, 256
    g = torch.Generator().manual_seed(51)
    a = torch.randn(M, K, generator=g).to(out_dtype)
    w = (torch.randn(N, K, generator=g) / 16).to(out_dtype)
    r = torch.randn(M, N, generator=g).to(out_dtype)
    a[7, 3] = float("nan")            # row 7 of the product is NaN
    r[100, 5] = float("nan")          # one element of the residual
    spec = EpilogueSpec(0, 1, (EpiOp("relu"), EpiOp("add", 2), EpiOp("scale", scalar=4.0e4)), out_dtype,
                        store_tile=True, reductions=("sum", "amax"), reduce_axis=1,
                        reduce_dtypes=(torch.float32,) * 2,
                        outputs=(("tile",), ("red", "sum"), ("red", "amax")))
    tile, s, mx = _launcher(spec, 3)(a.cuda(), w.t().cuda(), r.cuda())
    torch.cuda.synchronize()
    v = (torch.relu(a.float() @ w.float().t()) + r.float()) * 4.0e4
    assert torch.equal(torch.isnan(tile.cpu()), torch.isnan(v))
    assert torch.isnan(mx[7]) and torch.isnan(mx[100]) and torch.isnan(s[7]) and torch.isnan(s[100])
    finite = ~torch.isnan(v).any(1)
    assert not torch.isnan(mx.cpu()[finite]).any()
    if out_dtype == torch.float16:  # saturation still applies to the finite values
        assert (tile.cpu()[finite].abs() <= 65504).all()


# ---------------------------------------------------------------------------
# Operands beyond 2 GiB (buffer resources based at each tile's origin)
# ---------------------------------------------------------------------------


def test_tile_operand_and_output_beyond_2gib():
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp

    M, N, K = 36864, 32768, 64          # residual and output: 2.4 GB each
    _case(f"residual/output beyond 2 GiB {M}x{N}x{K}")
    g = torch.Generator().manual_seed(61)
    a = torch.randn(M, K, generator=g).to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g) / 8).to(torch.bfloat16)
    rows = _rows(M, n=16, seed=6)
    r = torch.empty(M, N, dtype=torch.bfloat16, device="cuda")
    r.copy_(torch.arange(N, dtype=torch.float32, device="cuda").remainder(17).sub(8).mul(0.125).expand(M, N))
    spec = EpilogueSpec(0, 1, (EpiOp("add", 2),), torch.bfloat16)
    y = _launcher(spec, 3)(a.cuda(), w.t().cuda(), r)
    torch.cuda.synchronize()
    ref = ora.gemm(_np(a)[rows], _np(w).T) + _np(r[torch.as_tensor(rows).cuda()])
    _close(y[torch.as_tensor(rows).cuda()], ref, "beyond 2 GiB")
    del r, y
    torch.cuda.empty_cache()


def test_gemm_operand_beyond_2gib():
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp

    M, N, K = 131072, 256, 8704          # A: 2.28 GB
    _case(f"A operand beyond 2 GiB {M}x{N}x{K}")
    g = torch.Generator(device="cuda").manual_seed(62)
    a = torch.randn(M, K, generator=g, device="cuda").to(torch.bfloat16)
    w = (torch.randn(N, K, generator=g, device="cuda") / 64).to(torch.bfloat16)
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), torch.bfloat16)
    y = _launcher(spec, 2)(a, w.t())
    torch.cuda.synchronize()
    rows = _rows(M, n=16, seed=7)
    ri = torch.as_tensor(rows).cuda()
    ref = ora.relu(ora.gemm(_np(a[ri]), _np(w).T))
    _close(y[ri], ref, "A beyond 2 GiB")
    del a, y
    torch.cuda.empty_cache()
