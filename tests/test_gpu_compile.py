"""End to end on the GPU: torch.compile(model, backend=FuseMLCompiler()).

Each workload (benchmark configs C1-C5; M scaled down so the float64 oracle
stays fast, every other dimension at full size) is compiled, run under
no_grad, and compared with the CPU oracle on the same bf16 inputs.  The test
also asserts that the fused HIP launchers actually ran (no silent eager path).
Tolerances: tiles rtol/atol 2e-2; fp32 reductions 1e-2 of |ref| (floored at
1e-3 of the same reduction of |v|, for sums that cancel).
"""

import numpy as np
import pytest
import torch

from oracle import workloads as ora_w

pytestmark = pytest.mark.gpu


def _f64(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _compile(model, **kw):
    from fuseml_amd.compiler import FuseMLCompiler

    torch._dynamo.reset()
    # The workloads are scaled down (fewer output tiles than CUs at K >= 2048 for
    # some GEMMs), and the long-K groups lose to eager's GEMM, so the cost
    # model would route them to eager: keep the fused kernels under test.
    kw.setdefault("min_tiles_long_k", 0)
    kw.setdefault("k_per_epilogue_pass", 0)  # long-K groups would route to eager
    be = FuseMLCompiler(**kw)
    return torch.compile(model, backend=be), be


def _launches(be):
    """Kernel launches made by the backend's launchers (a cached launcher counts once)."""
    uniq = {id(l): l for l in be.launchers}
    return sum(getattr(l, "launch_count", 0) for l in uniq.values())


def _close(got, ref, what):
    g = _f64(got)
    bad = ~np.isclose(g, ref, rtol=2e-2, atol=2e-2)
    assert not bad.any(), f"{what}: {bad.sum()} mismatches, max err {np.abs(g - ref).max()}"


def test_few_tiles_long_k_is_routed_to_eager():
    """Cost model on the device: Linear(4096 -> 1024) + GELU at M=1024 has 64
    output tiles of 128x128 (256 of the 32x128 tiles it would run on, 160
    operand rows per CU) at K=4096, over the rows x K budget, so the group runs
    eager; with the few-tile rule off (min_tiles_long_k=0) the same module is
    fused, and both match eager.  At K=2048 the default fuses it."""
    from fuseml_amd.compiler import MIN_TILES_LONG_K

    gen = torch.Generator().manual_seed(3)
    for K, fused_by_default in ((4096, False), (2048, True)):
        lin = torch.nn.Linear(K, 1024).to(torch.bfloat16)
        m = torch.nn.Sequential(lin, torch.nn.GELU()).to("cuda")
        x = torch.randn(1024, K, generator=gen).to(torch.bfloat16).to("cuda")
        print(f"case few-tile Linear({K} -> 1024) + GELU at M=1024", flush=True)
        with torch.no_grad():
            ref = m(x)
            compiled, be = _compile(m, min_tiles_long_k=MIN_TILES_LONG_K)
            out = compiled(x)
        assert bool(be.launchers) == fused_by_default and be.fusion_applied == fused_by_default
        _close(out, _f64(ref), f"default-routed Linear({K})+GELU")
        with torch.no_grad():
            compiled, be = _compile(m)
            out = compiled(x)
        assert be.fusion_applied and _launches(be) == 1
        _close(out, _f64(ref), f"fused Linear({K})+GELU")


class _NegReluAmax(torch.nn.Module):
    def __init__(self, w):
        super().__init__()
        self.w = torch.nn.Parameter(w, requires_grad=False)

    def forward(self, x):
        return (torch.relu(x @ self.w.t()) * -1).amax(-1)


def test_compiled_amax_of_negated_relu():
    """(relu(x @ W.T) * -1).amax(-1) under the default cost model: default
    discovery forms one group mm -> relu -> mul(-1) -> amax (three eager
    passes at K = 1024, so it fuses).  Every value is <= 0 and relu's +0
    becomes -0.0, so each row maximum is -0.0 (row 7 of x is zero: that whole
    row is -0.0); the fused amax must return -0.0 there, not -inf or the
    largest strictly negative value."""
    from fuseml_amd.compiler import FuseMLCompiler

    gen = torch.Generator().manual_seed(71)
    x = torch.randn(1024, 1024, generator=gen).to(torch.bfloat16)
    x[7] = 0
    w = (torch.randn(2048, 1024, generator=gen) / 32).to(torch.bfloat16)
    m = _NegReluAmax(w).to("cuda")
    xd = x.to("cuda")
    torch._dynamo.reset()
    be = FuseMLCompiler()
    compiled = torch.compile(m, backend=be)
    with torch.no_grad():
        got = compiled(xd)
        eager = m(xd)
    torch.cuda.synchronize()
    assert be.fusion_applied and len(be.launchers) == 1 and _launches(be) == 1
    assert be.launchers[0].spec.reductions == ("amax",)
    ref = (-np.maximum(_f64(x) @ _f64(w).T, 0.0)).max(axis=1)
    g = _f64(got)
    assert np.isfinite(g).all(), f"rows with -inf: {np.argwhere(~np.isfinite(g)).ravel()[:8]}"
    assert np.allclose(g, ref, rtol=2e-2, atol=2e-2)
    assert torch.equal(got.float(), eager.float())
    assert g[7] == 0.0 and np.signbit(g[7])


def test_c1_fp32_small_compiled():
    """C1 (fp32, 64 rows): with the calibrated cost model its one group
    (addmm + GELU(tanh); the second addmm has no op after it, so it is no
    group) fuses as a split product and matches eager fp32 to 1e-4; the
    reference's tiny-output rule (min_output_elements=500 000) bypasses it
    instead."""
    from fuseml_amd.compiler import REFERENCE_MIN_OUTPUT_ELEMENTS
    from fuseml_amd.workloads import c1_transformer_mlp_small

    wl = c1_transformer_mlp_small().to("cuda")
    compiled, be = _compile(wl.model)
    with torch.no_grad():
        out = compiled(*wl.inputs)
        ref = wl.model(*wl.inputs)
    torch.cuda.synchronize()
    assert be.fusion_applied and be.fusion_strategy == "hip" and _launches(be) == 1
    assert torch.allclose(out, ref, rtol=1e-4, atol=1e-4)
    compiled, be = _compile(wl.model, min_output_elements=REFERENCE_MIN_OUTPUT_ELEMENTS)
    with torch.no_grad():
        out = compiled(*wl.inputs)
    assert be.fusion_applied is False
    assert torch.allclose(out, ref)


def test_c2_mlp_block_compiled():
    from fuseml_amd.workloads import c2_mlp_block

    wl = c2_mlp_block(scale=1 / 8).to("cuda")  # x[2048,1024]
    compiled, be = _compile(wl.model)
    with torch.no_grad():
        y = compiled(*wl.inputs)
        y = compiled(*wl.inputs)
    torch.cuda.synchronize()
    assert be.fusion_applied and be.fusion_strategy == "hip"
    assert len(be.launchers) == 2 and _launches(be) == 4
    m = wl.model
    x = wl.inputs[0]
    ref = ora_w.transformer_mlp(_f64(x), _f64(m.linear1.weight), _f64(m.linear1.bias),
                                _f64(m.linear2.weight), _f64(m.linear2.bias))
    _close(y, ref, "C2")


def test_c3_activation_heavy_compiled():
    from fuseml_amd.workloads import c3_activation_heavy

    wl = c3_activation_heavy(scale=1 / 8).to("cuda")
    compiled, be = _compile(wl.model)
    with torch.no_grad():
        y = compiled(*wl.inputs)
    torch.cuda.synchronize()
    assert be.fusion_applied and len(be.launchers) == 1 and _launches(be) == 1
    m = wl.model
    x, g = wl.inputs
    ref = ora_w.activation_heavy(_f64(x), _f64(m.linear.weight), _f64(m.linear.bias), _f64(g), _f64(m.row))
    _close(y, ref, "C3")


def test_c4_row_reductions_compiled_with_sibling_fusion():
    from fuseml_amd.workloads import c4_gemm_row_reductions

    wl = c4_gemm_row_reductions(scale=1 / 8).to("cuda")  # x[1024,2048] -> [1024,8192]
    compiled, be = _compile(wl.model, fuse_sibling_reductions=True)
    with torch.no_grad():
        h, s, mx, mean = compiled(*wl.inputs)
    torch.cuda.synchronize()
    assert be.fusion_applied and len(be.launchers) == 1 and _launches(be) == 1
    ref = ora_w.gemm_row_reductions(_f64(wl.inputs[0]), _f64(wl.model.linear.weight))
    _close(h, ref["tile"], "C4 tile")
    a = np.abs(ref["tile"])
    for got, key, scale in ((s, "sum", a.sum(1)), (mx, "amax", a.max(1)), (mean, "mean", a.mean(1))):
        assert got.dtype == torch.float32
        g = _f64(got)
        assert np.all(np.abs(g - ref[key]) <= 1e-2 * np.maximum(np.abs(ref[key]), 1e-3 * scale) + 1e-7), key


def test_c4_default_discovery_matches_reference_grouping():
    from fuseml_amd.workloads import c4_gemm_row_reductions

    wl = c4_gemm_row_reductions(scale=1 / 8).to("cuda")
    compiled, be = _compile(wl.model)
    with torch.no_grad():
        h, s, mx, mean = compiled(*wl.inputs)
        rh, rs, rmx, rmean = wl.model(*wl.inputs)
    torch.cuda.synchronize()
    assert len(be.launchers) == 1  # mm + relu only, reductions stay eager (reference behaviour)
    assert be.launchers[0].spec.reductions == ()
    _close(h, _f64(rh), "C4 tile vs eager")


def test_compiled_c4_replays_in_a_hip_graph():
    """The compiled module (fused GEMM + ReLU + three row reductions) captured
    in a HIP graph: every replay, after a new input is copied in and with an
    eager call of the compiled module between replays, matches that eager
    call (tile and amax bit for bit, sum and mean to 1e-5 relative)."""
    from fuseml_amd.workloads import c4_gemm_row_reductions

    wl = c4_gemm_row_reductions(scale=1 / 8).to("cuda")  # x[1024,2048] -> [1024,8192]
    compiled, be = _compile(wl.model, fuse_sibling_reductions=True)
    x = wl.inputs[0].clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.no_grad(), torch.cuda.stream(side):
        compiled(x)  # compile and build the launch plan outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.no_grad(), torch.cuda.graph(graph):
        outs = compiled(x)
    assert be.fusion_applied and len(be.launchers) == 1
    gen = torch.Generator().manual_seed(9)
    for i in range(3):
        x.copy_(torch.randn(x.shape, generator=gen).to(x.dtype))
        with torch.no_grad():
            eager = compiled(x)
        torch.cuda.synchronize()
        for o in outs:
            o.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for name, g, e in zip(("tile", "sum", "amax", "mean"), outs, eager):
            if name in ("tile", "amax"):
                assert torch.equal(g, e), f"replay {i}: {name} differs from the eager call"
            else:
                assert torch.allclose(g, e, rtol=1e-5, atol=1e-5), f"replay {i}: {name}"


def test_fp32_mlp_compiled_as_split_products():
    """An fp32 TransformerMLP (x[2048,1024] -> 4096 -> 1024): both groups fuse,
    each GEMM as one bf16 launch over the split operands; the result matches
    the float64 oracle to 1e-4 (eager fp32 is also within that)."""
    from fuseml_amd.workloads import TransformerMLP

    torch.manual_seed(5)
    m = TransformerMLP(1024, 4096).eval().to("cuda")
    x = torch.randn(2048, 1024, generator=torch.Generator().manual_seed(6)).to("cuda")
    compiled, be = _compile(m)
    with torch.no_grad():
        y = compiled(x)
        eager = m(x)
    torch.cuda.synchronize()
    assert be.fusion_applied and len(be.launchers) == 2 and _launches(be) == 2
    assert y.dtype == torch.float32
    ref = ora_w.transformer_mlp(_f64(x), _f64(m.linear1.weight), _f64(m.linear1.bias),
                                _f64(m.linear2.weight), _f64(m.linear2.bias))
    for got, what in ((y, "fused fp32"), (eager, "eager fp32")):
        g = _f64(got)
        assert np.allclose(g, ref, rtol=1e-4, atol=1e-4), f"{what}: max err {np.abs(g - ref).max()}"


def test_c5_stacked_compiled_two_blocks():
    from fuseml_amd.workloads import c5_stacked_mlp

    wl = c5_stacked_mlp(scale=1 / 16, num_blocks=2).to("cuda")  # x[512,4096]
    compiled, be = _compile(wl.model)
    with torch.no_grad():
        y = compiled(*wl.inputs)
    torch.cuda.synchronize()
    assert be.fusion_applied and _launches(be) == 4
    blocks = [(_f64(b.linear1.weight), _f64(b.linear1.bias), _f64(b.linear2.weight), _f64(b.linear2.bias))
              for b in wl.model.blocks]
    rows = np.arange(0, 512, 16)
    ref = ora_w.stacked_mlp(_f64(wl.inputs[0]), blocks, rows=rows)
    _close(y[torch.as_tensor(rows).cuda()], ref, "C5")


def test_forced_fallback_on_gpu(monkeypatch):
    from fuseml_amd.fallback import FORCE_FAIL_ENV
    from fuseml_amd.workloads import c2_mlp_block

    wl = c2_mlp_block(scale=1 / 8).to("cuda")
    compiled, be = _compile(wl.model)
    with torch.no_grad():
        compiled(*wl.inputs)
        monkeypatch.setenv(FORCE_FAIL_ENV, "1")
        y = compiled(*wl.inputs)
        ref = wl.model(*wl.inputs)
    torch.cuda.synchronize()
    assert sum(l.fallback_count for l in {id(l): l for l in be.launchers}.values()) == 2
    assert torch.equal(y, ref)


# ---------------------------------------------------------------------------
# 3-D activations (FuseMLCompiler(fuse_leading_views=True)): x[B,S,D] through
# nn.Linear lowers to view -> addmm -> view -> pointwise.
# ---------------------------------------------------------------------------


def test_c2_mlp_block_3d_activations():
    from fuseml_amd.workloads import c2_mlp_block

    wl = c2_mlp_block(scale=1 / 8).to("cuda")      # x[2048,1024] -> [4,512,1024]
    x3 = wl.inputs[0].view(4, 512, 1024)
    compiled, be = _compile(wl.model, fuse_leading_views=True)
    with torch.no_grad():
        y = compiled(x3)
    torch.cuda.synchronize()
    assert be.fusion_applied and be.fusion_strategy == "hip"
    assert len(be.launchers) == 2 and _launches(be) == 2
    assert y.shape == (4, 512, 1024)
    m = wl.model
    ref = ora_w.transformer_mlp(_f64(wl.inputs[0]), _f64(m.linear1.weight), _f64(m.linear1.bias),
                                _f64(m.linear2.weight), _f64(m.linear2.bias))
    _close(y.reshape(2048, 1024), ref, "C2 3-D")


class _Gated3D(torch.nn.Module):
    """relu(l(x)) * g + r with a per-batch gate g[B,1,N] (no single stride over
    the flattened rows: the launcher materialises it) and a row r[N]; then the
    last-dimension sum of the result as a second group."""

    def __init__(self, d, n):
        super().__init__()
        self.l = torch.nn.Linear(d, n)
        self.l2 = torch.nn.Linear(d, n)

    def forward(self, x, g, r):
        y = torch.relu(self.l(x)) * g + r
        s = torch.sigmoid(self.l2(x)).sum(-1)
        return y, s


def test_3d_broadcast_operands_and_last_dim_reduction():
    B, S, D, N = 4, 256, 512, 768
    gen = torch.Generator().manual_seed(31)
    m = _Gated3D(D, N).to(torch.bfloat16)
    x = torch.randn(B, S, D, generator=gen).to(torch.bfloat16)
    g = torch.rand(B, 1, N, generator=gen).to(torch.bfloat16)
    r = (torch.rand(N, generator=gen) - 0.5).to(torch.bfloat16)
    m, x, g, r = m.cuda(), x.cuda(), g.cuda(), r.cuda()
    compiled, be = _compile(m, fuse_leading_views=True, min_output_elements=0)
    with torch.no_grad():
        y, s = compiled(x, g, r)
    torch.cuda.synchronize()
    assert be.fusion_applied and _launches(be) == 2
    assert y.shape == (B, S, N) and s.shape == (B, S)
    W, b = _f64(m.l.weight), _f64(m.l.bias)
    h = np.maximum(_f64(x) @ W.T + b, 0.0)
    _close(y, h * _f64(g) + _f64(r), "gated 3-D")
    v = 1.0 / (1.0 + np.exp(-(_f64(x) @ _f64(m.l2.weight).T + _f64(m.l2.bias))))
    ref_s = v.sum(-1)
    err = np.abs(_f64(s) - ref_s)
    assert (err <= 1e-2 * np.maximum(np.abs(ref_s), 1e-3 * np.abs(v).sum(-1))).all(), err.max()
