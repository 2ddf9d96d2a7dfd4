"""FuseMLCompiler backend plumbing on the CPU (no kernel launches).

* Without a gfx950 device the backend bypasses (the reference's
  _NoFusionPossible path, fuseml/compiler.py:219-228): the original forward
  runs and ``fusion_applied`` is False.
* With the device check disabled and the launcher factory replaced by a
  recorder, the whole pipeline — AOT lowering, cost model, discovery, surgery,
  launcher binding — runs and the compiled module still equals eager.
* A group the kernel family cannot express gets its eager closure: no
  placeholder is ever left in the graph.
"""

import pytest
import torch
import torch.nn as nn
import torch.nn.functional as F

import fuseml_amd.compiler as comp
from fuseml_amd.compiler import FuseMLCompiler, trigger_is_fusible
from fuseml_amd.workloads import ActivationHeavy, GemmRowReductions, TransformerMLP

BF = torch.bfloat16


def _compile(model, backend):
    torch._dynamo.reset()
    return torch.compile(model, backend=backend)


def test_bypass_without_gfx950():
    torch.manual_seed(0)
    m = TransformerMLP(64, 256).eval()
    x = torch.randn(32, 64)
    be = FuseMLCompiler()
    with torch.no_grad():
        out = _compile(m, be)(x)
        ref = m(x)
    assert torch.allclose(out, ref)
    assert be.fusion_applied is False and be.fusion_strategy == "none"


class Recorded:
    """Launcher stand-in: runs the group's eager module and records the spec."""

    built = []

    def __init__(self, group):
        from fuseml_amd.epilogue import spec_from_group

        self.__name__ = "fuseml_fused_kernel"
        self.spec = spec_from_group(group)
        self.module = group.eager_module
        Recorded.built.append(self)

    def __call__(self, *args):
        return self.module(*args)


@pytest.fixture
def recorded(monkeypatch):
    Recorded.built = []
    monkeypatch.setattr(comp, "build_hip_launcher", lambda group, eager_fn=None: Recorded(group))
    return Recorded


def test_full_pipeline_bf16_mlp(recorded):
    torch.manual_seed(0)
    m = TransformerMLP(64, 256).to(BF).eval()
    x = torch.randn(32, 64, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        out = _compile(m, be)(x)
        ref = m(x)
    assert torch.allclose(out.float(), ref.float(), atol=1e-2)
    assert be.fusion_applied and be.fusion_strategy == "hip"
    assert [s.spec.describe() for s in recorded.built] == [
        "gemm(1,2) -> add[0] -> gelu_erf", "gemm(1,2) -> add[0] -> add[3]"]


def test_full_pipeline_sibling_reductions(recorded):
    torch.manual_seed(0)
    m = GemmRowReductions(64, 128).to(BF).eval()
    x = torch.randn(32, 64, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0, fuse_sibling_reductions=True)
    with torch.no_grad():
        got = _compile(m, be)(x)
        ref = m(x)
    for a, b in zip(got, ref):
        assert torch.allclose(a.float(), b.float(), atol=1e-2)
    assert len(recorded.built) == 1 and recorded.built[0].spec.reductions == ("sum", "amax", "mean")


def test_tiny_output_bypasses_under_the_reference_rule(recorded):
    m = TransformerMLP(64, 256).to(BF).eval()
    x = torch.randn(32, 64, dtype=BF)   # 32 x 256 < 500 000 outputs
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=comp.REFERENCE_MIN_OUTPUT_ELEMENTS)
    with torch.no_grad():
        _compile(m, be)(x)
    assert be.fusion_applied is False and recorded.built == []


def test_tiny_output_fuses_by_default(recorded):
    """The calibrated default has no output-size floor: a tiny group fuses."""
    m = TransformerMLP(64, 256).to(BF).eval()
    x = torch.randn(32, 64, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False)
    with torch.no_grad():
        out = _compile(m, be)(x)
    assert torch.allclose(out.float(), m(x).float(), atol=1e-2)
    assert be.fusion_applied and len(recorded.built) == 2


def test_fp32_gemm_fuses_as_split_product(recorded):
    """fp32 groups fuse (the reference fuses them through Triton's tf32 dot,
    kernel_generator.py:1536); K need not be a multiple of 8 (the split pads
    it), and the K-per-pass crossover, calibrated against eager bf16 GEMMs,
    does not apply (eager fp32 runs at the fp32 MFMA rate)."""
    m = TransformerMLP(60, 256).eval()
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        out = _compile(m, be)(torch.randn(32, 60))
        ref = m(torch.randn(32, 60))
    assert out.dtype == torch.float32 and out.shape == ref.shape
    assert be.fusion_applied and [s.spec.describe() for s in recorded.built] == [
        "gemm(1,2) -> add[0] -> gelu_erf", "gemm(1,2) -> add[0] -> add[3]"]
    assert comp.fused_beats_eager(recorded.built[1].spec, 16384, dtype=torch.float32)[0]
    assert not comp.fused_beats_eager(recorded.built[1].spec, 16384, dtype=torch.bfloat16)[0]


def test_fp64_gemm_bypasses(recorded):
    m = TransformerMLP(64, 256).to(torch.float64).eval()
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        _compile(m, be)(torch.randn(32, 64, dtype=torch.float64))
    assert be.fusion_applied is False and recorded.built == []


def test_fp32_few_tiles_rule_uses_the_split_k_loop():
    """The few-tile rule looks at the K loop the kernel runs: 3 ceil8(K) for fp32."""
    assert comp.effective_k(1000, torch.float32) == 3000
    assert comp.effective_k(1001, torch.float32) == 3024
    assert comp.effective_k(1000, torch.bfloat16) == 1000


def test_unbuildable_group_runs_eager(monkeypatch):
    monkeypatch.setattr(comp, "build_hip_launcher", lambda group, eager_fn=None: None)
    torch.manual_seed(0)
    m = ActivationHeavy(64, 256).to(BF).eval()
    x, g = torch.randn(32, 64, dtype=BF), torch.rand(32, 256, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        out = _compile(m, be)(x, g)
        ref = m(x, g)
    assert torch.allclose(out.float(), ref.float(), atol=1e-2)
    assert be.fusion_applied is False and be.fusion_strategy == "eager"


def test_cache_hits_on_identical_blocks(recorded):
    from fuseml_amd.workloads import StackedMLP

    torch.manual_seed(0)
    m = StackedMLP(64, 256, 3).to(BF).eval()
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        _compile(m, be)(torch.randn(32, 64, dtype=BF))
    # three identical blocks: one launcher per distinct (chain, layout), reused by the others
    assert (be.cache.misses, be.cache.hits, len(be.cache)) == (2, 4, 2)
    assert len(be.launchers) == 6 and len({id(x) for x in be.launchers}) == 2


def test_cost_model_rules():
    import torch.fx as fx
    from torch.fx.experimental.proxy_tensor import make_fx

    def f(x, w):
        return torch.mm(x, w)

    gm = make_fx(f)(torch.randn(1024, 64, dtype=BF), torch.randn(64, 1024, dtype=BF))
    mm = [n for n in gm.graph.nodes if n.op == "call_function"][0]
    assert trigger_is_fusible(mm)[0]
    gm2 = make_fx(f)(torch.randn(16, 64, dtype=BF), torch.randn(64, 16, dtype=BF))
    mm2 = [n for n in gm2.graph.nodes if n.op == "call_function"][0]
    assert trigger_is_fusible(mm2)[0]  # no output-size floor by default
    assert trigger_is_fusible(mm2, min_output_elements=comp.REFERENCE_MIN_OUTPUT_ELEMENTS) == \
        (False, "tiny output 16x16")
    gm3 = make_fx(f)(torch.randn(1024, 60, dtype=BF), torch.randn(60, 1024, dtype=BF))
    mm3 = [n for n in gm3.graph.nodes if n.op == "call_function"][0]
    assert trigger_is_fusible(mm3)[0] is False


def test_cost_model_few_tiles_long_k():
    """Fewer 128x128 output tiles than two per CU: fused while K x (operand rows
    per CU on the library's lock-step tile) stays within the measured budget;
    two full rounds of tiles are fused whatever K."""
    from torch.fx.experimental.proxy_tensor import make_fx

    def f(x, w):
        return torch.mm(x, w)

    def node(M, K, N):
        gm = make_fx(f)(torch.randn(M, K, dtype=BF), torch.randn(K, N, dtype=BF))
        return [n for n in gm.graph.nodes if n.op == "call_function"][0]

    # 8 x 8 = 64 tiles: 256 of 32x128, 160 rows per CU
    ok, why = trigger_is_fusible(node(1024, 4096, 1024))
    assert ok is False and "64 output tiles at a K loop of 4096" in why and "32x128" in why
    assert trigger_is_fusible(node(1024, 4096, 1024), min_tiles_long_k=0)[0]
    assert trigger_is_fusible(node(1024, 2048, 1024))[0]       # 160 x 2048 rows within the budget
    assert not trigger_is_fusible(node(2048, 2048, 2048))[0]   # 256 tiles of 128x128: 256 x 2048 rows
    assert trigger_is_fusible(node(2048, 1024, 2048))[0]       # 256 x 1024
    assert trigger_is_fusible(node(4096, 2048, 2048))[0]       # 32 x 16 = 512 tiles
    assert trigger_is_fusible(node(1024, 1024, 1024))[0]
    # the reference's medium preset's second GEMM (128 tiles, 64x128 tiles, K = 4096) stays eager
    assert not trigger_is_fusible(node(2048, 4096, 1024))[0]
    # decode-sized M against a wide weight streams the weight either way: no few-tile objection
    assert trigger_is_fusible(node(128, 8192, 32768))[0] and trigger_is_fusible(node(16, 4096, 65536))[0]
    assert not trigger_is_fusible(node(128, 8192, 16384))[0]   # 128 column tiles: fewer than one per CU


def test_weight_streaming_groups_fuse_to_4096_per_pass():
    """fused_beats_eager: with M and N given, M <= 128 and a 128-column tile
    per CU fuse while K <= 4096 x passes (one pass: 4096, where the pass rule
    stops at 2048); without them, or at M = 129, the pass rule."""
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp

    spec = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("gelu_erf")), BF)
    assert not comp.fused_beats_eager(spec, 4096)[0]
    assert comp.fused_beats_eager(spec, 4096, M=128, N=65536)[0]
    assert not comp.fused_beats_eager(spec, 8192, M=128, N=65536)[0]
    assert not comp.fused_beats_eager(spec, 4096, M=129, N=65536)[0]
    assert not comp.fused_beats_eager(spec, 4096, M=128, N=16384)[0]
    two = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("gelu_erf"), EpiOp("add", 3)), BF)
    assert comp.fused_beats_eager(two, 8192, M=64, N=65536)[0]
    assert comp.weight_streaming(1, 32768) and not comp.weight_streaming(1, 32640)


def test_partial_round_tile_mirrors_the_library():
    """compiler.partial_round_tile names the tile the library's own choice picks
    (fuseml_gemm_epilogue_config, 256 CUs without a device)."""
    import ctypes

    from fuseml_amd import _abi

    lib = _abi.load_library()
    cfg = (ctypes.c_int32 * 4)()
    shapes = [(M, N, K) for M, N in ((1, 4096), (64, 512), (128, 256), (128, 1024), (512, 4096), (1000, 900),
                                     (1024, 1024), (2048, 1024), (2048, 2048), (2048, 4096), (128, 16384),
                                     (128, 32768), (96, 65536), (64, 65536), (16, 65536))
              for K in (1024, 4096)]
    for M, N, K in shapes:
        d = _abi.GemmDesc()
        d.M, d.N, d.K = M, N, K
        d.a, d.lda, d.b, d.ldb = 0x10000, K, 0x20000, K
        d.ab_dtype = _abi.BF16
        d.out.ptr, d.out.ld, d.out.dtype = 0x30000, N, _abi.BF16
        assert lib.fuseml_gemm_epilogue_config(ctypes.byref(d), cfg) == 0, _abi.last_error(lib)
        assert (cfg[0], cfg[1]) == comp.partial_round_tile(M, N, K)[0], (M, N, K)


class _TwoReductionChains(nn.Module):
    """Two mm -> gelu -> {sum, amax} chains of equal shapes; in the second the
    GELU value is also returned, so its group returns (sum, amax, tile)."""

    def __init__(self):
        super().__init__()
        self.a = nn.Linear(64, 128, bias=False)
        self.b = nn.Linear(64, 128, bias=False)

    def forward(self, x):
        h1 = F.gelu(self.a(x))
        h2 = F.gelu(self.b(x))
        return h1.sum(-1), h1.amax(-1), h2.sum(-1), h2.amax(-1), h2


def test_cache_key_separates_return_signatures(recorded):
    torch.manual_seed(0)
    m = _TwoReductionChains().to(BF).eval()
    x = torch.randn(32, 64, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0, fuse_sibling_reductions=True)
    with torch.no_grad():
        got = _compile(m, be)(x)
        ref = m(x)
    for a, b in zip(got, ref):
        assert a.shape == b.shape and torch.allclose(a.float(), b.float(), atol=1e-2)
    assert (be.cache.misses, be.cache.hits) == (2, 0)
    outs = sorted(r.spec.outputs for r in recorded.built)
    assert outs == sorted([(("red", "sum"), ("red", "amax")),
                           (("red", "sum"), ("red", "amax"), ("tile",))])


def test_epilogue_passes_and_crossover_rule():
    """The measured crossover: fuse iff K <= 1024 x (elementwise passes eager
    would run after the GEMM).  The benchmark configs' groups land on the
    measured side of it."""
    from fuseml_amd.compiler import epilogue_passes, fused_beats_eager
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp

    g1 = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("gelu_erf")), BF)
    g2 = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("add", 3)), BF)
    c3 = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("relu"), EpiOp("mul", 3), EpiOp("sigmoid"), EpiOp("add", 4)), BF)
    c4 = EpilogueSpec(0, 1, (EpiOp("relu"),), BF, reductions=("sum", "amax", "mean"))
    alpha = EpilogueSpec(1, 2, (EpiOp("scale", scalar=0.5), EpiOp("add", 0), EpiOp("store", 0), EpiOp("relu")), BF)
    assert [epilogue_passes(s) for s in (g1, g2, c3, c4, alpha)] == [1, 1, 4, 4, 1]
    assert fused_beats_eager(g1, 1024)[0] and fused_beats_eager(c3, 1024)[0] and fused_beats_eager(c4, 2048)[0]
    assert not fused_beats_eager(g2, 4096)[0] and not fused_beats_eager(g1, 4096)[0]
    assert not fused_beats_eager(g2, 16384)[0]
    assert fused_beats_eager(g2, 16384, k_per_pass=0)[0]
    # After an mm (no addmm bias) a leading add is an eager pass of its own.
    mm_add = EpilogueSpec(0, 1, (EpiOp("add", 2),), BF)
    mm_add_gelu = EpilogueSpec(0, 1, (EpiOp("add", 2), EpiOp("gelu_erf")), BF)
    assert epilogue_passes(mm_add, gemm_is_addmm=False) == 1
    assert epilogue_passes(mm_add, gemm_is_addmm=True) == 0
    assert epilogue_passes(mm_add_gelu, gemm_is_addmm=False) == 2
    assert fused_beats_eager(mm_add, 1024, gemm_is_addmm=False)[0]
    assert fused_beats_eager(mm_add_gelu, 4096, gemm_is_addmm=False)[0]
    assert not fused_beats_eager(mm_add_gelu, 4096, gemm_is_addmm=True)[0]


class _MmAddGelu(nn.Module):
    """gelu(x @ W.T + b) written without F.linear: the graph is mm -> add ->
    gelu, two eager passes after the GEMM."""

    def __init__(self, d_in, d_out):
        super().__init__()
        self.w = nn.Parameter(torch.randn(d_out, d_in) / d_in ** 0.5)
        self.b = nn.Parameter(torch.randn(d_out) * 0.1)

    def forward(self, x):
        return F.gelu(x @ self.w.t() + self.b)


def test_mm_add_counts_the_add_as_a_pass(recorded):
    """K = 2048 with two passes (add, gelu) is inside the measured crossover
    (K <= 1024 x passes), so the mm-based group fuses; counted as an addmm's
    free bias it would have one pass and stay eager."""
    torch.manual_seed(0)
    m = _MmAddGelu(2048, 256).to(BF).eval()
    x = torch.randn(64, 2048, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0, min_tiles_long_k=0)
    with torch.no_grad():
        out = _compile(m, be)(x)
    assert torch.allclose(out.float(), m(x).float(), atol=2e-2)
    assert [s.spec.describe() for s in recorded.built] == ["gemm(0,1) -> add[2] -> gelu_erf"]
    assert be.fusion_strategy == "hip"


def test_long_k_groups_route_to_eager(recorded):
    """StackedMLP at K = 4096 / 16384 (C5's widths, few rows): every group has
    one elementwise pass, so the default cost model keeps them eager."""
    from fuseml_amd.workloads import StackedMLP

    torch.manual_seed(0)
    m = StackedMLP(4096, 16384, 1).to(BF).eval()
    x = torch.randn(64, 4096, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False, min_tiles_long_k=0)
    with torch.no_grad():
        out = _compile(m, be)(x)
    assert torch.allclose(out.float(), m(x).float(), atol=1e-2)
    assert recorded.built == [] and be.fusion_strategy == "eager"


class _MutatesInput(nn.Module):
    def __init__(self):
        super().__init__()
        self.lin = nn.Linear(64, 256)

    def forward(self, x):
        x.mul_(2.0)
        return F.gelu(self.lin(x))


class _ReturnsInputView(nn.Module):
    def __init__(self):
        super().__init__()
        self.lin = nn.Linear(64, 256)

    def forward(self, x):
        return F.gelu(self.lin(x)), x.view(-1)


def test_direct_dispatch_when_aot_wrapper_is_identity(recorded):
    """An inference graph with no mutated inputs and no aliased outputs: the
    backend returns the fused graph's forward itself (no AOTAutograd runtime
    wrapper), and the compiled module still equals eager, also when called
    with autograd on."""
    torch.manual_seed(0)
    m = TransformerMLP(64, 256).to(BF).eval()
    x = torch.randn(32, 64, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        c = _compile(m, be)
        out = c(x)
        assert torch.allclose(out.float(), m(x).float(), atol=1e-2)
    assert be.dispatch == ["direct"] and be.fusion_applied
    off = FuseMLCompiler(require_gfx950=False, min_output_elements=0, direct_dispatch=False)
    with torch.no_grad():
        assert torch.equal(_compile(m, off)(x), out)
    assert off.dispatch == ["aot: direct dispatch off"]


def test_mutated_input_keeps_the_aot_wrapper(recorded):
    torch.manual_seed(0)
    m = _MutatesInput().to(BF).eval()
    x = torch.randn(32, 64, dtype=BF)
    x_ref = x.clone()
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        out = _compile(m, be)(x)
        ref = m(x_ref)
    assert torch.equal(x, x_ref)  # the input mutation was applied by the wrapper
    assert torch.allclose(out.float(), ref.float(), atol=1e-2)
    assert be.dispatch and be.dispatch[0].startswith("aot: mutated inputs")


def test_output_aliasing_an_input_keeps_the_aot_wrapper(recorded):
    torch.manual_seed(0)
    m = _ReturnsInputView().to(BF).eval()
    x = torch.randn(32, 64, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        y, v = _compile(m, be)(x)
        ry, _ = m(x)
    assert torch.allclose(y.float(), ry.float(), atol=1e-2)
    assert v.data_ptr() == x.data_ptr() and v.shape == (32 * 64,)  # still a view of the input
    assert be.dispatch and be.dispatch[0].startswith("aot: aliased outputs")
