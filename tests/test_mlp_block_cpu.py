"""The single-kernel MLP block's host side on the CPU (no kernel launch).

* ``FuseMLCompiler(fuse_mlp_block=True)`` binds the two groups of
  ``linear2(gelu(linear1(x))) + x`` to one ``HipMlpLauncher``; the default
  (``"auto"``) binds them only where the measured rule says the single kernel
  is faster, else keeps the reference's two groups.  The launch is forced onto
  its eager fallback, which chains the two groups' original nodes, so the
  compiled module equals eager.
* The launcher fills ``fuseml_mlp_desc`` from the graph's layouts.
* The shape rule mirrors the kernel's limits.
"""

import ctypes

import pytest
import torch

import fuseml_amd.compiler as comp
from fuseml_amd import _abi
from fuseml_amd.compiler import FuseMLCompiler
from fuseml_amd.fallback import FORCE_FAIL_ENV
from fuseml_amd.mlp import HipMlpLauncher, mlp_block_beats_two_launches, mlp_shape_supported
from fuseml_amd.workloads import ActivationHeavyMLP, StackedMLP, TransformerMLP

BF = torch.bfloat16


def _compile(model, be):
    torch._dynamo.reset()
    return torch.compile(model, backend=be)


@pytest.mark.parametrize("approximate", ["none", "tanh"])
def test_mlp_block_opt_in_binds_one_launcher(monkeypatch, approximate):
    torch.manual_seed(0)
    m = TransformerMLP(256, 1024, approximate=approximate).to(BF).eval()
    x = torch.randn(64, 256, dtype=BF)
    monkeypatch.setenv(FORCE_FAIL_ENV, "1")
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0, fuse_mlp_block=True)
    with torch.no_grad():
        out = _compile(m, be)(x)
        ref = m(x)
    assert torch.equal(out, ref)
    assert len(be.launchers) == 1 and isinstance(be.launchers[0], HipMlpLauncher)
    assert be.launchers[0].approximate == approximate and be.launchers[0].fallback_count == 1


def test_mlp_block_small_batch_keeps_two_groups_by_default(monkeypatch):
    torch.manual_seed(0)
    m = TransformerMLP(256, 1024).to(BF).eval()
    x = torch.randn(64, 256, dtype=BF)
    monkeypatch.setenv(FORCE_FAIL_ENV, "1")
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0)
    with torch.no_grad():
        out = _compile(m, be)(x)
    assert torch.equal(out, m(x))
    assert len(be.launchers) == 2 and not any(isinstance(l, HipMlpLauncher) for l in be.launchers)


def test_auto_rule_follows_the_measured_crossover():
    assert mlp_block_beats_two_launches(16384, 256, 1024)[0]          # memory_bound preset
    assert mlp_block_beats_two_launches(65536, 256, 4096)[0]
    assert not mlp_block_beats_two_launches(8192, 256, 1024)[0]       # fewer 64-row blocks than CUs
    assert not mlp_block_beats_two_launches(16384, 512, 2048)[0]      # D = 512 ties at best
    assert not mlp_block_beats_two_launches(16384, 1024, 4096)[0]     # C2: D = 1024
    assert not mlp_block_beats_two_launches(16384, 256, 96)[0]        # I not a multiple of 128


def test_auto_binds_where_the_single_kernel_wins(monkeypatch):
    """Default options: the memory_bound shape (x[16384,256] -> 1024 -> 256)
    runs as one single-kernel MLP launch; a D = 512 block keeps two launches."""
    torch.manual_seed(0)
    monkeypatch.setenv(FORCE_FAIL_ENV, "1")
    m = TransformerMLP(256, 1024).to(BF).eval()
    x = torch.randn(16384, 256, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False)
    with torch.no_grad():
        assert torch.equal(_compile(m, be)(x), m(x))
    assert len(be.launchers) == 1 and isinstance(be.launchers[0], HipMlpLauncher)
    m = TransformerMLP(512, 1024).to(BF).eval()
    x = torch.randn(16384, 512, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False)
    with torch.no_grad():
        assert torch.equal(_compile(m, be)(x), m(x))
    assert len(be.launchers) == 2 and not any(isinstance(l, HipMlpLauncher) for l in be.launchers)


def test_activation_heavy_block_binds_with_its_scalar_ops(monkeypatch):
    """The reference's activation-heavy block, gelu(linear1(x)) * 0.5 + 0.125
    into linear2 + x, at the memory_bound shape: one single-kernel launch whose
    post-GELU ops are the scale and the shift, in graph order."""
    torch.manual_seed(0)
    monkeypatch.setenv(FORCE_FAIL_ENV, "1")
    m = ActivationHeavyMLP(256, 1024).to(BF).eval()
    x = torch.randn(16384, 256, dtype=BF)
    be = FuseMLCompiler(require_gfx950=False)
    with torch.no_grad():
        assert torch.equal(_compile(m, be)(x), m(x))
    (L,) = be.launchers
    assert isinstance(L, HipMlpLauncher) and L.post == (("scale", 0.5), ("add_scalar", 0.125))


def test_first_group_matcher_takes_scalar_ops_only():
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp
    from fuseml_amd.mlp import mlp_first_group

    base = (EpiOp("add", 0), EpiOp("gelu_erf"))
    m1 = mlp_first_group(EpilogueSpec(1, 2, base + (EpiOp("scale", scalar=0.5), EpiOp("add_scalar", scalar=0.125)), BF))
    assert m1 is not None and m1["post"] == (("scale", 0.5), ("add_scalar", 0.125))
    assert mlp_first_group(EpilogueSpec(1, 2, base, BF))["post"] == ()
    assert mlp_first_group(EpilogueSpec(1, 2, base + (EpiOp("relu"),), BF)) is None
    assert mlp_first_group(EpilogueSpec(1, 2, base + (EpiOp("add", 3),), BF)) is None
    five = base + tuple(EpiOp("scale", scalar=2.0) for _ in range(_abi.MLP_MAX_POST + 1))
    assert mlp_first_group(EpilogueSpec(1, 2, five, BF)) is None


def test_fuse_mlp_block_rejects_unknown_modes():
    with pytest.raises(ValueError):
        FuseMLCompiler(fuse_mlp_block="always")


def test_mlp_block_stacked_blocks_each_one_launcher(monkeypatch):
    torch.manual_seed(1)
    m = StackedMLP(512, 1024, 3).to(BF).eval()
    x = torch.randn(32, 512, dtype=BF)
    monkeypatch.setenv(FORCE_FAIL_ENV, "1")
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0, fuse_mlp_block=True)
    with torch.no_grad():
        out = _compile(m, be)(x)
    assert torch.equal(out, m(x))
    assert len(be.launchers) == 3 and all(isinstance(l, HipMlpLauncher) for l in be.launchers)


def test_unsupported_width_keeps_two_launches(monkeypatch):
    """D = 768 is not a width the kernel holds in registers: two launches."""
    torch.manual_seed(0)
    m = TransformerMLP(768, 1024).to(BF).eval()
    x = torch.randn(64, 768, dtype=BF)
    monkeypatch.setenv(FORCE_FAIL_ENV, "1")
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0, fuse_mlp_block=True)
    with torch.no_grad():
        assert torch.equal(_compile(m, be)(x), m(x))
    assert len(be.launchers) == 2


def test_pair_with_a_tiny_second_gemm_keeps_two_launches(monkeypatch):
    """x[256,256] -> 4096 -> 256: the first GEMM's output (1M elements) passes
    the tiny-output rule, the second's (65k) does not, so the pair is not bound
    to the single-kernel MLP: the first group fuses and the second runs eager."""
    torch.manual_seed(0)
    m = TransformerMLP(256, 4096).to(BF).eval()
    x = torch.randn(256, 256, dtype=BF)
    monkeypatch.setenv(FORCE_FAIL_ENV, "1")
    be = FuseMLCompiler(require_gfx950=False, fuse_mlp_block=True)
    with torch.no_grad():
        assert torch.equal(_compile(m, be)(x), m(x))
    assert not any(isinstance(l, HipMlpLauncher) for l in be.launchers)
    assert len(be.launchers) == 1 and be.fusion_strategy == "mixed"


class _Recorder:
    def __init__(self):
        self.calls = []

    def fuseml_mlp_block(self, desc_ref, stream):
        d = ctypes.cast(desc_ref, ctypes.POINTER(_abi.MlpDesc)).contents
        self.calls.append({f: getattr(d, f) for f, _ in _abi.MlpDesc._fields_})
        return 0

    def fuseml_last_error(self):
        return b""


def test_mlp_descriptor_from_graph_layouts():
    M, D, I = 48, 256, 1024
    x = torch.randn(M, D, dtype=BF)
    w1, b1 = torch.randn(I, D, dtype=BF), torch.randn(I, dtype=BF)
    w2, b2 = torch.randn(D, I, dtype=BF), torch.randn(D, dtype=BF)
    L = HipMlpLauncher("tanh")
    rec = _Recorder()
    L._lib = rec
    y = L(x, w1.t(), b1, w2.t(), b2, x)
    (c,) = rec.calls
    assert y.shape == (M, D) and y.dtype == BF
    assert (c["M"], c["D"], c["I"], c["ldx"], c["ldw1"], c["ldw2"], c["ldr"], c["ldy"]) == (M, D, I, D, D, I, D, D)
    assert c["x"] == x.data_ptr() and c["r"] == x.data_ptr() and c["w1"] == w1.data_ptr()
    assert c["dtype"] == _abi.BF16 and c["gelu"] == _abi.OP_GELU_TANH and c["n_post"] == 0
    with pytest.raises(ValueError):
        L(x, w1.t(), b1)
    with pytest.raises(_abi.FuseMLHipError):   # shapes that do not chain
        L(x, w1.t(), b1, w1.t(), b2, x)


def test_mlp_descriptor_carries_the_scalar_ops():
    M, D, I = 16, 256, 128
    x = torch.randn(M, D, dtype=BF)
    w1, b1, w2 = torch.randn(I, D, dtype=BF), torch.randn(I, dtype=BF), torch.randn(D, I, dtype=BF)
    L = HipMlpLauncher(post=(("scale", 0.5), ("add_scalar", 0.125)))
    rec = _Recorder()
    L._lib = rec
    L(x, w1.t(), b1, w2.t(), None, None)
    (c,) = rec.calls
    assert c["n_post"] == 2 and list(c["post_kind"])[:2] == [_abi.OP_SCALE, _abi.OP_ADD_SCALAR]
    assert list(c["post_scalar"])[:2] == [0.5, 0.125]
    with pytest.raises(ValueError):
        HipMlpLauncher(post=(("relu", 0.0),))
    with pytest.raises(ValueError):
        HipMlpLauncher(post=(("scale", 2.0),) * (_abi.MLP_MAX_POST + 1))


def test_mlp_shape_rule():
    assert mlp_shape_supported(16384, 1024, 4096, BF)[0]
    assert mlp_shape_supported(64, 256, 32, torch.float16)[0]
    assert not mlp_shape_supported(8192, 4096, 16384, BF)[0]      # C5: D too wide
    assert not mlp_shape_supported(64, 512, 100, BF)[0]           # I % 32
    assert not mlp_shape_supported(64, 512, 1024, torch.float32)[0]


def test_mlp_launcher_refuses_host_tensors():
    """With the real library bound, CPU tensors raise before any device call."""
    D, I, M = 256, 64, 8
    x = torch.randn(M, D, dtype=BF)
    w1t, w2t = torch.randn(I, D, dtype=BF).t(), torch.randn(D, I, dtype=BF).t()
    b1, b2 = torch.randn(I, dtype=BF), torch.randn(D, dtype=BF)
    launcher = HipMlpLauncher()
    assert isinstance(launcher._lib, ctypes.CDLL)
    with pytest.raises(_abi.FuseMLHipError, match="must be on the launch's GPU"):
        launcher(x, w1t, b1, w2t, b2, x)
