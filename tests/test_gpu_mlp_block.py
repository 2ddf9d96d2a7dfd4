"""GPU parity of the single-kernel MLP block (``fuseml_mlp_block``) against the
float64 oracle.

``y = post(GELU(x W1^T + b1)) W2^T + b2 + r`` with ``h`` kept on chip (post:
scalar scale/shift ops, the reference's activation-heavy block).  The kernel
rounds ``h`` to the operand dtype before the second GEMM, as the two-launch
path (and eager bf16) do.  Cases: every supported width D (256, 512, 1024),
ragged M (not a multiple of the 64-row block), I down to one 32-column chunk,
GELU erf and tanh, bf16 and fp16, no bias/residual, and the C2 config at full
size through the launcher and through ``FuseMLCompiler(fuse_mlp_block=True)``.
The shapes run both kernels: the I-split one (D of 256 or 512 and I a multiple
of 128) and the D-split one (D = 1024 or I not a multiple of 128).

Tolerance: ``allclose(rtol=2e-2, atol=2e-2)`` against the float64 oracle.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from oracle import gemm_epilogue as ora
from oracle import workloads as ora_w

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().float().cpu().numpy().astype(np.float64)


def _close(got, ref, what):
    g = _np(got)
    assert g.shape == ref.shape, (what, g.shape, ref.shape)
    bad = ~np.isclose(g, ref, rtol=2e-2, atol=2e-2)
    assert not bad.any(), f"{what}: {bad.sum()} of {bad.size} mismatches, max err {np.abs(g - ref).max()}"


def _inputs(M, D, I, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(M, D, generator=g).to(dtype)
    w1 = (torch.randn(I, D, generator=g) / D ** 0.5).to(dtype)
    b1 = (torch.rand(I, generator=g) * 0.2 - 0.1).to(dtype)
    w2 = (torch.randn(D, I, generator=g) / I ** 0.5).to(dtype)
    b2 = (torch.rand(D, generator=g) * 0.2 - 0.1).to(dtype)
    r = torch.randn(M, D, generator=g).to(dtype)
    return x, w1, b1, w2, b2, r


def _oracle(x, w1, b1, w2, b2, r, approximate="none", dtype=None, post=()):
    h = ora_w.linear(_np(x), _np(w1), _np(b1))
    h = ora.gelu_tanh(h) if approximate == "tanh" else ora.gelu_erf(h)
    h, _ = ora.apply_chain(h, [(kind, 0, s) for kind, s in post], [])
    y = ora_w.linear(h, _np(w2), None if b2 is None else _np(b2))
    return y if r is None else y + _np(r)


@pytest.mark.parametrize("approximate", ["none", "tanh"])
@pytest.mark.parametrize("shape", [(300, 256, 1024), (129, 512, 96), (64, 1024, 32), (1, 256, 64), (200, 1024, 2048),
                                   (129, 512, 384), (1, 256, 128), (65, 256, 1152), (640, 512, 2048)],
                         ids=lambda s: "x".join(map(str, s)))
def test_mlp_block_parity(shape, approximate):
    from fuseml_amd.mlp import HipMlpLauncher

    M, D, I = shape
    print(f"case mlp_block shape={shape} gelu={approximate}", flush=True)
    x, w1, b1, w2, b2, r = _inputs(M, D, I, torch.bfloat16, seed=M + D + I)
    y = HipMlpLauncher(approximate)(x.cuda(), w1.t().cuda(), b1.cuda(), w2.t().cuda(), b2.cuda(), r.cuda())
    torch.cuda.synchronize()
    _close(y, _oracle(x, w1, b1, w2, b2, r, approximate), f"mlp_block {shape} {approximate}")


@pytest.mark.parametrize("post", [(("scale", 0.5), ("add_scalar", 0.125)),
                                  (("add_scalar", -0.25), ("scale", 3.0), ("scale", -0.5), ("add_scalar", 1.0))],
                         ids=["act_heavy", "four_ops"])
@pytest.mark.parametrize("shape", [(300, 256, 1024), (129, 512, 96), (64, 1024, 32)], ids=lambda s: "x".join(map(str, s)))
def test_mlp_block_post_gelu_ops(shape, post):
    """Scalar ops between the GELU and the second GEMM (the reference's
    activation-heavy block scales and shifts the GELU), on both kernels."""
    from fuseml_amd.mlp import HipMlpLauncher

    M, D, I = shape
    print(f"case mlp_block post ops shape={shape} post={post}", flush=True)
    x, w1, b1, w2, b2, r = _inputs(M, D, I, torch.bfloat16, seed=7 * M + D + I)
    y = HipMlpLauncher(post=post)(x.cuda(), w1.t().cuda(), b1.cuda(), w2.t().cuda(), b2.cuda(), r.cuda())
    torch.cuda.synchronize()
    _close(y, _oracle(x, w1, b1, w2, b2, r, post=post), f"mlp_block {shape} post {post}")


def test_activation_heavy_memory_bound_compiled():
    """The reference's activation_heavy_memory_bound preset (x[16384,256] ->
    1024 -> 256) under the default options: one single-kernel launch carrying
    the block's * 0.5 + 0.125, against the float64 oracle at sampled rows."""
    from fuseml_amd.compiler import FuseMLCompiler
    from fuseml_amd.mlp import HipMlpLauncher
    from fuseml_amd.workloads import reference_preset

    print("case mlp_block compiled activation_heavy_memory_bound", flush=True)
    wl = reference_preset("activation_heavy_memory_bound")
    m, x = wl.model, wl.inputs[0]
    rng = np.random.default_rng(11)
    rows = np.unique(np.concatenate([[0, 16383], rng.integers(0, 16384, 64)]))
    xs = x[torch.as_tensor(rows)]
    ref = _oracle(xs, m.linear1.weight, m.linear1.bias, m.linear2.weight, m.linear2.bias, xs,
                  post=(("scale", 0.5), ("add_scalar", 0.125)))
    wl.to("cuda")
    torch._dynamo.reset()
    be = FuseMLCompiler()
    with torch.no_grad():
        y = torch.compile(wl.model, backend=be)(*wl.inputs)
    torch.cuda.synchronize()
    (L,) = be.launchers
    assert isinstance(L, HipMlpLauncher) and L.launch_count == 1 and L.fallback_count == 0
    assert L.post == (("scale", 0.5), ("add_scalar", 0.125))
    _close(y[torch.as_tensor(rows).cuda()], ref, "compiled activation_heavy_memory_bound")


@pytest.mark.parametrize("shape", [(300, 256, 1024), (129, 512, 384)], ids=lambda s: "x".join(map(str, s)))
def test_mlp_block_unpacked_weights(shape):
    """The I-split kernel reading W1 and W2 as they are (no repacked copy: a
    C-ABI caller that passes no wpack) against the oracle and bitwise against
    the packed path (the same fragments in the same order)."""
    from fuseml_amd.mlp import HipMlpLauncher

    M, D, I = shape
    print(f"case mlp_block unpacked shape={shape}", flush=True)
    x, w1, b1, w2, b2, r = _inputs(M, D, I, torch.bfloat16, seed=3 * M + D + I)
    args = (x.cuda(), w1.t().cuda(), b1.cuda(), w2.t().cuda(), b2.cuda(), r.cuda())
    y = HipMlpLauncher(pack_weights=False)(*args)
    yp = HipMlpLauncher()(*args)
    torch.cuda.synchronize()
    _close(y, _oracle(x, w1, b1, w2, b2, r), f"mlp_block unpacked {shape}")
    assert torch.equal(y, yp)


@pytest.mark.parametrize("mode", [False, True], ids=["two_launches", "single_kernel"])
def test_activation_heavy_block_compiled_both_paths(mode):
    """The activation-heavy block (gelu(.) * 0.5 + 0.125 between the GEMMs) at
    M = 1000 (ragged, below the auto rule's row blocks) through the compiler
    with two fused launches and forced onto the single kernel."""
    from fuseml_amd.compiler import FuseMLCompiler
    from fuseml_amd.mlp import HipMlpLauncher
    from fuseml_amd.workloads import ActivationHeavyMLP

    print(f"case activation-heavy block compiled fuse_mlp_block={mode}", flush=True)
    torch.manual_seed(4)
    m = ActivationHeavyMLP(256, 1024).to(torch.bfloat16).eval()
    x = torch.randn(1000, 256, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16)
    ref = _oracle(x, m.linear1.weight, m.linear1.bias, m.linear2.weight, m.linear2.bias, x,
                  post=(("scale", 0.5), ("add_scalar", 0.125)))
    m, xd = m.to("cuda"), x.cuda()
    torch._dynamo.reset()
    be = FuseMLCompiler(fuse_mlp_block=mode, min_output_elements=0)
    with torch.no_grad():
        y = torch.compile(m, backend=be)(xd)
    torch.cuda.synchronize()
    singles = [L for L in be.launchers if isinstance(L, HipMlpLauncher)]
    assert be.fusion_strategy == "hip" and len(singles) == (1 if mode else 0)
    assert len(be.launchers) == (1 if mode else 2)
    _close(y, ref, f"activation-heavy compiled fuse_mlp_block={mode}")


def test_mlp_block_fp16_without_bias_and_residual():
    from fuseml_amd.mlp import HipMlpLauncher

    M, D, I = 257, 512, 512
    print("case mlp_block fp16 no b2/r", flush=True)
    x, w1, b1, w2, _, _ = _inputs(M, D, I, torch.float16, seed=5)
    y = HipMlpLauncher()(x.cuda(), w1.t().cuda(), b1.cuda(), w2.t().cuda(), None, None)
    torch.cuda.synchronize()
    _close(y, _oracle(x, w1, b1, w2, None, None), "mlp_block fp16")


def test_mlp_block_c2_full_size_launcher():
    from fuseml_amd.mlp import HipMlpLauncher
    from fuseml_amd.workloads import c2_mlp_block

    print("case mlp_block C2 full size", flush=True)
    wl = c2_mlp_block()
    m, x = wl.model, wl.inputs[0]
    W1, b1, W2, b2 = m.linear1.weight, m.linear1.bias, m.linear2.weight, m.linear2.bias
    xd = x.cuda()
    y = HipMlpLauncher()(xd, W1.t().cuda(), b1.cuda(), W2.t().cuda(), b2.cuda(), xd)
    torch.cuda.synchronize()
    rng = np.random.default_rng(9)
    rows = np.unique(np.concatenate([[0, 16383], rng.integers(0, 16384, 64)]))
    ref = ora_w.transformer_mlp(_np(x), _np(W1), _np(b1), _np(W2), _np(b2), rows=rows)
    _close(y[torch.as_tensor(rows).cuda()], ref, "C2 mlp_block")


def test_mlp_block_compiled_c2():
    from fuseml_amd.compiler import FuseMLCompiler
    from fuseml_amd.mlp import HipMlpLauncher
    from fuseml_amd.workloads import c2_mlp_block

    print("case mlp_block compiled C2 (scale 1/8)", flush=True)
    wl = c2_mlp_block(scale=1 / 8)
    m, x = wl.model, wl.inputs[0]
    ref = ora_w.transformer_mlp(_np(x), _np(m.linear1.weight), _np(m.linear1.bias),
                                _np(m.linear2.weight), _np(m.linear2.bias))
    wl.to("cuda")
    torch._dynamo.reset()
    # at 1/8 scale the second GEMM has 128 tiles at K = 4096, which the
    # few-tile rule keeps eager (and with it the pair): lower the floor
    be = FuseMLCompiler(fuse_mlp_block=True, min_tiles_long_k=0)
    with torch.no_grad():
        y = torch.compile(wl.model, backend=be)(*wl.inputs)
    torch.cuda.synchronize()
    (L,) = be.launchers
    assert isinstance(L, HipMlpLauncher) and L.launch_count == 1 and L.fallback_count == 0
    _close(y, ref, "compiled mlp_block")
