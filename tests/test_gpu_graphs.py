"""HIP-graph replay of compiled forwards (``FuseMLCompiler(hip_graph=True)``)
on the device, against the same module compiled without graphs.

Each case replays the captured graph several times on fresh inputs, with
unrelated eager work and synchronisations between the replays, and checks
every replay bitwise against the graph-free compiled forward (the same
kernels on the same inputs): the reference's presets with the single-kernel
MLP (memory_bound), two fused launches (small) and a fused launch beside an
eager hipBLASLt GEMM (medium).  A weight modified in place makes the next call
run without the graph and the one after capture again, on the new weight.
"""

from __future__ import annotations

import pytest
import torch

pytestmark = pytest.mark.gpu


def _compiled(model, **kw):
    from fuseml_amd.compiler import FuseMLCompiler

    torch._dynamo.reset()
    be = FuseMLCompiler(**kw)
    return torch.compile(model, backend=be), be


@pytest.mark.parametrize("name", ["memory_bound", "small", "medium"])
def test_graph_replays_match_the_compiled_forward(name):
    from fuseml_amd.workloads import reference_preset

    print(f"case hip_graph preset={name}", flush=True)
    wl = reference_preset(name).to("cuda")
    m, x0 = wl.model, wl.inputs[0]
    gen = torch.Generator(device="cuda").manual_seed(1)
    xs = [torch.randn(x0.shape, generator=gen, device="cuda").to(x0.dtype) for _ in range(6)]
    noise = torch.randn(512, 512, device="cuda")
    with torch.no_grad():
        plain, _ = _compiled(m)
        want = [plain(x).clone() for x in xs]
        graphed, be = _compiled(m, hip_graph=True)
        got = []
        for i, x in enumerate(xs):
            got.append(graphed(x).clone())
            noise = torch.tanh(noise @ noise) * 0.5    # unrelated eager work between replays
            if i % 2:
                torch.cuda.synchronize()
        torch.cuda.synchronize()
    assert be.dispatch == ["direct+hip_graph"], be.dispatch
    (g,) = be.graph_forwards
    # captured over the third call's input, then again over private buffers
    # when the fourth call's input sits elsewhere
    assert g.captures == 2 and g.replays == len(xs) - 2
    for i, (a, b) in enumerate(zip(got, want)):
        assert torch.equal(a, b), f"{name}: call {i} differs from the graph-free forward"


def test_graph_reads_a_refilled_input_in_place():
    """A serving-style loop over one input buffer: captured once, read where it is."""
    from fuseml_amd.workloads import reference_preset

    print("case hip_graph input refilled in place", flush=True)
    wl = reference_preset("small").to("cuda")
    m, x0 = wl.model, wl.inputs[0]
    gen = torch.Generator(device="cuda").manual_seed(2)
    xs = [torch.randn(x0.shape, generator=gen, device="cuda").to(x0.dtype) for _ in range(5)]
    buf = torch.empty_like(x0)
    with torch.no_grad():
        plain, _ = _compiled(m)
        want = [plain(x).clone() for x in xs]
        graphed, be = _compiled(m, hip_graph=True)
        got = []
        for x in xs:
            buf.copy_(x)
            got.append(graphed(buf).clone())
        torch.cuda.synchronize()
    (g,) = be.graph_forwards
    assert g.captures == 1 and g.replays == len(xs) - 2
    assert all(torch.equal(a, b) for a, b in zip(got, want))


def test_graph_with_fused_row_reductions():
    """C4's module at 1/8 of its rows with sibling reductions fused: the sum,
    amax and mean outputs are initialised inside the graph (fill kernels) and
    accumulated by the kernel's atomics on every replay.  Sums and means are
    compared with a tolerance (atomic order), the tile and the amax bitwise."""
    from fuseml_amd.workloads import c4_gemm_row_reductions

    print("case hip_graph fused row reductions (C4 at 1/8)", flush=True)
    wl = c4_gemm_row_reductions(scale=1 / 8).to("cuda")
    m, x0 = wl.model, wl.inputs[0]
    gen = torch.Generator(device="cuda").manual_seed(3)
    xs = [torch.randn(x0.shape, generator=gen, device="cuda").to(x0.dtype) for _ in range(5)]
    buf = torch.empty_like(x0)
    with torch.no_grad():
        plain, _ = _compiled(m, fuse_sibling_reductions=True, min_tiles_long_k=0)
        want = [tuple(t.clone() for t in plain(x)) for x in xs]
        graphed, be = _compiled(m, fuse_sibling_reductions=True, min_tiles_long_k=0, hip_graph=True)
        got = []
        for x in xs:
            buf.copy_(x)
            got.append(tuple(t.clone() for t in graphed(buf)))
        torch.cuda.synchronize()
    assert be.dispatch == ["direct+hip_graph"] and be.graph_forwards[0].captures == 1
    for i, (g, w) in enumerate(zip(got, want)):
        assert len(g) == len(w)
        for a, b in zip(g, w):
            if a.dtype == torch.float32 and a.dim() == 1:
                assert torch.allclose(a, b, rtol=1e-5, atol=1e-3), f"call {i}: reduction differs"
            else:
                assert torch.equal(a, b), f"call {i}: output differs"


def test_weight_change_recaptures():
    from fuseml_amd.workloads import reference_preset

    print("case hip_graph weight change", flush=True)
    wl = reference_preset("memory_bound").to("cuda")
    m, x = wl.model, wl.inputs[0]
    with torch.no_grad():
        graphed, be = _compiled(m, hip_graph=True)
        for _ in range(4):
            graphed(x)
        (g,) = be.graph_forwards
        assert g.captures == 1
        m.linear1.weight.add_(0.01)                # in place: a new version of a static input
        y_plain_call = graphed(x).clone()          # runs without the graph
        y_recaptured = graphed(x).clone()          # captured again
        plain, _ = _compiled(m)
        want = plain(x).clone()
        torch.cuda.synchronize()
    assert g.captures == 2
    assert torch.equal(y_plain_call, want) and torch.equal(y_recaptured, want)
