"""HIP-graph replay wrapper (fuseml_amd.graphs) on the CPU: the capture/replay
state machine with a stand-in graph object (no device), and the compiler's
hip_graph option declining a graph off the GPU."""

import pytest
import torch

import fuseml_amd.compiler as comp
from fuseml_amd import graphs
from fuseml_amd.compiler import FuseMLCompiler
from fuseml_amd.workloads import TransformerMLP


class _FakeGraph:
    """Records the function captured under ``torch.cuda.graph`` and runs it
    again on replay (on the static buffers it was captured with)."""

    current = None

    def __init__(self):
        self.fn = None

    def replay(self):
        self.fn()


class _Capture:
    def __init__(self, g):
        self.g = g

    def __enter__(self):
        _FakeGraph.current = self.g
        return self

    def __exit__(self, *exc):
        _FakeGraph.current = None
        return False


def _patch(monkeypatch):
    monkeypatch.setattr(torch.cuda, "CUDAGraph", _FakeGraph)
    monkeypatch.setattr(torch.cuda, "graph", _Capture)
    monkeypatch.setattr(torch.cuda, "synchronize", lambda *a, **k: None)


def _fwd_recording(calls):
    """fwd(w, x) = w * x into a fresh output; while capturing, registers a
    replay closure that writes into the output returned at capture."""

    def fwd(w, x):
        calls.append("run")
        out = w * x
        g = _FakeGraph.current
        if g is not None:
            def again(w=w, x=x, out=out):
                out.copy_(w * x)
            g.fn = again
        return out
    return fwd


def test_warmup_capture_replay_and_weight_change(monkeypatch):
    """One input tensor refilled in place between calls (read where it is)."""
    _patch(monkeypatch)
    calls = []
    w = torch.full((4,), 2.0)
    x = torch.ones(4)
    f = graphs.HipGraphForward(_fwd_recording(calls), static_args={0}, warmup=2)
    assert torch.equal(f(w, x), w * x) and torch.equal(f(w, x), w * x)      # warm-up: plain calls
    assert f.captures == 0 and len(calls) == 2
    x.fill_(3.0)
    y = f(w, x)                                                               # capture + replay
    assert f.captures == 1 and f.replays == 1 and torch.equal(y, w * x)
    x.fill_(5.0)
    y2 = f(w, x)                                                              # replay only: static output reused
    assert f.replays == 2 and y2 is y and torch.equal(y2, w * x) and len(calls) == 3
    w.mul_(10.0)                                                              # weight modified in place
    y3 = f(w, x)
    assert f.captures == 1 and torch.equal(y3, w * x) and y3 is not y         # plain call on the new weight
    x.fill_(7.0)
    y4 = f(w, x)                                                              # captured again
    assert f.captures == 2 and torch.equal(y4, w * x)


def test_new_input_address_switches_to_private_buffers(monkeypatch):
    _patch(monkeypatch)
    w = torch.full((4,), 2.0)
    f = graphs.HipGraphForward(_fwd_recording([]), static_args={0}, warmup=0)
    x1, x2, x3 = torch.ones(4), torch.full((4,), 3.0), torch.full((4,), 5.0)
    assert torch.equal(f(w, x1), w * x1) and f.captures == 1                 # captured over x1 itself
    assert torch.equal(f(w, x2), w * x2) and f.captures == 2                 # another address: private buffers
    assert torch.equal(f(w, x3), w * x3) and torch.equal(f(w, x1), w * x1) and f.captures == 2
    assert torch.equal(x1, torch.ones(4))                                     # the caller's tensors untouched


def test_replaced_weight_storage_recaptures(monkeypatch):
    _patch(monkeypatch)
    f = graphs.HipGraphForward(_fwd_recording([]), static_args={0}, warmup=0)
    w1, w2, x = torch.full((4,), 2.0), torch.full((4,), 7.0), torch.ones(4)
    assert torch.equal(f(w1, x), w1 * x) and f.captures == 1
    assert torch.equal(f(w2, x), w2 * x) and f.captures == 1   # another storage: plain call
    assert torch.equal(f(w2, x), w2 * x) and f.captures == 2


def test_capture_failure_keeps_the_plain_forward(monkeypatch):
    """An operation the stream capture refuses: a warning, the call's result
    from the plain forward, and no further capture attempts."""
    _patch(monkeypatch)
    calls = []

    def fwd(w, x):
        calls.append("run")
        if _FakeGraph.current is not None:
            raise RuntimeError("operation not permitted when stream is capturing")
        return w * x

    w, x = torch.full((4,), 2.0), torch.ones(4)
    f = graphs.HipGraphForward(fwd, static_args={0}, warmup=1)
    assert torch.equal(f(w, x), w * x) and f.capture_error is None
    with pytest.warns(RuntimeWarning, match="capture failed"):
        y = f(w, x)
    assert torch.equal(y, w * x) and f.captures == 0 and "not permitted" in f.capture_error
    n = len(calls)
    x.fill_(3.0)
    assert torch.equal(f(w, x), w * x) and len(calls) == n + 1 and f.captures == 0


def test_static_shapes_rule():
    assert not graphs.static_shapes([torch.ones(2)])            # off the GPU
    assert not graphs.static_shapes([1.0])


def test_compiler_declines_the_graph_off_the_gpu(monkeypatch):
    monkeypatch.setattr(comp, "build_hip_launcher",
                        lambda group, eager_fn=None: comp.EagerGroupLauncher(group.eager_module))
    torch.manual_seed(0)
    m = TransformerMLP(64, 256).to(torch.bfloat16).eval()
    x = torch.randn(32, 64, dtype=torch.bfloat16)
    be = FuseMLCompiler(require_gfx950=False, min_output_elements=0, fuse_mlp_block=False, hip_graph=True)
    torch._dynamo.reset()
    with torch.no_grad():
        out = torch.compile(m, backend=be)(x)
    assert torch.equal(out, m(x))
    assert be.dispatch and be.dispatch[0].startswith("direct (no HIP graph") and be.graph_forwards == []
