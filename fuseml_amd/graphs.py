"""HIP-graph replay of a compiled forward (``FuseMLCompiler(hip_graph=True)``).

On MI355X the reference's smaller presets run 10-40 us of kernels per forward,
so the host time of dispatching them (Dynamo's guards, the graph's Python, one
launcher call per fused group, the eager ops left in the graph) is most of what
a synchronised forward costs.  :class:`HipGraphForward` captures the fused
graph's forward once into a HIP graph (``torch.cuda.CUDAGraph``) and replays
it: the whole forward is one graph launch.  The graph reads the activations
where the call that captured it passed them while later calls pass the same
tensors (a benchmark loop, a serving loop over one input buffer); after the
first call with an activation at another address it is captured again over
private input buffers, and every call then copies its activations into them.

Semantics, as ``torch.compile(mode="reduce-overhead")``'s CUDA graphs:

* the returned tensors are the graph's static outputs, overwritten by the next
  call of the same compiled function (clone what must outlive it);
* parameters and buffers (the graph's static inputs) are read in place: a call
  whose static input was replaced (another storage) or modified in place (a
  new version counter) runs once without the graph and captures it again on
  the following call, so results always follow the current weights;
* the first ``warmup`` calls run without the graph (they build the launchers'
  plans and the single-kernel MLP's packed weights outside the capture);
* a forward that cannot be captured (an operation the stream capture refuses)
  is run without the graph from then on, with a warning: the capture error is
  not raised to the caller.

Only graphs with static shapes on one GPU are captured (the compiler checks);
the graph replays on the caller's current stream.  The reference has no
counterpart (it launches every kernel from Python on every call,
kernel_launcher.py:640-821).
"""

from __future__ import annotations

import warnings
from typing import Any, Callable, List, Optional, Sequence, Set

import torch


def static_shapes(inputs: Sequence[Any]) -> bool:
    """Every input is a CUDA tensor with concrete sizes and strides, all on one device."""
    devs = set()
    for t in inputs:
        if not isinstance(t, torch.Tensor) or t.device.type != "cuda":
            return False
        if any(isinstance(s, torch.SymInt) for s in (*t.shape, *t.stride())):
            return False
        devs.add(t.device)
    return len(devs) == 1


class HipGraphForward:
    """Callable replaying ``fwd`` from a HIP graph (see the module docstring).

    ``static_args`` holds the call-argument indices that are parameters or
    buffers (read in place, checked for identity and version on every call);
    the other arguments (activations) are read in place while they stay at the
    captured addresses, else copied into private buffers before each replay.
    ``params`` are tensors ``fwd`` reads that are not call arguments (lifted
    parameters bound by the caller), checked the same way.
    """

    def __init__(self, fwd: Callable, static_args: Set[int], params: Sequence[torch.Tensor] = (),
                 warmup: int = 2) -> None:
        self.__name__ = "fuseml_hip_graph_forward"
        self._fwd = fwd
        self._static_args = set(static_args)
        self._static_list = sorted(self._static_args)
        self._params = list(params)
        # Activations read in place (True) or copied into private buffers.
        self._alias = True
        self._alias_ptrs: List[tuple] = []
        self._warmup = warmup
        self._calls = 0
        self._graph: Optional[torch.cuda.CUDAGraph] = None
        self._bufs: List[Optional[torch.Tensor]] = []
        self._outputs: Any = None
        self._stamp: List[tuple] = []
        self.captures = 0
        self.replays = 0
        # Set when a capture failed: every later call runs fwd without a graph.
        self.capture_error: Optional[str] = None

    def _stamps(self, args: Sequence[torch.Tensor]) -> List[tuple]:
        return [(args[i].data_ptr(), args[i]._version) for i in self._static_list] + \
               [(p.data_ptr(), p._version) for p in self._params]

    def _capture(self, args: Sequence[torch.Tensor]) -> bool:
        """Capture fwd over ``args`` (or private copies); False if the capture failed."""
        self._graph = None
        dynamic = [i for i in range(len(args)) if i not in self._static_args]
        if self._alias:
            self._bufs = [None] * len(args)
            self._alias_ptrs = [(i, args[i].data_ptr()) for i in dynamic]
        else:
            self._bufs = [None if i in self._static_args else a.detach().clone() for i, a in enumerate(args)]
            self._alias_ptrs = []
        call = [a if b is None else b for a, b in zip(args, self._bufs)]
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        try:
            with torch.cuda.graph(g):
                out = self._fwd(*call)
        except Exception as exc:  # noqa: BLE001 - any capture failure: keep the plain forward
            self._graph, self._outputs, self._bufs = None, None, []
            self.capture_error = f"{type(exc).__name__}: {exc}"
            warnings.warn(f"fuseml: HIP-graph capture failed, running the forward without a graph "
                          f"({self.capture_error})", RuntimeWarning, stacklevel=3)
            return False
        self._graph, self._outputs = g, out
        self._stamp = self._stamps(args)
        self.captures += 1
        return True

    def __call__(self, *args: torch.Tensor) -> Any:
        if self.capture_error is not None:
            return self._fwd(*args)
        if self._graph is not None and self._stamps(args) != self._stamp:
            # a weight changed: this call without the graph (it also refreshes
            # what launchers derive from weights), the next captures again
            self._graph, self._outputs = None, None
            self._calls = self._warmup - 1
        if self._graph is not None and self._alias and any(args[i].data_ptr() != p for i, p in self._alias_ptrs):
            # an activation at another address: from now on over private buffers
            self._alias = False
            if not self._capture(args):
                return self._fwd(*args)
        if self._graph is None:
            self._calls += 1
            if self._calls <= self._warmup or not self._capture(args):
                return self._fwd(*args)
        for a, b in zip(args, self._bufs):
            if b is not None:
                b.copy_(a)
        self._graph.replay()
        self.replays += 1
        return self._outputs
