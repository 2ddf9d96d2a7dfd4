"""FusionGroup — the boundary type handed from graph analysis to the HIP path.

Field for field the reference's dataclass (fuseml/fusion_group.py:18-122): a
group produced by the reference's own ``FuseMLFusionPass`` can be passed to
:func:`fuseml_amd.compiler.build_hip_launcher` unchanged.  Two optional fields
are added, both defaulting to "absent", so the reference's groups need neither:

* ``sibling_outputs`` — further reduction nodes fused beside ``output_node``
  when the opt-in sibling-reduction discovery is on (several reductions of
  one value, as in ``h.sum(-1), h.amax(-1), h.mean(-1)``);
* ``eager_module`` — a standalone ``GraphModule`` holding the group's
  original nodes, used as the eager fallback (the reference's compiler never
  wires one, fuseml/compiler.py:572-582).
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Tuple, Union

import torch


@dataclass
class FusionGroup:
    base_node: torch.fx.Node
    fused_nodes: List[torch.fx.Node] = field(default_factory=list)
    inputs: List[torch.fx.Node] = field(default_factory=list)
    output_node: torch.fx.Node = None  # type: ignore[assignment]
    output_metadata: Dict[str, Any] = field(default_factory=dict)
    intermediate_outputs: List[torch.fx.Node] = field(default_factory=list)
    param_bindings: Dict[str, Union[torch.nn.Parameter, torch.Tensor]] = field(default_factory=dict)
    node_args_snapshot: Dict[str, tuple] = field(default_factory=dict)
    fusion_strategy: str = "hip"
    cublas_pattern: Any = None
    sibling_outputs: List[torch.fx.Node] = field(default_factory=list)
    eager_module: Optional[torch.fx.GraphModule] = None

    def __post_init__(self) -> None:
        if self.output_node is None:
            self.output_node = self.base_node

    @property
    def all_nodes(self) -> List[torch.fx.Node]:
        return [self.base_node] + self.fused_nodes

    @property
    def result_nodes(self) -> List[torch.fx.Node]:
        """Nodes whose values the fused call returns, in return order."""
        return [self.output_node, *self.sibling_outputs, *self.intermediate_outputs]

    @property
    def op_signature(self) -> Tuple[str, ...]:
        return tuple(str(n.target) for n in self.all_nodes if n.op == "call_function")

    def __len__(self) -> int:
        return 1 + len(self.fused_nodes)

    def __repr__(self) -> str:
        names = [n.name for n in self.all_nodes]
        return f"FusionGroup({' -> '.join(names)}, inputs={len(self.inputs)})"
