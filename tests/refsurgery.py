"""Reference-shaped fusion groups and surgery, for the drop-in boundary tests.

``RefGroup`` holds exactly the ten fields of the reference's dataclass
(fuseml/fusion_group.py:74-85) and nothing else: no ``eager_module`` and no
``sibling_outputs``.  ``reference_surgery`` rewrites a traced graph the way the
reference's pass leaves it (fuseml/passes/fusion_pass.py:644-778): one
placeholder per group with ``args=tuple(group.inputs)``, consumers rewired
(through ``getitem`` when the group has escapes), later groups' ``inputs``
patched to the replacements but their ``node_args_snapshot`` left as taken at
discovery, then the orphan sweep, which erases the group's nodes (FX nulls the
Node arguments of an erased node).  ``bind`` then replaces each placeholder by
``build(group)``, as the reference compiler's loop does (fuseml/compiler.py:343-409).
"""

from __future__ import annotations

import operator
from dataclasses import dataclass, field
from typing import Any, Dict, List

import torch
import torch.fx

from fuseml_amd.fusion_pass import FuseMLFusionPass, fuseml_fused_kernel_placeholder


@dataclass
class RefGroup:
    base_node: torch.fx.Node
    fused_nodes: List[torch.fx.Node] = field(default_factory=list)
    inputs: List[torch.fx.Node] = field(default_factory=list)
    output_node: torch.fx.Node = None  # type: ignore[assignment]
    output_metadata: Dict[str, Any] = field(default_factory=dict)
    intermediate_outputs: List[torch.fx.Node] = field(default_factory=list)
    param_bindings: Dict[str, Any] = field(default_factory=dict)
    node_args_snapshot: Dict[str, tuple] = field(default_factory=dict)
    fusion_strategy: str = "triton"
    cublas_pattern: Any = None

    @property
    def all_nodes(self) -> List[torch.fx.Node]:
        return [self.base_node] + self.fused_nodes

    def __len__(self) -> int:
        return 1 + len(self.fused_nodes)


@dataclass
class CublasPatternStub:
    """The fields of the reference's CublasEpiloguePattern (cublas_epilogue.py:100-137)."""

    epilogue_type: str
    trigger_node: Any
    absorbed_nodes: List[Any] = field(default_factory=list)
    output_node: Any = None
    has_bias: bool = True
    use_gelu: bool = True
    residual_arg_index: Any = None


def reference_groups(gm: torch.fx.GraphModule, example_inputs, cublas: bool = False) -> List[RefGroup]:
    """Discovery (same rules as the reference's pass), returned as RefGroups."""
    p = FuseMLFusionPass(gm)
    torch.fx.passes.shape_prop.ShapeProp(gm).propagate(*example_inputs)
    groups = []
    for g in p._find_fusion_groups():
        strategy, pattern = "triton", None
        if cublas:
            strategy = "cublas_epilogue"
            kinds = [n.target for n in g.fused_nodes]
            etype = "GELU_BIAS" if torch.ops.aten.gelu.default in kinds else (
                "RELU_BIAS" if torch.ops.aten.relu.default in kinds else "BIAS_RESIDUAL")
            pattern = CublasPatternStub(etype, g.base_node, list(g.fused_nodes), g.output_node,
                                        use_gelu=etype == "GELU_BIAS",
                                        residual_arg_index=0 if etype == "BIAS_RESIDUAL" else None)
        groups.append(RefGroup(
            base_node=g.base_node, fused_nodes=list(g.fused_nodes), inputs=list(g.inputs),
            output_node=g.output_node, output_metadata=dict(g.output_metadata),
            intermediate_outputs=list(g.intermediate_outputs), param_bindings=dict(g.param_bindings),
            node_args_snapshot=dict(g.node_args_snapshot), fusion_strategy=strategy, cublas_pattern=pattern))
    return groups


def reference_surgery(gm: torch.fx.GraphModule, groups: List[RefGroup]) -> List[torch.fx.Node]:
    graph = gm.graph
    placeholders = []
    for group in groups:
        with graph.inserting_after(group.output_node):
            ph = graph.call_function(fuseml_fused_kernel_placeholder, args=tuple(group.inputs))
        ph.meta["fusion_group"] = group
        if not group.intermediate_outputs:
            group.output_node.replace_all_uses_with(ph, propagate_meta=False)
            rewire = {group.output_node: ph}
        else:
            prev = ph
            rewire = {}
            for k, n in enumerate([group.output_node, *group.intermediate_outputs]):
                with graph.inserting_after(prev):
                    item = graph.call_function(operator.getitem, args=(ph, k))
                rewire[n] = item
                prev = item
            members = set(group.all_nodes)
            group.output_node.replace_all_uses_with(rewire[group.output_node], propagate_meta=False)
            for n, item in rewire.items():
                if n is group.output_node:
                    continue
                for u in list(n.users):
                    if u not in members and u is not item:
                        u.replace_input_with(n, item)
        for other in groups:
            if other is not group:
                other.inputs = [rewire.get(i, i) for i in other.inputs]
        placeholders.append(ph)
    for n in reversed(list(graph.nodes)):
        if len(n.users) == 0 and n.op in ("get_attr", "call_function") and \
                n.target is not fuseml_fused_kernel_placeholder:
            graph.erase_node(n)
    graph.eliminate_dead_code()
    graph.lint()
    gm.recompile()
    return placeholders


def bind(gm: torch.fx.GraphModule, placeholders: List[torch.fx.Node], build) -> List[Any]:
    """Replace each placeholder by build(group); return the callables bound."""
    bound = []
    for ph in placeholders:
        fn = build(ph.meta["fusion_group"])
        assert fn is not None, "the builder left the placeholder in the graph"
        with gm.graph.inserting_after(ph):
            new = gm.graph.call_function(fn, args=ph.args)
        ph.replace_all_uses_with(new)
        gm.graph.erase_node(ph)
        bound.append(fn)
    gm.graph.eliminate_dead_code()
    gm.recompile()
    return bound
