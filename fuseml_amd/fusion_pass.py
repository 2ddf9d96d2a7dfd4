"""Fusion discovery and graph surgery over an ATen-level FX graph.

Behaviour follows the reference pass (fuseml/passes/fusion_pass.py) so that
the groups reaching the HIP path are the ones the reference would form:

* triggers are ``aten.addmm`` / ``aten.mm`` (fuseml/passes/topology.py:55-58);
* greedy forward absorption while the current node has exactly one user
  (fusion_pass.py:203-291): pointwise ops (relu, gelu, sigmoid, add, mul and
  their in-place forms when the mutated value is the group's own) are
  absorbed; shape-preserving 2-D views are absorbed as no-ops; a
  ``keepdim=False`` reduction (sum.dim_IntList, amax, mean.dim) is absorbed and
  ends the group; anything else ends it;
* escape analysis: group nodes other than the output with users outside the
  group become ``intermediate_outputs`` (300-329);
* only groups with at least one absorbed node are kept (335-345), with the
  output metadata and an args snapshot of every node (342-343);
* surgery inserts ``call_function(fuseml_fused_kernel_placeholder,
  *group.inputs)`` after the output node with ``meta["fusion_group"]``
  (687-704) and rewires consumers, through ``operator.getitem`` when the group
  returns several values (783-887).

Extension (off by default, so default discovery is the reference's):
``fuse_sibling_reductions=True`` lets a node whose users are several
reductions over the same axis (plus any other consumers) absorb all of them;
the reduced value itself then escapes.  That is the only way the C4 workload
(``h.sum(-1), h.amax(-1), h.mean(-1)`` of one ``h``) becomes one kernel.

Extension (off by default): ``fuse_leading_views=True`` also absorbs a view,
reshape or _unsafe_view that only splits or merges the row dimension of the
group's value ([M,N] <-> [*lead, N], fuseml/passes/fusion_pass.py:537-579 stops
there), when the node after it is itself absorbed.  ``nn.Linear`` on a [B,S,D]
activation lowers to ``view -> addmm -> view(B,S,N) -> pointwise``, so this is
what lets 3-D (transformer-shaped) activations fuse; the trailing flatten that
feeds the next GEMM stays outside the group.

Each kept group also gets ``eager_module``: a standalone GraphModule of its
original nodes, the eager fallback for that group.
"""

from __future__ import annotations

import logging
import operator
from typing import Any, Dict, List, Optional, Sequence, Set

import torch
import torch.fx
from torch.fx.passes.shape_prop import ShapeProp

from .epilogue import (
    ADD_TARGETS,
    GELU_TARGETS,
    MUL_TARGETS,
    REDUCTION_TARGETS,
    TRANSPARENT_TARGETS,
    TRIGGER_TARGETS,
    UNARY_TARGETS,
    UnsupportedGroup,
    _group_args,
    group_nodes,
    input_slots,
    is_full_reduction,
    leading_dim_view,
    reduction_dims,
    transparent_is_identity,
)
from .fusion_group import FusionGroup

logger = logging.getLogger("fuseml_amd")

aten = torch.ops.aten

INPLACE_TARGETS = {aten.relu_.default, aten.add_.Tensor, aten.mul_.Tensor, aten.sigmoid_.default}
POINTWISE_TARGETS = set(UNARY_TARGETS) | set(GELU_TARGETS) | set(ADD_TARGETS) | set(MUL_TARGETS)


def fuseml_fused_kernel_placeholder(*args):
    """Stand-in target of a fused group until the compiler binds a launcher.

    Same contract as the reference's placeholder (fusion_pass.py:45-55): it is
    never meant to run, and raises if it does.
    """
    raise RuntimeError(
        "fuseml_fused_kernel_placeholder must be replaced by a fused launcher before execution"
    )


def group_result_nodes(group: Any) -> List[torch.fx.Node]:
    """Nodes whose values a fused call returns, in return order: the output
    node, any sibling reductions, then the escapes (the order of the surgery's
    ``getitem`` indices, fuseml/passes/fusion_pass.py:824-880)."""
    return [group.output_node, *(getattr(group, "sibling_outputs", None) or []),
            *(getattr(group, "intermediate_outputs", None) or [])]


def group_eager_module(group: Any) -> torch.fx.GraphModule:
    """The group's own nodes as a standalone GraphModule: ``*group.inputs -> results``.

    Built only from the reference's ``FusionGroup`` fields (fuseml/fusion_group.py:74-85):
    ``inputs``, ``base_node``/``fused_nodes`` with their targets and kwargs,
    ``node_args_snapshot`` for their args (surgery erases the nodes and FX
    nulls their Node arguments, fusion_pass.py:342-343), ``output_node`` and
    ``intermediate_outputs``.  It is the eager fallback of a fused launch and
    the callable bound when no kernel variant fits, so no raising placeholder
    is ever left in the graph (the reference's compiler keeps one,
    fuseml/compiler.py:393-398).  An operand that the reference resolved
    through view ops to their source is re-viewed here from the live view
    nodes; raises :class:`UnsupportedGroup` if those are gone.
    """
    slots, via_view = input_slots(group)
    g = torch.fx.Graph()
    inputs = list(group.inputs)
    ph = [g.placeholder(f"in{i}") for i in range(len(inputs))]
    env: Dict[int, torch.fx.Node] = {}

    def external(a: torch.fx.Node) -> torch.fx.Node:
        if id(a) in env:
            return env[id(a)]
        slot = slots[id(a)]
        val = ph[slot]
        if id(a) in via_view:
            chain = []
            cur = a
            while cur is not inputs[slot]:
                if (getattr(cur, "op", None) != "call_function" or cur.target not in TRANSPARENT_TARGETS
                        or not cur.args or not isinstance(cur.args[0], torch.fx.Node)):
                    raise UnsupportedGroup(f"view chain from {inputs[slot]} to {a.name} is not available")
                chain.append(cur)
                cur = cur.args[0]
            for v in reversed(chain):
                val = g.call_function(v.target, (val, *v.args[1:]), dict(v.kwargs))
        env[id(a)] = val
        return val

    members = {id(n) for n in group_nodes(group)}

    def arg(a: Any) -> Any:
        if isinstance(a, torch.fx.Node):
            return env[id(a)] if id(a) in members else external(a)
        if isinstance(a, (list, tuple)):
            return type(a)(arg(x) for x in a)
        return a

    for n in group_nodes(group):
        args = tuple(arg(a) for a in _group_args(group, n))
        if any(isinstance(v, torch.fx.Node) for v in n.kwargs.values()):
            raise UnsupportedGroup(f"{n.name}: a tensor keyword argument is not part of the group's inputs")
        env[id(n)] = g.call_function(n.target, args, dict(n.kwargs))
    res = [env[id(n)] for n in group_result_nodes(group)]
    g.output(res[0] if len(res) == 1 else tuple(res))
    return torch.fx.GraphModule(torch.nn.Module(), g)


def _meta_shape(node: Any):
    if not isinstance(node, torch.fx.Node):
        return None
    tm = node.meta.get("tensor_meta")
    if tm is not None and hasattr(tm, "shape"):
        return tuple(tm.shape)
    val = node.meta.get("val")
    if val is not None and hasattr(val, "shape"):
        return tuple(val.shape)
    return None


def _meta_dict(node: torch.fx.Node) -> Dict[str, Any]:
    tm = node.meta.get("tensor_meta")
    if tm is not None and hasattr(tm, "shape"):
        return {"shape": tuple(tm.shape), "stride": tuple(tm.stride), "dtype": tm.dtype}
    val = node.meta.get("val")
    if val is not None and hasattr(val, "shape"):
        return {"shape": tuple(val.shape), "stride": tuple(val.stride()), "dtype": val.dtype}
    return {}


def _keepdim(node: torch.fx.Node) -> bool:
    if len(node.args) > 2:
        return bool(node.args[2])
    return bool(node.kwargs.get("keepdim", False))


def _red_dims(node: torch.fx.Node):
    dims = reduction_dims(node)
    if is_full_reduction(dims):
        return None
    return tuple(int(d) % 2 for d in (dims if isinstance(dims, (list, tuple)) else [dims]))


def _fusible_reduction(node: torch.fx.Node) -> bool:
    """A row/column reduction the kernel can take: keepdim=False and a ``dim``.

    A reduction with ``dim`` omitted, None or empty reduces every element to a
    0-d result; it stays outside the group (the reference absorbs it and its
    kernel reduces along one axis only, kernel_generator.py:1909-1931).
    """
    return not _keepdim(node) and not is_full_reduction(reduction_dims(node))


class FuseMLFusionPass:
    """Find fusion groups in an ATen graph and replace them with placeholders."""

    def __init__(self, graph_module: torch.fx.GraphModule, registry: Any = None,
                 fuse_sibling_reductions: bool = False, fuse_leading_views: bool = False) -> None:
        self.graph_module = graph_module
        self.registry = registry
        self.fuse_sibling_reductions = fuse_sibling_reductions
        self.fuse_leading_views = fuse_leading_views
        self.groups: List[FusionGroup] = []

    # ------------------------------------------------------------------
    def run(self, example_inputs: Optional[Sequence[Any]] = None) -> torch.fx.GraphModule:
        if example_inputs is not None and not self._has_meta():
            ShapeProp(self.graph_module).propagate(*example_inputs)
        self.groups = self._find_fusion_groups()
        if self.groups:
            self._apply_surgery(self.groups)
        return self.graph_module

    def _has_meta(self) -> bool:
        for n in self.graph_module.graph.nodes:
            if n.op == "call_function" and n.target in TRIGGER_TARGETS:
                return "val" in n.meta or "tensor_meta" in n.meta
        return True

    # ------------------------------------------------------------------
    @staticmethod
    def _shape_preserving_2d(node: torch.fx.Node) -> bool:
        """A 2-D view op that changes neither the shape nor the element order.

        The reference absorbs any shape-preserving transparent op
        (fusion_pass.py:537-579); a non-identity ``permute`` of a square value
        keeps the shape but transposes it, so it is not absorbed here.
        """
        src = node.args[0] if node.args else None
        a, b = _meta_shape(src), _meta_shape(node)
        return (a is not None and b is not None and len(a) == 2 and a == b
                and transparent_is_identity(node))

    _LEADING_VIEW_TARGETS = (aten.view.default, aten._unsafe_view.default, aten.reshape.default)

    def _leading_view(self, node: torch.fx.Node) -> bool:
        """A row-dimension-only view whose single user the group absorbs next."""
        if not self.fuse_leading_views or node.target not in self._LEADING_VIEW_TARGETS:
            return False
        src = node.args[0] if node.args else None
        if not leading_dim_view(_meta_shape(src), _meta_shape(node)):
            return False
        users = list(node.users)
        if len(users) != 1 or users[0].op != "call_function":
            return False
        u = users[0]
        if u.target in REDUCTION_TARGETS:
            return _fusible_reduction(u)
        if u.target in INPLACE_TARGETS:
            return bool(u.args) and u.args[0] is node
        return u.target in POINTWISE_TARGETS

    def _sibling_reductions(self, node: torch.fx.Node) -> List[torch.fx.Node]:
        """Reduction users of `node` that can be fused together (same axis, no keepdim)."""
        reds = [u for u in node.users if u.op == "call_function" and u.target in REDUCTION_TARGETS]
        if len(reds) < 1:
            return []
        if not all(_fusible_reduction(u) for u in reds):
            return []
        axes = {_red_dims(u) for u in reds}
        if len(axes) != 1:
            return []
        kinds = [REDUCTION_TARGETS[u.target] for u in reds]
        if len(set(kinds)) != len(kinds):
            return []
        order = {n: i for i, n in enumerate(self.graph_module.graph.nodes)}
        return sorted(reds, key=lambda u: order[u])

    @staticmethod
    def _collect_inputs(node: torch.fx.Node, members: Set[torch.fx.Node], group: FusionGroup) -> None:
        for arg in node.args:
            if isinstance(arg, torch.fx.Node) and arg not in members and arg not in group.inputs:
                group.inputs.append(arg)

    def _find_fusion_groups(self) -> List[FusionGroup]:
        groups: List[FusionGroup] = []
        consumed: Set[torch.fx.Node] = set()
        for node in self.graph_module.graph.nodes:
            if node.op != "call_function" or node.target not in TRIGGER_TARGETS or node in consumed:
                continue
            group = FusionGroup(base_node=node)
            members: Set[torch.fx.Node] = {node}
            consumed.add(node)
            self._collect_inputs(node, members, group)

            def absorb(n: torch.fx.Node, is_output: bool = True) -> None:
                group.fused_nodes.append(n)
                members.add(n)
                consumed.add(n)
                self._collect_inputs(n, members, group)
                if is_output:
                    group.output_node = n

            current = node
            while True:
                users = list(current.users)
                if len(users) != 1:
                    if self.fuse_sibling_reductions and len(users) > 1 and current is not node:
                        reds = self._sibling_reductions(current)
                        if len(reds) >= 2:
                            absorb(reds[0])
                            for r in reds[1:]:
                                absorb(r, is_output=False)
                                group.sibling_outputs.append(r)
                    break
                nxt = users[0]
                if nxt.op != "call_function":
                    break
                t = nxt.target
                if t in REDUCTION_TARGETS:
                    if not _fusible_reduction(nxt):
                        break
                    absorb(nxt)
                    break
                if t in TRANSPARENT_TARGETS:
                    if self._shape_preserving_2d(nxt) or self._leading_view(nxt):
                        absorb(nxt, is_output=False)
                        current = nxt
                        continue
                    break
                if t in INPLACE_TARGETS:
                    # Safe only when the mutated value is the group's own.
                    if nxt.args and nxt.args[0] is current:
                        absorb(nxt)
                        current = nxt
                        continue
                    break
                if t in POINTWISE_TARGETS:
                    absorb(nxt)
                    current = nxt
                    continue
                break

            # Escapes: group nodes other than the returned ones with outside users.
            returned = {group.output_node, *group.sibling_outputs}
            for n in group.all_nodes:
                if n in returned:
                    continue
                if any(u not in members for u in n.users):
                    group.intermediate_outputs.append(n)
            if len(group) > 1 and not self._placeable(group, members):
                logger.debug("dropping %s: a returned value is consumed before its inputs exist", group)
                continue
            if len(group) > 1:
                group.output_metadata = _meta_dict(group.output_node)
                for n in group.all_nodes:
                    group.node_args_snapshot[n.name] = tuple(n.args)
                self._resolve_params(group)
                group.eager_module = group_eager_module(group)
                groups.append(group)
        return groups

    @staticmethod
    def _anchor(group: FusionGroup, order: Dict[torch.fx.Node, int]) -> torch.fx.Node:
        return max([group.base_node, *group.inputs], key=lambda n: order[n])

    def _placeable(self, group: FusionGroup, members: Set[torch.fx.Node]) -> bool:
        """Every outside consumer of a returned value follows the insertion point."""
        order = {n: i for i, n in enumerate(self.graph_module.graph.nodes)}
        at = order[self._anchor(group, order)]
        for n in group.result_nodes:
            for u in n.users:
                if u not in members and order[u] <= at:
                    return False
        return True

    def _resolve_params(self, group: FusionGroup) -> None:
        for n in group.inputs:
            if n.op == "get_attr":
                obj: Any = self.graph_module
                try:
                    for part in str(n.target).split("."):
                        obj = getattr(obj, part)
                except AttributeError:
                    continue
                if isinstance(obj, torch.Tensor):
                    group.param_bindings[str(n.target)] = obj

    # ------------------------------------------------------------------
    def _apply_surgery(self, groups: List[FusionGroup]) -> None:
        graph = self.graph_module.graph
        order = {n: i for i, n in enumerate(graph.nodes)}
        for group in groups:
            members = set(group.all_nodes)
            results = group.result_nodes
            # Insert right after the last input definition (or the base node):
            # every consumer of a returned value comes later (checked at discovery).
            anchor = self._anchor(group, order)
            with graph.inserting_after(anchor):
                fused = graph.call_function(fuseml_fused_kernel_placeholder, args=tuple(group.inputs))
            order[fused] = order[anchor]
            fused.meta["fusion_group"] = group
            fused.meta["fused_op_names"] = [n.name for n in group.all_nodes]
            replaced: Dict[torch.fx.Node, torch.fx.Node] = {}
            if len(results) == 1:
                if "tensor_meta" in group.output_node.meta:
                    fused.meta["tensor_meta"] = group.output_node.meta["tensor_meta"]
                if "val" in group.output_node.meta:
                    fused.meta["val"] = group.output_node.meta["val"]
                self._rewire(group.output_node, fused, members)
                replaced[group.output_node] = fused
            else:
                last = fused
                for k, n in enumerate(results):
                    with graph.inserting_after(last):
                        item = graph.call_function(operator.getitem, args=(fused, k))
                    for key in ("tensor_meta", "val"):
                        if key in n.meta:
                            item.meta[key] = n.meta[key]
                    self._rewire(n, item, members)
                    replaced[n] = item
                    last = item
            # Later groups may list a node this group returned as an input
            # (e.g. GEMM2 consuming GEMM1's GELU): point them at its replacement
            # (the reference patches the same lists, fusion_pass.py:716-740).
            for other in groups:
                if other is not group:
                    other.inputs = [replaced.get(n, n) for n in other.inputs]
                    other.node_args_snapshot = {
                        k: tuple(replaced.get(a, a) if isinstance(a, torch.fx.Node) else a for a in v)
                        for k, v in other.node_args_snapshot.items()
                    }
                    for n in list(replaced):
                        order.setdefault(replaced[n], order[anchor])
            for n in reversed(group.all_nodes):
                if len(n.users) == 0:
                    graph.erase_node(n)
        graph.eliminate_dead_code()
        graph.lint()
        self.graph_module.recompile()

    @staticmethod
    def _rewire(old: torch.fx.Node, new: torch.fx.Node, members: Set[torch.fx.Node]) -> None:
        for user in list(old.users):
            if user in members or user is new:
                continue
            user.replace_input_with(old, new)
