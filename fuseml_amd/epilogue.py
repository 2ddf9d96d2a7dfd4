"""Epilogue specification: what one fused kernel launch computes.

An :class:`EpilogueSpec` is the host-side description of one fusion group in
the vocabulary of the C ABI: which launcher inputs are the GEMM operands, the
ordered register ops applied to the fp32 accumulator, the escape stores, the
fused reductions, and the order of the returned tensors.

:func:`spec_from_group` derives it from a :class:`~fuseml_amd.fusion_group.FusionGroup`.
It replaces the reference's descriptor/codegen glue (fuseml/compiler.py:443-585
``_build_launcher`` and the epilogue emitters of
fuseml/codegen/kernel_generator.py:912-1065, 1599-2018) with the same op
semantics and three corrections:

* the addmm bias is bound by ROLE (``addmm.args[0]``), not by rank — the
  reference adds every 1-D input after the K loop (kernel_generator.py:884-901);
* ``gelu(approximate='tanh')`` is honoured — the reference always emits the erf
  form (kernel_generator.py:1607-1642);
* ``add``'s ``alpha`` and ``addmm``'s ``alpha``/``beta`` are honoured.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Any, Dict, List, Optional, Sequence, Tuple

import torch

aten = torch.ops.aten

TRIGGER_TARGETS = (aten.addmm.default, aten.mm.default)
UNARY_TARGETS = {
    aten.relu.default: "relu",
    aten.relu_.default: "relu",
    aten.sigmoid.default: "sigmoid",
    aten.sigmoid_.default: "sigmoid",
}
GELU_TARGETS = (aten.gelu.default,)
ADD_TARGETS = (aten.add.Tensor, aten.add_.Tensor)
MUL_TARGETS = (aten.mul.Tensor, aten.mul_.Tensor)
REDUCTION_TARGETS = {
    aten.sum.dim_IntList: "sum",
    aten.amax.default: "amax",
    aten.mean.dim: "mean",
}
# Shape-preserving view ops the discovery pass may absorb; no-ops in the kernel
# (fuseml/passes/topology.py:84-96).
TRANSPARENT_TARGETS = (
    aten.view.default,
    aten._unsafe_view.default,
    aten.reshape.default,
    aten.unsqueeze.default,
    aten.squeeze.dim,
    aten.expand.default,
    aten.permute.default,
    aten.slice.Tensor,
    aten.select.int,
)

SUPPORTED_DTYPES = (torch.bfloat16, torch.float16)


class UnsupportedGroup(ValueError):
    """The group cannot be expressed as one kernel launch (-> eager bypass)."""


@dataclass(frozen=True)
class EpiOp:
    """One register op on the accumulator.

    kind:    add | mul | relu | gelu_erf | gelu_tanh | sigmoid | scale |
             add_scalar | store | add_self | mul_self
    operand: launcher input index (add/mul) or escape-output index (store)
    scalar:  add: multiplier of the operand; scale/add_scalar/add_self: value
    """

    kind: str
    operand: int = -1
    scalar: float = 1.0


@dataclass(frozen=True)
class EpilogueSpec:
    left: int
    right: int
    ops: Tuple[EpiOp, ...]
    out_dtype: torch.dtype
    store_tile: bool = True
    reductions: Tuple[str, ...] = ()
    reduce_axis: int = 1
    reduce_dtypes: Tuple[torch.dtype, ...] = ()
    extra_dtypes: Tuple[torch.dtype, ...] = ()
    # Return order: ("tile",), ("red", name) or ("extra", k).
    outputs: Tuple[Tuple[Any, ...], ...] = (("tile",),)
    # N-D groups (the GEMM's [M,N] result viewed as [*lead, N]): the value shape
    # each such operand is broadcast against, as (input index, shape) pairs, and
    # the shape each returned value is viewed as (None: the natural [M,N]/[M]/[N]).
    operand_shapes: Tuple[Tuple[int, Tuple[int, ...]], ...] = ()
    output_shapes: Tuple[Optional[Tuple[int, ...]], ...] = ()

    def chain(self) -> List[Tuple[str, int, float]]:
        """Plain-data form of the op chain, as consumed by the CPU oracle."""
        return [(o.kind, o.operand, float(o.scalar)) for o in self.ops]

    def describe(self) -> str:
        parts = [o.kind if o.operand < 0 else f"{o.kind}[{o.operand}]" for o in self.ops]
        red = f" | {'+'.join(self.reductions)}(axis={self.reduce_axis})" if self.reductions else ""
        return f"gemm({self.left},{self.right}) -> {' -> '.join(parts) or 'id'}{red}"


# ---------------------------------------------------------------------------
# FusionGroup -> EpilogueSpec
# ---------------------------------------------------------------------------


def _node_dtype(node: Any) -> Optional[torch.dtype]:
    meta = getattr(node, "meta", {}) or {}
    tm = meta.get("tensor_meta")
    if tm is not None and hasattr(tm, "dtype"):
        return tm.dtype
    val = meta.get("val")
    if val is not None and hasattr(val, "dtype"):
        return val.dtype
    return None


def _is_node(x: Any) -> bool:
    return isinstance(x, torch.fx.Node)


def _node_shape(node: Any) -> Optional[Tuple[int, ...]]:
    meta = getattr(node, "meta", {}) or {}
    for key in ("tensor_meta", "val"):
        v = meta.get(key)
        if v is not None and hasattr(v, "shape"):
            try:
                return tuple(int(d) for d in v.shape)
            except (TypeError, ValueError):  # symbolic sizes
                return None
    return None


def leading_dim_view(src_shape: Optional[Tuple[int, ...]], out_shape: Optional[Tuple[int, ...]]) -> bool:
    """A view between [*a, N] and [*b, N] with prod(a) == prod(b): only the row
    (M) dimension is split or merged, so the row-major [M,N] layout is unchanged."""
    if not src_shape or not out_shape or len(src_shape) < 2 or len(out_shape) < 2:
        return False
    if src_shape[-1] != out_shape[-1]:
        return False
    pa = pb = 1
    for d in src_shape[:-1]:
        pa *= d
    for d in out_shape[:-1]:
        pb *= d
    return pa == pb


def _group_args(group: Any, node: torch.fx.Node) -> tuple:
    snap = getattr(group, "node_args_snapshot", None) or {}
    return tuple(snap.get(node.name, node.args))


def group_nodes(group: Any) -> List[Any]:
    """``base_node`` followed by ``fused_nodes`` (the reference's ``all_nodes``)."""
    return [group.base_node, *group.fused_nodes]


def input_slots(group: Any) -> Tuple[Dict[int, int], Dict[int, Any]]:
    """Launcher position of every external node the group's nodes consume.

    Returns ``(slots, via_view)``.  ``slots`` maps ``id(node)``, for each node
    that the argument snapshot names outside the group, to its index in
    ``group.inputs``.  ``via_view`` holds the operands that reach the group
    through a transparent view op: the launcher receives the view's source,
    not the view.

    Groups formed by this repository's pass name their inputs directly.  A
    group from the reference's own pass can differ in two ways, both handled
    by position (the reference collects inputs in first-appearance order over
    each node's args, fuseml/passes/fusion_pass.py:500-535):

    * its surgery patches ``inputs`` to the replacement of an earlier group's
      output but not ``node_args_snapshot`` (fusion_pass.py:716-727), so the
      snapshot still names the erased node;
    * it resolves an argument through transparent view ops to the defining
      node (fuseml/passes/topology.py:198-226).
    Raises :class:`UnsupportedGroup` when the two lists do not line up.
    """
    inputs = list(group.inputs)
    members = {id(n) for n in group_nodes(group)}
    ordered: List[Any] = []
    seen = set()
    for n in group_nodes(group):
        for a in _group_args(group, n):
            if _is_node(a) and id(a) not in members and id(a) not in seen:
                seen.add(id(a))
                ordered.append(a)
    direct = {id(n): i for i, n in enumerate(inputs)}
    if all(id(a) in direct for a in ordered):
        return {id(a): direct[id(a)] for a in ordered}, {}
    if len(ordered) != len(inputs):
        raise UnsupportedGroup(
            f"{len(inputs)} group inputs do not line up with the {len(ordered)} external arguments")
    slots: Dict[int, int] = {}
    via_view: Dict[int, Any] = {}
    for i, a in enumerate(ordered):
        if id(a) in direct and direct[id(a)] != i:
            raise UnsupportedGroup(f"input {a.name} is at position {direct[id(a)]}, expected {i}")
        slots[id(a)] = i
        if a is not inputs[i] and getattr(a, "op", None) == "call_function" and a.target in TRANSPARENT_TARGETS:
            via_view[id(a)] = a
    return slots, via_view


def reduction_dims(node: Any, args: Optional[tuple] = None) -> Any:
    """The ``dim`` argument of a sum.dim_IntList / amax / mean.dim node (None if absent)."""
    args = tuple(node.args) if args is None else tuple(args)
    if len(args) > 1:
        return args[1]
    return node.kwargs.get("dim")


def is_full_reduction(dims: Any) -> bool:
    """``dim`` None or empty: the op reduces over every element (a 0-d result).

    That is the meaning of an omitted or empty ``dim`` for ``amax`` and of
    ``dim=None`` / ``dim=[]`` for ``sum.dim_IntList`` and ``mean.dim``.  Such a
    reduction is not a row or column reduction of the tile.
    """
    if dims is None:
        return True
    return isinstance(dims, (list, tuple)) and len(dims) == 0


def transparent_is_identity(node: Any, args: Optional[tuple] = None) -> bool:
    """A shape-preserving transparent op that also keeps the element order.

    A ``permute`` with non-identity dims on a square value keeps the shape but
    transposes the data (the reference treats every shape-preserving
    transparent op as a no-op, fuseml/passes/topology.py:84-96, and would
    drop the transpose).  Strides are compared too when both nodes carry them.
    """
    args = tuple(node.args) if args is None else tuple(args)
    if node.target is aten.permute.default:
        dims = args[1] if len(args) > 1 else node.kwargs.get("dims")
        if dims is None:
            return False
        nd = len(dims)
        if [int(d) % nd for d in dims] != list(range(nd)):
            return False
    src = args[0] if args else None
    a, b = _node_stride(src), _node_stride(node)
    if a is not None and b is not None and a != b:
        return False
    return True


def _node_stride(node: Any) -> Optional[Tuple[int, ...]]:
    meta = getattr(node, "meta", {}) or {}
    tm = meta.get("tensor_meta")
    if tm is not None and hasattr(tm, "stride"):
        try:
            return tuple(int(s) for s in tm.stride)
        except (TypeError, ValueError):
            return None
    val = meta.get("val")
    if val is not None and hasattr(val, "stride"):
        try:
            return tuple(int(s) for s in val.stride())
        except (TypeError, ValueError):
            return None
    return None


def reduction_axis(dims: Any, ndim: int = 2) -> int:
    """Map reduction dims of a 2-D [M,N] value to a tile axis.

    Follows fuseml/codegen/kernel_generator.py:1909-1931: dims are normalised
    modulo 2; any 1 means "reduce along N" (axis 1, result [M]); otherwise axis 0.
    An N-D value ([*lead, N], ndim > 2) supports only the last dimension
    (axis 1, result [*lead]).  ``dim`` None or empty reduces over every
    element (a 0-d result), which is no tile axis: :class:`UnsupportedGroup`.
    """
    if is_full_reduction(dims):
        raise UnsupportedGroup("a reduction over all elements is not a row/column reduction")
    if isinstance(dims, int):
        dims = [dims]
    if ndim > 2:
        if sorted({int(d) % ndim for d in dims}) != [ndim - 1]:
            raise UnsupportedGroup("an N-D value is reduced only over its last dimension")
        return 1
    norm = [int(d) % 2 for d in dims]
    if len(set(norm)) > 1:
        raise UnsupportedGroup("reduction over both axes is not a single-axis row/column reduction")
    if 1 in norm:
        return 1
    return 0


def spec_from_group(group: Any) -> EpilogueSpec:
    """Build the launch spec of *group* (raises :class:`UnsupportedGroup`)."""
    base = group.base_node
    if base.target not in TRIGGER_TARGETS:
        raise UnsupportedGroup(f"base node {base.target} is not addmm/mm")
    index, via_view = input_slots(group)
    members = {id(n) for n in [base, *group.fused_nodes]}
    escapes = list(getattr(group, "intermediate_outputs", []) or [])
    escape_idx = {id(n): k for k, n in enumerate(escapes)}

    def input_index(n: Any) -> int:
        if not _is_node(n) or id(n) not in index:
            raise UnsupportedGroup(f"operand {n!r} is not a group input")
        if id(n) in via_view:
            raise UnsupportedGroup(f"operand {n.name} reaches the group through a view of another input")
        return index[id(n)]

    ops: List[EpiOp] = []
    bargs = _group_args(group, base)
    if base.target is aten.addmm.default:
        bias, mat1, mat2 = bargs[0], bargs[1], bargs[2]
        beta = float(base.kwargs.get("beta", 1))
        alpha = float(base.kwargs.get("alpha", 1))
        left, right = input_index(mat1), input_index(mat2)
        if alpha != 1.0:
            ops.append(EpiOp("scale", scalar=alpha))
        if beta != 0.0:
            if _is_node(bias):
                ops.append(EpiOp("add", operand=input_index(bias), scalar=beta))
            else:
                ops.append(EpiOp("add_scalar", scalar=beta * float(bias)))
    else:
        left, right = input_index(bargs[0]), input_index(bargs[1])
    if id(base) in escape_idx:
        ops.append(EpiOp("store", operand=escape_idx[id(base)]))

    reductions: List[Tuple[str, torch.dtype]] = []
    red_axis: Optional[int] = None
    red_source: Optional[int] = None
    tile_node = base
    # Shape of the value the ops act on: the GEMM's [M,N], or [*lead, N] after a
    # leading-dimension view.  Operands of ops on an N-D value are broadcast
    # against that shape (the launcher merges it back to [M,N]).
    base_shape = _node_shape(base)
    cur_shape = base_shape
    operand_shapes: Dict[int, Tuple[int, ...]] = {}

    def note_operand(k: int) -> None:
        if cur_shape is None or len(cur_shape) == 2:
            if k in operand_shapes:
                raise UnsupportedGroup("operand broadcast against values of different ranks")
            return
        if operand_shapes.setdefault(k, cur_shape) != cur_shape:
            raise UnsupportedGroup("operand broadcast against values of different shapes")

    for node in group.fused_nodes:
        t = node.target
        args = _group_args(group, node)
        if t in REDUCTION_TARGETS:
            src = args[0]
            if red_source is None:
                red_source = id(src)
            elif id(src) != red_source:
                raise UnsupportedGroup("reductions consume different values")
            keepdim = bool(args[2]) if len(args) > 2 else bool(node.kwargs.get("keepdim", False))
            if keepdim:
                raise UnsupportedGroup("keepdim=True reductions are not fused")
            ax = reduction_axis(reduction_dims(node, args), len(cur_shape) if cur_shape else 2)
            if red_axis is not None and ax != red_axis:
                raise UnsupportedGroup("sibling reductions along different axes")
            red_axis = ax
            dt = _node_dtype(node) or node.kwargs.get("dtype") or _node_dtype(src)
            reductions.append((REDUCTION_TARGETS[t], dt))
            continue
        if reductions:
            raise UnsupportedGroup("op after a reduction")
        if t in TRANSPARENT_TARGETS:
            new_shape = _node_shape(node)
            if new_shape == cur_shape and not transparent_is_identity(node, args):
                raise UnsupportedGroup(f"{node.name}: {t} keeps the shape but reorders the elements")
            if new_shape != cur_shape:
                if t is aten.permute.default:
                    raise UnsupportedGroup(f"{node.name}: permute changes the layout")
                if not leading_dim_view(cur_shape, new_shape):
                    raise UnsupportedGroup(f"{node.name}: view changes more than the row dimension")
                cur_shape = new_shape
            if id(node) in escape_idx:  # an escaping view holds the current value
                ops.append(EpiOp("store", operand=escape_idx[id(node)]))
            continue
        if t in UNARY_TARGETS:
            ops.append(EpiOp(UNARY_TARGETS[t]))
        elif t in GELU_TARGETS:
            approx = node.kwargs.get("approximate", args[1] if len(args) > 1 else "none")
            ops.append(EpiOp("gelu_tanh" if approx == "tanh" else "gelu_erf"))
        elif t in ADD_TARGETS or t in MUL_TARGETS:
            is_add = t in ADD_TARGETS
            alpha = float(node.kwargs.get("alpha", 1)) if is_add else 1.0
            a, b = args[0], args[1]
            a_in = _is_node(a) and id(a) in members
            b_in = _is_node(b) and id(b) in members
            if a_in and b_in:
                ops.append(EpiOp("add_self", scalar=alpha) if is_add else EpiOp("mul_self"))
            elif a_in or b_in:
                other = b if a_in else a
                if _is_node(other):
                    k = input_index(other)
                    note_operand(k)
                    if is_add:
                        if a_in:  # v + alpha * other
                            ops.append(EpiOp("add", operand=k, scalar=alpha))
                        else:  # other + alpha * v
                            if alpha != 1.0:
                                ops.append(EpiOp("scale", scalar=alpha))
                            ops.append(EpiOp("add", operand=k, scalar=1.0))
                    else:
                        ops.append(EpiOp("mul", operand=k))
                else:
                    s = float(other)
                    if is_add:
                        if a_in:
                            ops.append(EpiOp("add_scalar", scalar=alpha * s))
                        else:
                            if alpha != 1.0:
                                ops.append(EpiOp("scale", scalar=alpha))
                            ops.append(EpiOp("add_scalar", scalar=s))
                    else:
                        ops.append(EpiOp("scale", scalar=s))
            else:
                raise UnsupportedGroup(f"{node.name}: no operand comes from inside the group")
        else:
            raise UnsupportedGroup(f"op {t} has no epilogue implementation")
        tile_node = node
        if id(node) in escape_idx:
            ops.append(EpiOp("store", operand=escape_idx[id(node)]))

    out_node = group.output_node
    outputs: List[Tuple[Any, ...]] = []
    store_tile = True
    tile_dtype = _node_dtype(tile_node) or _node_dtype(out_node)
    if reductions:
        # Reduction groups return the reductions; a tile output is returned too
        # only if the tile node itself escapes (sibling-reduction groups list it
        # in intermediate_outputs).
        store_tile = False
        outputs = [("red", name) for name, _ in reductions]
    else:
        outputs = [("tile",)]
    extra_dtypes = []
    for k, n in enumerate(escapes):
        extra_dtypes.append(_node_dtype(n) or tile_dtype)
        outputs.append(("extra", k))
    if tile_dtype is None:
        meta = getattr(group, "output_metadata", {}) or {}
        tile_dtype = meta.get("dtype")
    if tile_dtype is None:
        raise UnsupportedGroup("output dtype unknown (run shape propagation)")
    names = [n for n, _ in reductions]
    if len(set(names)) != len(names):
        raise UnsupportedGroup("duplicate reduction kind in one group")
    # A reduced value that also escapes (sibling-reduction groups) is written
    # as the primary tile, which takes the coalesced staged-store path.
    if reductions and escapes and ops and ops[-1].kind == "store" and ops[-1].operand == len(escapes) - 1 \
            and escapes[-1] is tile_node:
        ops.pop()
        store_tile = True
        k = len(escapes) - 1
        outputs = [("tile",) if o == ("extra", k) else o for o in outputs]
        tile_dtype = extra_dtypes.pop()
    # Views of the returned values when the group's values are N-D.
    def view_of(shape: Optional[Tuple[int, ...]]) -> Optional[Tuple[int, ...]]:
        return shape if shape is not None and len(shape) != 2 else None

    output_shapes: List[Optional[Tuple[int, ...]]] = []
    for o in outputs:
        if o[0] == "tile":
            output_shapes.append(view_of(_node_shape(tile_node) if not reductions else cur_shape))
        elif o[0] == "extra":
            output_shapes.append(view_of(_node_shape(escapes[o[1]])))
        else:
            output_shapes.append(tuple(cur_shape[:-1]) if cur_shape is not None and len(cur_shape) > 2
                                 and red_axis == 1 else None)
    return EpilogueSpec(
        left=left,
        right=right,
        ops=tuple(ops),
        out_dtype=tile_dtype,
        store_tile=store_tile,
        reductions=tuple(names),
        reduce_axis=1 if red_axis is None else red_axis,
        reduce_dtypes=tuple(dt or torch.float32 for _, dt in reductions),
        extra_dtypes=tuple(extra_dtypes),
        outputs=tuple(outputs),
        operand_shapes=tuple(sorted(operand_shapes.items())),
        output_shapes=tuple(output_shapes) if any(sh is not None for sh in output_shapes) else (),
    )
