"""``FuseMLCompiler`` — the ``torch.compile`` backend, bound to the HIP kernel family.

Usage is the reference's (README.md:48-54)::

    compiled = torch.compile(model, backend=FuseMLCompiler())
    with torch.no_grad():
        out = compiled(x)

Pipeline (fuseml/compiler.py:173-437, same entry, same bypass, same
attributes ``fusion_applied`` / ``fusion_strategy`` / ``fusion_candidates``):

1. ``aot_module_simplified`` lowers the Dynamo graph to ATen.
2. Pre-scan: no ``addmm``/``mm`` trigger, or none worth fusing under the cost
   model -> ``_NoFusionPossible`` -> the original ``gm.forward`` is returned
   (no AOT wrapper on the bypass path, compiler.py:219-228).
3. :class:`~fuseml_amd.fusion_pass.FuseMLFusionPass` finds the groups and
   inserts placeholders.
4. Each placeholder is replaced by :func:`build_hip_launcher` — the HIP
   launcher wrapped in an eager fallback — or, when no kernel variant fits the
   group, by the group's eager closure.  A placeholder is never left in the
   graph (the reference keeps it when a build fails, compiler.py:393-398).

The cost model (replacing topology.py:479-571's NVIDIA tables and the
Triton/cuBLAS/bypass split) is two-way: the fused HIP kernel when the device
is gfx950, the operands are bf16/f16 (or fp32, run as a three-term bf16 split
product), the group fits one launch and its output
has at least ``min_output_elements`` (the reference's tiny-output rule,
fusion_pass.py:463 and 498, M*N < 500 000 bypasses; calibrated to 0 here, see
MIN_FUSION_OUTPUT_ELEMENTS), the GEMM is not a
few-tile problem with a long K loop, and the epilogue saves more than the K
loop gives up against hipBLASLt (:func:`fused_beats_eager`), else eager.  The last rule is measured on
MI355X (bias+GELU chains against eager addmm + GELU): with K >= 2048 and fewer
128x128 output tiles than the 256 CUs, each CU runs one tile's whole K loop
while hipBLASLt's stream-K kernel splits K, and the fused kernel runs at
0.41-0.91x of eager (K=8192, 1024x1024: 77 against 35 us); from 256 tiles on
every measured shape is at 0.88x or better, and at K = 1024 the fused kernel
wins at every size (1.2-1.36x below 256 tiles).
"""

from __future__ import annotations

import logging
from typing import Any, Callable, Dict, List, Optional, Tuple, Union

import torch
import torch.fx
from torch._functorch.aot_autograd import aot_module_simplified, make_boxed_func

from .cache import LauncherCache, launcher_cache_key
from .epilogue import TRIGGER_TARGETS, EpilogueSpec, UnsupportedGroup, spec_from_group
from .fusion_group import FusionGroup
from .fusion_pass import FuseMLFusionPass, fuseml_fused_kernel_placeholder, group_eager_module

logger = logging.getLogger("fuseml_amd")

# The reference bypasses groups whose output has fewer than 500 000 elements
# (fusion_pass.py:463 and 498).  Measured on MI355X, the fused launch costs less
# host time than the eager kernels it replaces at every size: the reference's
# "small" preset (128 rows, 256 -> 1024 -> 256) takes 47.9 us compiled with
# both groups fused against 62.4 us bypassed and 54.0 us eager, and fp32 C1
# (64 rows) 77.3 against 77.6 us.  So no floor by default;
# min_output_elements=REFERENCE_MIN_OUTPUT_ELEMENTS restores the reference's rule.
REFERENCE_MIN_OUTPUT_ELEMENTS = 500_000
MIN_FUSION_OUTPUT_ELEMENTS = 0
# Few-tile groups (fewer 128x128 output tiles than MIN_TILES_LONG_K, two per CU
# of MI355X's 256) run on one of the library's smaller tiles (PARTIAL_ROUND_TILES,
# the choice mirrored by partial_round_tile), whose K loop is bound by the rate at
# which each CU pulls its tiles' A and W rows through the LDS DMA: such a group
# fuses while K x (rows per CU, weighted as partial_round_tile weighs them) <=
# MAX_K_ROWS_PER_CU, measured on MI355X (profiles/cost_model_calibration.json:
# fused 0.37-0.80 of eager's time up to 614k, 1.00-1.09 at 768k-1229k, 1.07-1.31
# beyond).
MIN_TILES_LONG_K = 512
MAX_K_ROWS_PER_CU = 704 * 1024
MI355X_CUS = 256
# (BM, BN, lock-step?): the library's tiles below one round of 256x256 tiles
# (choose_partial_round in csrc/gemm_epilogue.hip): three lock-step tiles and
# the 256x128 ping-pong one.
PARTIAL_ROUND_TILES = ((128, 128, True), (64, 128, True), (32, 128, True), (256, 128, False))
# Fuse a group only while K <= K_PER_EPILOGUE_PASS * (elementwise passes the
# eager path would run over the [M,N] output) - K_CROSSOVER_OFFSET: the
# crossover measured on MI355X (fuseml_amd/calibration.py; the measurement is
# profiles/cost_model_calibration.json): 2048 for one pass, 11264 for four.
K_PER_EPILOGUE_PASS = 3072
K_CROSSOVER_OFFSET = 1024
# fp32 operands run as a three-term bf16 split product (K' = 3 ceil8(K)).
SUPPORTED_GEMM_DTYPES = (torch.bfloat16, torch.float16, torch.float32)


def effective_k(K: int, dtype: Any) -> int:
    """Length of the K loop the kernel runs: 3 ceil8(K) for fp32 operands (the
    split product), K otherwise."""
    return 3 * (-(-K // 8) * 8) if dtype == torch.float32 else K


class _NoFusionPossible(Exception):
    """No profitable fusion: return the original forward (no AOT overhead)."""


def aot_wrapper_is_identity(meta: Any, n_graph_inputs: int, n_call_inputs: int) -> Tuple[bool, str]:
    """Whether AOTAutograd's runtime wrapper around an inference graph would
    only call it: no input is mutated, no output aliases an input or an
    intermediate, no effect tokens, RNG functionalization, tensor subclasses,
    dynamic output dims or grad-mode changes, and the graph takes exactly the
    call's inputs (no deduplicated or synthetic-base inputs).  ``meta`` is the
    ``ViewAndMutationMeta`` AOTAutograd hands the forward compiler through the
    tracing context.  Then the graph's forward can be returned to Dynamo
    directly: per call that saves the wrapper's Python (about 20 us on the
    MI355X box's host, more than a kernel of the reference's smaller presets
    takes), with the same results."""
    if meta is None:
        return False, "no AOT metadata"
    try:
        from torch._functorch._aot_autograd.schemas import OutputType, PlainTensorMeta
    except ImportError:  # pragma: no cover - other torch layouts
        return False, "AOT schemas not importable"
    checks = [
        (not getattr(meta, "is_train", True), "training graph"),
        (n_graph_inputs == n_call_inputs, f"graph takes {n_graph_inputs} inputs for {n_call_inputs}"),
        (getattr(meta, "num_mutated_inp_runtime_indices", 1) == 0, "mutated inputs"),
        (not any(i.mutates_data or i.mutates_metadata or i.mutates_storage_metadata
                 for i in getattr(meta, "input_info", [None]) if i is not None), "mutated inputs"),
        (getattr(meta, "num_intermediate_bases", 1) == 0, "intermediate bases"),
        (getattr(meta, "num_outputs_aliased", 1) == 0, "aliased outputs"),
        (all(o.output_type == OutputType.non_alias for o in getattr(meta, "output_info", [])), "aliased outputs"),
        (not getattr(meta, "tokens", {1: 1}), "effect tokens"),
        (not getattr(meta, "is_rng_op_functionalized", True), "functionalized RNG"),
        (not getattr(meta, "dynamic_outputs", True), "dynamic outputs"),
        (getattr(meta, "grad_enabled_mutation", 0) is None, "grad-mode mutation"),
        (all(isinstance(s, (PlainTensorMeta, int)) for s in getattr(meta, "subclass_inp_meta", [None])),
         "tensor subclass inputs"),
        (all(isinstance(s, (PlainTensorMeta, int)) for s in getattr(meta, "subclass_fw_graph_out_meta", [None])),
         "tensor subclass outputs"),
    ]
    for ok, why in checks:
        if not ok:
            return False, why
    return True, "identity"


def _meta(node: Any):
    if not isinstance(node, torch.fx.Node):
        return None
    tm = node.meta.get("tensor_meta")
    if tm is not None and hasattr(tm, "shape"):
        return tm
    return node.meta.get("val")


def device_is_gfx950(device: Optional[torch.device] = None) -> bool:
    """True when `device` (default: current) is an MI355X-class gfx950 GPU."""
    if not torch.cuda.is_available():
        return False
    try:
        idx = torch.cuda.current_device() if device is None or device.index is None else device.index
        arch = getattr(torch.cuda.get_device_properties(idx), "gcnArchName", "")
    except Exception:  # pragma: no cover - no device
        return False
    return str(arch).startswith("gfx950")


def _gemm_dims(group: Any) -> Tuple[Optional[int], Any, Optional[int], Optional[int]]:
    """(K, dtype, M, N) of the group's GEMM from its operands' metadata (None
    where unknown)."""
    base = group.base_node
    args = (getattr(group, "node_args_snapshot", None) or {}).get(base.name, base.args)
    addmm = base.target is TRIGGER_TARGETS[0]
    mat1 = args[1] if addmm else args[0]
    mat2 = args[2] if addmm else args[1]
    m, w = _meta(mat1), _meta(mat2)
    if m is None or len(m.shape) != 2:
        return None, None, None, None
    try:
        K, M = int(m.shape[1]), int(m.shape[0])
    except (TypeError, ValueError):
        return None, None, None, None
    N = None
    if w is not None and len(w.shape) == 2:
        try:
            N = int(w.shape[1])
        except (TypeError, ValueError):
            N = None
    return K, getattr(m, "dtype", None), M, N


# Weight-streaming groups fuse while K <= this x elementwise passes
# (profiles/cost_model_calibration.json, decode rows: one pass 0.85-0.97 of
# eager's time at K = 2048-4096, 1.07 at K = 8192).
WEIGHT_STREAM_K_PER_PASS = 4096


def weight_streaming(M: int, N: int, cus: int = MI355X_CUS) -> bool:
    """Decode-sized M against a wide weight: M <= 128 with at least one
    128-column output tile per CU.  Both paths then stream the weight from HBM
    once (the library runs one row of tiles, in K stages of 64), so the fused
    kernel costs about eager's GEMM, saves its elementwise passes, and the
    few-tile rule does not apply (fused_beats_eager decides)."""
    return M <= 128 and -(-N // 128) >= cus


def partial_round_tile(M: int, N: int, K: int, cus: int = MI355X_CUS) -> Tuple[Tuple[int, int], float]:
    """The tile (BM, BN) the library runs an M x N x K GEMM on below one round
    of 256x256 tiles, and its busiest CU's K-loop work in operand rows per
    unit of K: ceil(tiles / cus) x (BM + BN), weighted by how fast a CU moves
    them (a lock-step tile x 1.6 when no CU holds two workgroups, x 1.4 for K >
    2048; the ping-pong tile x 1.2); the least, the first listed on a tie
    (choose_partial_round in csrc/gemm_epilogue.hip).  In the weight-streaming
    regime (weight_streaming) the tile with the smallest BM >= M."""
    if weight_streaming(M, N, cus):
        bm = 32 if M <= 32 else 64 if M <= 64 else 128
        tiles = -(-N // 128)
        return (bm, 128), -(-tiles // cus) * (bm + 128) * (1.6 if tiles <= cus else 1.0)
    one = 7 if K > 2048 else 8
    best: Optional[Tuple[Tuple[int, int], int]] = None
    for bm, bn, lockstep in PARTIAL_ROUND_TILES:
        tiles = -(-M // bm) * -(-N // bn)
        weight = (one if tiles <= cus else 5) if lockstep else 6
        work = -(-tiles // cus) * (bm + bn) * weight
        if best is None or work < best[1]:
            best = ((bm, bn), work)
    assert best is not None
    return best[0], best[1] / 5


def few_tile_verdict(M: int, N: int, k_loop: int, min_tiles: int = MIN_TILES_LONG_K) -> Optional[str]:
    """Why a few-tile group stays eager (None: no objection): fewer than
    ``min_tiles`` 128x128 output tiles and a K loop of ``k_loop`` over more
    than MAX_K_ROWS_PER_CU operand rows per CU."""
    tiles = -(-M // 128) * -(-N // 128)
    if tiles >= min_tiles:
        return None
    (bm, bn), rows = partial_round_tile(M, N, k_loop)
    if k_loop * rows <= MAX_K_ROWS_PER_CU:
        return None
    return (f"{tiles} output tiles at a K loop of {k_loop}: {rows:g} operand rows per CU on {bm}x{bn} tiles, "
            f"K x rows {k_loop * rows:.0f} > {MAX_K_ROWS_PER_CU}")


def trigger_is_fusible(node: torch.fx.Node, min_output_elements: int = MIN_FUSION_OUTPUT_ELEMENTS,
                       min_tiles_long_k: int = MIN_TILES_LONG_K) -> Tuple[bool, str]:
    """Cost model for one addmm/mm trigger: (fuse?, reason)."""
    if node.target is torch.ops.aten.addmm.default:
        mat1, mat2 = node.args[1], node.args[2]
    else:
        mat1, mat2 = node.args[0], node.args[1]
    m1, m2, out = _meta(mat1), _meta(mat2), _meta(node)
    if m1 is None or m2 is None or out is None:
        return False, "no shape metadata"
    if len(m1.shape) != 2 or len(m2.shape) != 2:
        return False, "GEMM operands are not 2-D"
    if m1.dtype not in SUPPORTED_GEMM_DTYPES or m2.dtype != m1.dtype:
        return False, f"GEMM dtype {m1.dtype}/{m2.dtype}: no MFMA variant (bf16, f16, fp32 split)"
    M, K = int(m1.shape[0]), int(m1.shape[1])
    N = int(m2.shape[1])
    if M * N < min_output_elements:
        return False, f"tiny output {M}x{N}"
    if K % 8 != 0 and m1.dtype != torch.float32:  # the fp32 split pads K
        return False, f"K={K} is not a multiple of 8"
    why = None if weight_streaming(M, N) else few_tile_verdict(M, N, effective_k(K, m1.dtype), min_tiles_long_k)
    if why is not None:
        return False, f"K={K}, " + why
    return True, "fused"


def _direct_forward(fwd: Callable, params_flat: List[torch.Tensor]) -> Callable:
    """The fused ATen graph's forward, called as AOTAutograd's inference wrapper
    calls it (lifted parameters first, autograd off during the call)."""
    if params_flat:
        def forward(*args):
            if torch.is_grad_enabled():
                with torch.no_grad():
                    return fwd(*params_flat, *args)
            return fwd(*params_flat, *args)
    else:
        def forward(*args):
            if torch.is_grad_enabled():
                with torch.no_grad():
                    return fwd(*args)
            return fwd(*args)
    return forward


class EagerGroupLauncher:
    """Callable that runs a group's original nodes (no fused kernel).

    Bound where no kernel variant fits a group, with the launcher's calling
    convention (``__name__``, positional ``*group.inputs``, the same return
    structure), so that no raising placeholder is left in the graph.
    """

    def __init__(self, module: torch.fx.GraphModule) -> None:
        self.__name__ = "fuseml_eager_group"
        self._module = module
        # The generated forward itself: nn.Module.__call__'s hook machinery
        # adds host time per call and a group module has no hooks.
        self._forward = getattr(module, "forward", module)

    def __call__(self, *args):
        return self._forward(*args)


_EagerGroup = EagerGroupLauncher


def group_eager_fn(group: Any) -> Optional[Callable[..., Any]]:
    """The group's eager closure: this repository's ``eager_module`` if the
    discovery pass set one, else one built from the reference's own fields
    (a group formed by the reference's pass has no such field).  None when it
    cannot be built."""
    mod = getattr(group, "eager_module", None)
    if mod is not None:
        return mod
    try:
        return group_eager_module(group)
    except Exception as exc:  # noqa: BLE001 - a malformed group must not abort compilation
        logger.warning("no eager closure for %s: %s: %s", group, type(exc).__name__, exc)
        return None


def epilogue_passes(spec: EpilogueSpec, gemm_is_addmm: bool = True) -> int:
    """Elementwise passes over the [M,N] result that eager PyTorch runs after
    the GEMM for this group: every epilogue op except the escape stores and,
    when the group's GEMM is an ``addmm``, its own alpha / bias terms
    (hipBLASLt applies those in its GEMM epilogue), plus one read per
    reduction.  After an ``mm`` every op is a pass of its own: ``x @ W + b``
    or a residual add runs as a separate eager kernel."""
    ops = list(spec.ops)
    i = 0
    if gemm_is_addmm:
        # the addmm's own terms come first: scale (alpha), then the bias (add
        # of a broadcast vector or scalar)
        if i < len(ops) and ops[i].kind == "scale":
            i += 1
        if i < len(ops) and ops[i].kind in ("add", "add_scalar"):
            i += 1
    passes = sum(1 for o in ops[i:] if o.kind != "store")
    return passes + len(spec.reductions)


def fused_beats_eager(spec: EpilogueSpec, K: int, k_per_pass: int = K_PER_EPILOGUE_PASS,
                      dtype: Any = None, gemm_is_addmm: bool = True,
                      k_offset: int = K_CROSSOVER_OFFSET, M: Optional[int] = None,
                      N: Optional[int] = None) -> Tuple[bool, str]:
    """The fused kernel against eager (hipBLASLt GEMM + elementwise kernels).

    Measured on one MI355X by ``python -m fuseml_amd.calibration`` (each group
    fused, eager and as a plain GEMM on the same inputs; the rows are
    profiles/cost_model_calibration.json).  Over hipBLASLt's plain GEMM, eager
    pays about one [M,N] HBM round trip per elementwise pass (0.06-0.07 ms per
    pass at 16384x4096, the same at every K), while the fused kernel pays its
    epilogue (which grows slower than the number of ops) plus a K loop that
    falls behind hipBLASLt's as K grows.  So the crossover K grows with the
    passes: one pass fuses at K = 1024 (bias + GELU 16384x4096: 0.161 against
    eager 0.172 ms) and K = 2048 (bias + residual 0.066 against 0.069 ms), ties
    at K = 4096 (8192x16384 bias + GELU: 0.854 against 0.851 ms) and loses
    beyond (bias + residual at K = 16384: 0.793 against 0.737 ms); four passes
    still win at K = 8192 (0.80 against 0.89 ms).  Rule: fuse iff
    K <= k_per_pass * passes - k_offset (3072 and 1024: K <= 2048 for one pass,
    5120 for two, 11264 for four); k_per_pass = 0 always fuses.

    fp32 groups always fuse: eager runs an fp32 GEMM at the fp32 MFMA rate
    (157 TFLOP/s peak), the split product at a third of the bf16 rate.
    Weight-streaming shapes (``M`` and ``N`` given, :func:`weight_streaming`)
    fuse while K <= WEIGHT_STREAM_K_PER_PASS x passes."""
    if k_per_pass <= 0 or dtype == torch.float32:
        return True, "fused"
    passes = epilogue_passes(spec, gemm_is_addmm)
    if M is not None and N is not None and weight_streaming(M, N):
        if K <= WEIGHT_STREAM_K_PER_PASS * passes:
            return True, "fused (decode-sized M: both paths stream the weight)"
        return False, (f"K={K} with {passes} elementwise pass(es) at decode-sized M: eager's GEMM streams "
                       f"the weight faster (fused iff K <= {WEIGHT_STREAM_K_PER_PASS} x passes)")
    limit = k_per_pass * passes - k_offset
    if K <= limit:
        return True, "fused"
    return False, (f"K={K} with {passes} elementwise pass(es): eager's GEMM is faster "
                   f"(crossover K <= {k_per_pass} x passes - {k_offset} = {limit})")


def build_hip_launcher(group: Any, eager_fn: Optional[Callable[..., Any]] = None, *,
                       spec: Optional[EpilogueSpec] = None, eager_if_unsupported: bool = True):
    """FusionGroup -> launcher: replaces compiler.py:443-585 (``_build_launcher``)
    and 591-630 (``_build_cublas_launcher``).

    Accepts this repository's :class:`FusionGroup` and the reference's
    (fuseml/fusion_group.py:74-85, any ``fusion_strategy``, with or without a
    ``cublas_pattern``): only the reference's fields are read.  Returns

    * a :class:`HipKernelLauncher` with the group's eager closure as its
      fallback, when a kernel variant expresses the group;
    * otherwise an :class:`EagerGroupLauncher` running the group's nodes
      (``eager_if_unsupported``), so the caller never keeps the raising
      placeholder;
    * ``None`` only when neither can be built, or ``eager_if_unsupported`` is
      False and no variant fits.

    Never raises for a group it cannot express (``AttributeError`` and the like
    from an unexpected group become the eager path).  A missing HIP library
    raises ``ImportError``: the product path does not fall back silently.
    """
    from .launcher import HipKernelLauncher

    if eager_fn is None:
        eager_fn = group_eager_fn(group)
    if spec is None:
        try:
            spec = spec_from_group(group)
        except UnsupportedGroup as exc:
            logger.info("group %s stays eager: %s", group, exc)
        except Exception as exc:  # noqa: BLE001
            logger.warning("group %s stays eager: %s: %s", group, type(exc).__name__, exc)
    if spec is None:
        if eager_if_unsupported and eager_fn is not None:
            return EagerGroupLauncher(eager_fn)
        return None
    return HipKernelLauncher(spec, len(group.inputs), eager_fn=eager_fn,
                             kernel_signature=f"{group!r}: {spec.describe()}")


class FuseMLCompiler:
    """``torch.compile`` backend fusing addmm/mm epilogue chains into HIP kernels."""

    def __init__(self, registry: Any = None, *, fuse_sibling_reductions: bool = False,
                 fuse_leading_views: bool = False, fuse_mlp_block: Union[bool, str] = "auto",
                 min_output_elements: int = MIN_FUSION_OUTPUT_ELEMENTS,
                 min_tiles_long_k: int = MIN_TILES_LONG_K,
                 k_per_epilogue_pass: int = K_PER_EPILOGUE_PASS,
                 require_gfx950: bool = True, direct_dispatch: bool = True, hip_graph: bool = False) -> None:
        self.registry = registry
        # Replay each directly dispatched, static-shape forward from a HIP graph
        # (fuseml_amd.graphs.HipGraphForward: the returned tensors are static
        # outputs, overwritten by the next call, as with CUDA graphs under
        # torch.compile(mode="reduce-overhead")).  Off by default.
        self.hip_graph = hip_graph
        self.graph_forwards: List[Any] = []
        # Return the fused graph's forward to Dynamo without AOTAutograd's
        # runtime wrapper when that wrapper would only call it
        # (aot_wrapper_is_identity); `dispatch` records which path each
        # compiled graph got ("direct" or "aot: <reason>").
        self.direct_dispatch = direct_dispatch
        self.dispatch: List[str] = []
        self.fuse_sibling_reductions = fuse_sibling_reductions
        self.fuse_leading_views = fuse_leading_views
        if fuse_mlp_block not in (True, False, "auto"):
            raise ValueError(f"fuse_mlp_block must be True, False or 'auto', not {fuse_mlp_block!r}")
        self.fuse_mlp_block = fuse_mlp_block
        self.min_output_elements = min_output_elements
        self.min_tiles_long_k = min_tiles_long_k
        self.k_per_epilogue_pass = k_per_epilogue_pass
        self.require_gfx950 = require_gfx950
        self.fusion_candidates: List[torch.fx.Node] = []
        self.fusion_applied: bool = False
        self.fusion_strategy: str = "none"
        self.launchers: List[Any] = []
        self._cache = LauncherCache()

    # ------------------------------------------------------------------
    def __call__(self, gm: torch.fx.GraphModule, example_inputs: List[torch.Tensor]) -> Callable:
        captured: Dict[str, Any] = {}

        def _aten_compiler(aten_gm: torch.fx.GraphModule, aten_inputs: List[torch.Tensor]):
            from torch._guards import TracingContext

            fwd = self._compile_aten_graph(aten_gm, aten_inputs)
            ctx = TracingContext.try_get()
            captured.update(fwd=fwd, n_graph_inputs=len(aten_inputs),
                            meta=getattr(ctx, "fw_metadata", None) if ctx is not None else None)
            return make_boxed_func(fwd)

        # What AOTAutograd prepends to every call: the Dynamo graph's own
        # parameters and buffers (aot_module_simplified lifts them).
        params_flat = [t for _, t in gm.named_parameters(remove_duplicate=False)] + \
                      [t for _, t in gm.named_buffers(remove_duplicate=False)]
        amp = torch._C._is_any_autocast_enabled()
        try:
            compiled = aot_module_simplified(gm, example_inputs, fw_compiler=_aten_compiler)
        except _NoFusionPossible as exc:
            self.fusion_applied = False
            self.fusion_strategy = "none"
            logger.info("bypassing AOT lowering — %s", exc)
            return gm.forward
        if not self.direct_dispatch or "fwd" not in captured:
            self.dispatch.append("aot: direct dispatch off")
            return compiled
        ok, why = aot_wrapper_is_identity(captured["meta"], captured["n_graph_inputs"],
                                          len(params_flat) + len(example_inputs))
        if ok and amp:
            ok, why = False, "traced under autocast"
        if not ok:
            self.dispatch.append(f"aot: {why}")
            return compiled
        forward = _direct_forward(captured["fwd"], params_flat)
        if not self.hip_graph:
            self.dispatch.append("direct")
            return forward
        from .graphs import HipGraphForward, static_shapes

        if not static_shapes(params_flat + list(example_inputs)):
            self.dispatch.append("direct (no HIP graph: dynamic shapes or inputs off one GPU)")
            return forward
        # The graph's parameter and buffer inputs (AOTAutograd's
        # static_input_indices, over the lifted parameters and then the call's
        # arguments) are read in place; the other arguments are copied.
        n_p = len(params_flat)
        static = {i - n_p for i in getattr(captured["meta"], "static_input_indices", []) if i >= n_p}
        graph_forward = HipGraphForward(forward, static, params=params_flat)
        self.graph_forwards.append(graph_forward)
        self.dispatch.append("direct+hip_graph")
        return graph_forward

    # ------------------------------------------------------------------
    def _device_ok(self, inputs: List[Any]) -> bool:
        if not self.require_gfx950:
            return True
        devs = {t.device for t in inputs if isinstance(t, torch.Tensor)}
        cuda = [d for d in devs if d.type == "cuda"]
        return bool(cuda) and all(device_is_gfx950(d) for d in cuda)

    def _compile_aten_graph(self, gm: torch.fx.GraphModule, example_inputs: List[Any]) -> Callable:
        self.fusion_candidates = []
        if not self._device_ok(example_inputs):
            raise _NoFusionPossible("inputs are not on a gfx950 GPU")
        has_trigger = False
        fusible = False
        for node in gm.graph.nodes:
            if node.op == "call_function" and node.target in TRIGGER_TARGETS:
                has_trigger = True
                ok, why = trigger_is_fusible(node, self.min_output_elements, self.min_tiles_long_k)
                node.meta["fuseml_cost_model"] = why
                if ok:
                    fusible = True
                    self.fusion_candidates.append(node)
        if not has_trigger:
            raise _NoFusionPossible("no addmm/mm trigger in graph")
        if not fusible:
            raise _NoFusionPossible("every trigger is below the fusion threshold or unsupported")

        fpass = FuseMLFusionPass(gm, self.registry, fuse_sibling_reductions=self.fuse_sibling_reductions,
                                 fuse_leading_views=self.fuse_leading_views)
        gm = fpass.run(example_inputs)
        placeholders = [n for n in gm.graph.nodes
                        if n.op == "call_function" and n.target is fuseml_fused_kernel_placeholder]
        if not placeholders:
            raise _NoFusionPossible("fusion pass found no fusible sequence")

        strategies = set()
        if self.fuse_mlp_block:
            placeholders = self._bind_mlp_blocks(gm, placeholders, strategies)
        for ph in placeholders:
            group: FusionGroup = ph.meta["fusion_group"]
            # the pre-scan's verdict (the base node's args are gone after surgery)
            ok = group.base_node.meta.get("fuseml_cost_model") == "fused"
            launcher = None
            if ok:
                try:
                    spec = spec_from_group(group)
                except UnsupportedGroup as exc:
                    logger.info("group %s stays eager: %s", group, exc)
                    spec = None
                if spec is not None:
                    K, ab_dtype, gM, gN = _gemm_dims(group)
                    addmm = group.base_node.target is TRIGGER_TARGETS[0]
                    win, why = (fused_beats_eager(spec, K, self.k_per_epilogue_pass, ab_dtype, addmm, M=gM, N=gN)
                                if K else (True, "fused"))
                    if not win:
                        logger.info("group %s stays eager: %s", group, why)
                        spec = None
                key = launcher_cache_key(group, spec) if spec is not None else None
                launcher = self._cache.lookup(key) if key is not None else None
                if launcher is None and spec is not None:
                    launcher = build_hip_launcher(group)
                    if isinstance(launcher, EagerGroupLauncher):
                        launcher = None
                    if launcher is not None and key is not None:
                        self._cache.store(key, launcher)
            if launcher is None:
                target: Callable = EagerGroupLauncher(group.eager_module)
                strategies.add("eager")
            else:
                target = launcher
                strategies.add("hip")
                self.launchers.append(launcher)
            with gm.graph.inserting_after(ph):
                new = gm.graph.call_function(target, args=ph.args)
            new.meta.update({k: v for k, v in ph.meta.items() if k != "fusion_group"})
            ph.replace_all_uses_with(new)
            gm.graph.erase_node(ph)

        gm.graph.eliminate_dead_code()
        gm.recompile()
        self.fusion_applied = "hip" in strategies
        self.fusion_strategy = "hip" if strategies == {"hip"} else ("mixed" if self.fusion_applied else "eager")
        return gm.forward

    def _bind_mlp_blocks(self, gm: torch.fx.GraphModule, placeholders: List[torch.fx.Node],
                         strategies: set) -> List[torch.fx.Node]:
        """Bind each (GEMM1+bias+GELU[+scalar ops], GEMM2+bias+residual) placeholder pair whose
        GELU output feeds only the second GEMM to one single-kernel MLP launcher
        (``fuse_mlp_block=True``, or ``"auto"`` where the single kernel measured
        faster); return the placeholders left to bind."""
        from .mlp import (HipMlpLauncher, mlp_block_beats_two_launches, mlp_eager_fn, mlp_first_group,
                          mlp_second_group, mlp_shape_supported)

        specs: Dict[torch.fx.Node, Any] = {}
        for ph in placeholders:
            try:
                specs[ph] = spec_from_group(ph.meta["fusion_group"])
            except UnsupportedGroup:
                specs[ph] = None
        used: set = set()
        for ph2 in placeholders:
            sp2 = specs.get(ph2)
            m2 = mlp_second_group(sp2) if sp2 is not None else None
            if m2 is None:
                continue
            ph1 = ph2.args[m2["h"]]
            if not isinstance(ph1, torch.fx.Node) or ph1 not in specs or ph1 in used or specs[ph1] is None:
                continue
            m1 = mlp_first_group(specs[ph1])
            if m1 is None or list(ph1.users) != [ph2]:
                continue
            g1, g2 = ph1.meta["fusion_group"], ph2.meta["fusion_group"]
            if self.fuse_mlp_block is True:
                # forced: both GEMMs must still pass the pre-scan's cost model
                # (tiny outputs and few-tile long-K GEMMs stay eager whichever
                # kernel would run them); "auto" applies its measured rule below,
                # which compares the single kernel with the default path
                verdicts = [g.base_node.meta.get("fuseml_cost_model") for g in (g1, g2)]
                if verdicts != ["fused", "fused"]:
                    logger.info("MLP pair %s + %s stays unbound: %s", g1, g2, verdicts)
                    continue
            n1, n2 = len(g1.inputs), len(g2.inputs)
            slots1 = {k: m1[k] for k in ("x", "w1t", "b1")}
            slots2 = {k: m2[k] for k in ("h", "w2t", "b2", "r")}
            if sorted(slots1.values()) != list(range(n1)) or sorted(slots2.values()) != list(range(n2)):
                continue
            xm, wm, dt = _meta(ph1.args[m1["x"]]), _meta(ph1.args[m1["w1t"]]), specs[ph1].out_dtype
            if xm is None or wm is None or len(xm.shape) != 2 or len(wm.shape) != 2:
                continue
            M, D, I = int(xm.shape[0]), int(xm.shape[1]), int(wm.shape[1])
            ok, why = mlp_shape_supported(M, D, I, dt)
            if ok and self.fuse_mlp_block == "auto":
                ok, why = mlp_block_beats_two_launches(M, D, I)
            if not ok:
                logger.info("MLP pair %s + %s keeps two launches: %s", g1, g2, why)
                continue
            eager = mlp_eager_fn(EagerGroupLauncher(g1.eager_module), EagerGroupLauncher(g2.eager_module),
                                 n1, n2, slots1, slots2)
            launcher = HipMlpLauncher(m1["approximate"], eager_fn=eager, post=m1["post"],
                                      kernel_signature=f"{g1!r} + {g2!r}: mlp_block")
            args = (ph1.args[m1["x"]], ph1.args[m1["w1t"]], ph1.args[m1["b1"]],
                    ph2.args[m2["w2t"]], ph2.args[m2["b2"]], ph2.args[m2["r"]])
            with gm.graph.inserting_after(ph2):
                new = gm.graph.call_function(launcher, args=args)
            new.meta.update({k: v for k, v in ph2.meta.items() if k != "fusion_group"})
            ph2.replace_all_uses_with(new)
            gm.graph.erase_node(ph2)
            gm.graph.erase_node(ph1)
            used.update((ph1, ph2))
            self.launchers.append(launcher)
            strategies.add("hip")
        return [ph for ph in placeholders if ph not in used]

    @property
    def cache(self) -> LauncherCache:
        return self._cache
