"""Runtime dispatch of one fused group through the C ABI.

:class:`HipKernelLauncher` keeps the calling convention of the reference's
``KernelLauncher`` (fuseml/codegen/kernel_launcher.py:309-821): it is called
with the group's external tensors positionally, in ``FusionGroup.inputs``
order, has a ``__name__`` for FX node naming (kernel_launcher.py:425-426),
checks arity with ``ValueError`` (685-689), copies negative-stride inputs
(694-703), reads M,K from the left operand and N from the right (709-711),
allocates fresh row-major outputs (723-746), launches on
``torch.cuda.current_stream()`` (622-633) with no host synchronisation, and
returns the primary output — or a tuple ``(primary, *intermediates)`` when the
group has escape outputs, which is what the surgery's ``getitem`` nodes expect
(fuseml/passes/fusion_pass.py:824-880; the reference returns only the primary,
kernel_launcher.py:821).

Instead of ``kernel_fn[grid](ptrs..., M, N, K, strides...)`` it fills a
``fuseml_gemm_desc`` and calls ``fuseml_gemm_epilogue``.  Reductions are
accumulated in fp32 buffers that the library initialises on the stream, then
cast to the reduction's dtype (the reference's fp32-mean path,
kernel_launcher.py:496-509, 816-821, extended to sum and amax).
"""

from __future__ import annotations

import ctypes
from typing import Any, Callable, Dict, List, Optional, Sequence, Tuple

import torch

from . import _abi
from .epilogue import EpilogueSpec
from .fallback import EagerFallbackGuard

_DTYPE_CODE = {torch.bfloat16: _abi.BF16, torch.float16: _abi.F16, torch.float32: _abi.F32}


def _dtype_code(dt: torch.dtype) -> int:
    try:
        return _DTYPE_CODE[dt]
    except KeyError:
        raise _abi.FuseMLHipError(_abi.EUNSUPPORTED, f"dtype {dt} not supported") from None


def _has_negative_stride(t: torch.Tensor) -> bool:
    return any(s < 0 for s in t.stride())


def _k_major_left(a: torch.Tensor) -> torch.Tensor:
    """A[M,K] with unit K stride, 8-element aligned rows, 16-byte aligned base."""
    if a.stride(1) == 1 and a.stride(0) % 8 == 0 and a.data_ptr() % 16 == 0 and (
        a.stride(0) >= a.shape[1] or a.shape[0] == 1
    ):
        return a
    return a.contiguous()


def _k_major_right(b: torch.Tensor) -> torch.Tensor:
    """B[K,N] with unit K stride (the t(W) view), 8-element aligned columns."""
    if b.stride(0) == 1 and b.stride(1) % 8 == 0 and b.data_ptr() % 16 == 0 and (
        b.stride(1) >= b.shape[0] or b.shape[1] == 1
    ):
        return b
    return b.t().contiguous().t()


def _distinct_bytes(tensors: Sequence[torch.Tensor]) -> int:
    """Bytes of each distinct tensor (by storage span) counted once: what a launch
    must move at least (inputs read once, outputs written once)."""
    seen, total = set(), 0
    for t in tensors:
        if isinstance(t, torch.Tensor):
            key = (t.data_ptr(), t.numel())
            if key not in seen:
                seen.add(key)
                total += t.numel() * t.element_size()
    return total


class HipKernelLauncher:
    """Callable that runs one fused group on the gfx950 kernel family."""

    def __init__(
        self,
        spec: EpilogueSpec,
        n_inputs: int,
        eager_fn: Optional[Callable[..., Any]] = None,
        kernel_signature: str = "",
    ) -> None:
        self.__name__ = "fuseml_fused_kernel"
        self.spec = spec
        self._n_inputs = n_inputs
        self._lib = _abi.load_library()
        self._descs: Dict[tuple, _abi.GemmDesc] = {}
        self._fallback_guard: Optional[EagerFallbackGuard] = None
        if eager_fn is not None:
            self._fallback_guard = EagerFallbackGuard(
                eager_fn=eager_fn, kernel_signature=kernel_signature or spec.describe()
            )
        self.launch_count = 0
        # Measurement hook: a list to receive, per launch, (start event, end
        # event, (M, N, K), algorithmic bytes) recorded on the launch stream
        # around the C call.  None (the default) records nothing.
        self.timing_events: Optional[List[Tuple[Any, Any, Tuple[int, int, int], int]]] = None

    # ------------------------------------------------------------------
    @property
    def fallback_count(self) -> int:
        return self._fallback_guard.fallback_count if self._fallback_guard else 0

    def __repr__(self) -> str:
        return f"HipKernelLauncher({self.spec.describe()})"

    # ------------------------------------------------------------------
    def _operand_tensors(self, inputs: Sequence[torch.Tensor], M: int, N: int) -> List[torch.Tensor]:
        """Broadcast every add/mul operand to a zero-stride [M,N] view.

        An operand of an op on an N-D value ([*lead, N], same memory order as
        [M,N]) is broadcast to that shape first and its leading dimensions
        merged; when their strides do not merge (e.g. [B,1,N] against
        [B,S,N]) the merge materialises the broadcast (a copy, still exact).
        """
        shapes = dict(self.spec.operand_shapes)
        seen: Dict[int, int] = {}
        ops: List[torch.Tensor] = []
        for op in self.spec.ops:
            if op.kind in ("add", "mul") and op.operand not in seen:
                t = inputs[op.operand]
                if t.dtype not in _DTYPE_CODE:
                    t = t.to(torch.float32)
                shape = shapes.get(op.operand)
                if shape is not None:
                    t = t.expand(shape).reshape(M, N)
                elif t.dim() > 2:
                    raise _abi.FuseMLHipError(_abi.EUNSUPPORTED, "operand rank > 2")
                else:
                    t = t.expand(M, N)
                seen[op.operand] = len(ops)
                ops.append(t)
        self._operand_slot = seen
        return ops

    def _desc(self, key: tuple) -> _abi.GemmDesc:
        d = self._descs.get(key)
        if d is None:
            d = _abi.GemmDesc()
            self._descs[key] = d
        return d

    def launch(self, *inputs: torch.Tensor) -> Any:
        """Allocate outputs, fill the descriptor and call the C ABI."""
        spec = self.spec
        a = _k_major_left(inputs[spec.left])
        b = _k_major_right(inputs[spec.right])
        if a.dtype != b.dtype or a.dtype not in (torch.bfloat16, torch.float16):
            raise _abi.FuseMLHipError(
                _abi.EUNSUPPORTED, f"GEMM operands {a.dtype}/{b.dtype}: bf16/f16 MFMA only"
            )
        M, K = int(a.shape[0]), int(a.shape[1])
        N = int(b.shape[1])
        dev = a.device
        operands = self._operand_tensors(inputs, M, N)

        tile = None
        if spec.store_tile:
            tile = torch.empty_strided((M, N), (N, 1), dtype=spec.out_dtype, device=dev)
        extras = [torch.empty_strided((M, N), (N, 1), dtype=dt, device=dev) for dt in spec.extra_dtypes]
        red_len = M if spec.reduce_axis == 1 else N
        reds = {name: torch.empty((red_len,), dtype=torch.float32, device=dev) for name in spec.reductions}

        if M == 0 or N == 0:
            # No launch.  A reduction over an empty axis follows torch: sum 0,
            # mean NaN, amax raises (IndexError, as torch.amax does).
            reduced_len = N if spec.reduce_axis == 1 else M
            if red_len > 0 and reduced_len == 0:
                if "amax" in reds:
                    raise IndexError("amax(): Expected reduction dim to have non-zero size.")
                for name, t in reds.items():
                    t.fill_(0.0 if name == "sum" else float("nan"))
            return self._assemble(tile, extras, reds)

        key = (M, N, K, a.stride(0), b.stride(1), tuple((o.stride(), o.dtype) for o in operands))
        d = self._desc(key)
        d.M, d.N, d.K = M, N, K
        d.a, d.lda = a.data_ptr(), a.stride(0)
        d.b, d.ldb = b.data_ptr(), b.stride(1)
        d.ab_dtype = _dtype_code(a.dtype)
        d.n_ops = len(spec.ops)
        if d.n_ops > _abi.MAX_OPS:
            raise _abi.FuseMLHipError(_abi.EUNSUPPORTED, "too many epilogue ops")
        for i, op in enumerate(spec.ops):
            e = d.ops[i]
            e.kind = _abi.OP_CODES[op.kind]
            if op.kind in ("add", "mul"):
                e.operand = self._operand_slot[op.operand]
            else:
                e.operand = op.operand
            e.scalar = op.scalar
        d.n_operands = len(operands)
        if d.n_operands > _abi.MAX_OPERANDS:
            raise _abi.FuseMLHipError(_abi.EUNSUPPORTED, "too many epilogue operands")
        for i, t in enumerate(operands):
            o = d.operands[i]
            sm, sn = t.stride()
            o.ptr = t.data_ptr()
            o.stride_m, o.stride_n = sm, sn
            o.extent = (M - 1) * sm + (N - 1) * sn + 1
            o.dtype = _DTYPE_CODE[t.dtype]
        if tile is not None:
            d.out.ptr, d.out.ld, d.out.dtype = tile.data_ptr(), N, _dtype_code(tile.dtype)
        else:
            d.out.ptr, d.out.ld, d.out.dtype = None, N, _abi.BF16
        d.n_extra = len(extras)
        for i, t in enumerate(extras):
            d.extra[i].ptr, d.extra[i].ld, d.extra[i].dtype = t.data_ptr(), N, _dtype_code(t.dtype)
        mask = 0
        for name, t in reds.items():
            mask |= _abi.RED_BITS[name]
            d.reduce_out[_abi.RED_SLOT[name]] = t.data_ptr()
        d.reduce_mask = mask
        d.reduce_axis = spec.reduce_axis

        stream = torch.cuda.current_stream(dev).cuda_stream if dev.type == "cuda" else 0
        timing = self.timing_events
        if timing is not None:
            ev0, ev1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
            ev0.record()
        rc = self._lib.fuseml_gemm_epilogue(ctypes.byref(d), ctypes.c_void_p(stream))
        if rc != _abi.OK:
            raise _abi.FuseMLHipError(rc, _abi.last_error(self._lib))
        if timing is not None:
            ev1.record()
            outs = [t for t in [tile, *extras, *reds.values()] if t is not None]
            timing.append((ev0, ev1, (M, N, K), _distinct_bytes([*inputs, *outs])))
        self.launch_count += 1
        return self._assemble(tile, extras, reds)

    def _assemble(self, tile, extras, reds) -> Any:
        outs = []
        red_dt = dict(zip(self.spec.reductions, self.spec.reduce_dtypes))
        for o in self.spec.outputs:
            if o[0] == "tile":
                outs.append(tile)
            elif o[0] == "red":
                r = reds[o[1]]
                dt = red_dt.get(o[1], torch.float32)
                outs.append(r if dt == torch.float32 else r.to(dt))
            else:
                outs.append(extras[o[1]])
        if self.spec.output_shapes:
            outs = [t if sh is None else t.view(sh) for t, sh in zip(outs, self.spec.output_shapes)]
        return outs[0] if len(outs) == 1 else tuple(outs)

    # ------------------------------------------------------------------
    def __call__(self, *inputs: torch.Tensor) -> Any:
        if len(inputs) != self._n_inputs:
            raise ValueError(f"Expected {self._n_inputs} input tensor(s), got {len(inputs)}.")
        if any(_has_negative_stride(t) for t in inputs if isinstance(t, torch.Tensor)):
            inputs = tuple(
                t.contiguous() if isinstance(t, torch.Tensor) and _has_negative_stride(t) else t
                for t in inputs
            )
        if self._fallback_guard is not None:
            return self._fallback_guard.execute(lambda: self.launch(*inputs), inputs)
        return self.launch(*inputs)
