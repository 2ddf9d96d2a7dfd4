"""The single-kernel MLP block: two fusion groups in one launch.

The reference forms two groups for ``linear2(gelu(linear1(x))) + x`` — an
addmm ends a group (fuseml/passes/topology.py:63-64) and absorption needs a
single user (fuseml/passes/fusion_pass.py:203-206) — so the GELU output ``h``
is written to HBM by the first launch and read back by the second.  With
``FuseMLCompiler(fuse_mlp_block=True)`` a pair of groups

    G1: addmm(b1, x, t(W1)) -> gelu [-> scale / add_scalar ...]   (h has one user: G2)
    G2: addmm(b2, h, t(W2)) -> add(., r)

is bound to one :class:`HipMlpLauncher`, which calls ``fuseml_mlp_block``:
``h`` stays in LDS chunk by chunk and never reaches HBM.  Up to
``_abi.MLP_MAX_POST`` scalar ops after the GELU (the reference's
activation-heavy block, ``gelu(.) * 0.5 + 0.125``, bench_mlp_block.py:185-207)
run in the kernel too, in order, in fp32.  The kernel holds a
64 x D fp32 accumulator per row block in registers, so it takes D (the model
width) of 256, 512 or 1024 only; other pairs keep their two launches.  The
default ``fuse_mlp_block="auto"`` binds a pair only where the single kernel
measured faster than the two launches (:func:`mlp_block_beats_two_launches`).

The launcher's calling convention is the fused launchers' (``__name__``,
positional inputs, ``ValueError`` on arity, fresh row-major output, launch on
the current stream with no host synchronisation) with the inputs
``(x, t(W1), b1, t(W2), b2, r)``; its eager fallback runs the two groups'
original nodes.
"""

from __future__ import annotations

import ctypes
from typing import Any, Callable, Dict, Optional, Tuple

import torch

from . import _abi
from .epilogue import EpilogueSpec
from .fallback import EagerFallbackGuard

MLP_WIDTHS = (256, 512, 1024)
MLP_CHUNK = 32
# The measured crossover (``python -m fuseml_amd.calibration --mlp``, rows in
# profiles/mlp_block_crossover.json): the single kernel streams every weight
# through each CU once per 64-row block, so it wins only where the row blocks
# fill the chip (at least one per CU) and the weights are small (D = 256):
# 0.84-0.92x of the two launches' time at M >= 16384 on 256 CUs (0.98x at
# M = 65536, I = 1024), 1.04-1.74x below that; D = 512 loses (1.06-1.41x) and
# D = 1024 too (2.24x).
MLP_AUTO_WIDTH = 256
MLP_AUTO_MIN_ROW_BLOCKS = 256

_DTYPES = {torch.bfloat16: _abi.BF16, torch.float16: _abi.F16}
_POST_KINDS = {"scale": _abi.OP_SCALE, "add_scalar": _abi.OP_ADD_SCALAR}


def mlp_shape_supported(M: int, D: int, I: int, dtype: torch.dtype) -> Tuple[bool, str]:
    """Host-side restatement of the kernel's shape limits (for the cost model)."""
    if dtype not in _DTYPES:
        return False, f"dtype {dtype}: bf16/f16 only"
    if D not in MLP_WIDTHS:
        return False, f"D={D}: the 64 x D accumulator fits registers for D in {MLP_WIDTHS} only"
    if I % MLP_CHUNK != 0:
        return False, f"I={I} is not a multiple of {MLP_CHUNK}"
    if M <= 0:
        return False, "empty batch"
    return True, "fused"


def mlp_block_beats_two_launches(M: int, D: int, I: int) -> Tuple[bool, str]:
    """The cost model's rule for ``fuse_mlp_block="auto"``: the single kernel
    (with packed weights) for D = 256, I a multiple of 128 and at least
    MLP_AUTO_MIN_ROW_BLOCKS 64-row blocks; otherwise the two launches."""
    if D != MLP_AUTO_WIDTH:
        return False, f"D={D}: the single kernel measured slower than two launches (D = {MLP_AUTO_WIDTH} only)"
    if I % 128 != 0:
        return False, f"I={I} is not a multiple of 128 (the weight-streaming kernel's slice)"
    if -(-M // 64) < MLP_AUTO_MIN_ROW_BLOCKS:
        return False, f"M={M}: fewer than {MLP_AUTO_MIN_ROW_BLOCKS} 64-row blocks"
    return True, "single kernel"


_WORD = 8
_MW = {f: getattr(_abi.MlpDesc, f).offset // _WORD for f in ("x", "w1", "b1", "w2", "b2", "r", "y", "wpack")}


class _MlpPlan:
    """What a call needs that depends only on its input signature: the
    descriptor with every non-pointer field filled (written through ``words``,
    the descriptor as uint64 words) and the packed-weight size (0: none)."""

    __slots__ = ("desc", "words", "desc_ref", "M", "D", "dtype", "pack_bytes")

    def __init__(self, desc: "_abi.MlpDesc", M: int, D: int, dtype: torch.dtype, pack_bytes: int) -> None:
        self.desc = desc
        self.words = (ctypes.c_uint64 * (ctypes.sizeof(_abi.MlpDesc) // _WORD)).from_buffer(desc)
        self.desc_ref = ctypes.byref(desc)
        self.M, self.D, self.dtype, self.pack_bytes = M, D, dtype, pack_bytes


class HipMlpLauncher:
    """Callable ``(x, t(W1), b1, t(W2), b2, r) -> y`` on ``fuseml_mlp_block``."""

    N_INPUTS = 6

    def __init__(self, approximate: str = "none", eager_fn: Optional[Callable[..., Any]] = None,
                 kernel_signature: str = "mlp_block", pack_weights: bool = True,
                 post: Tuple[Tuple[str, float], ...] = ()) -> None:
        self.__name__ = "fuseml_mlp_block"
        self.approximate = approximate
        # Scalar ops on the GELU's output, in order: ("scale", s) or ("add_scalar", s).
        if len(post) > _abi.MLP_MAX_POST or any(k not in _POST_KINDS for k, _ in post):
            raise ValueError(f"post ops: at most {_abi.MLP_MAX_POST} of {sorted(_POST_KINDS)}, got {post!r}")
        self.post = tuple((k, float(v)) for k, v in post)
        # Where the kernel streams weight fragments (D of 256 or 512, I a
        # multiple of 128), W1 and W2 are repacked once into fragment order
        # (fuseml_mlp_pack_weights: 4*D*I extra bytes, held here) and packed
        # again when either weight changes (pointer, stride or in-place version).
        self.pack_weights = pack_weights
        self._pack: Optional[torch.Tensor] = None
        self._pack_key: Optional[tuple] = None
        # Per input signature (shapes, strides, dtypes, device): a plan whose
        # calls only write pointers (see launch).
        self._plans: Dict[tuple, _MlpPlan] = {}
        self._gelu = _abi.OP_GELU_TANH if approximate == "tanh" else _abi.OP_GELU_ERF
        self._lib = _abi.load_library()
        self._desc = _abi.MlpDesc()
        self._guard = EagerFallbackGuard(eager_fn, kernel_signature) if eager_fn is not None else None
        self.launch_count = 0

    @property
    def fallback_count(self) -> int:
        return self._guard.fallback_count if self._guard else 0

    def __repr__(self) -> str:
        post = "".join(f", {k}={v:g}" for k, v in self.post)
        return f"HipMlpLauncher(gelu={self.approximate}{post})"

    def launch(self, x: torch.Tensor, w1t: torch.Tensor, b1: torch.Tensor, w2t: torch.Tensor,
               b2: Optional[torch.Tensor], r: Optional[torch.Tensor]) -> torch.Tensor:
        """A call whose signature was seen before writes only the pointers into
        that signature's descriptor; the first call of a signature checks and
        fills it (and calls with layouts that need copies always take that path)."""
        if isinstance(self._lib, ctypes.CDLL):
            key = (x.shape, x.stride(), x.dtype, x.device, w1t.shape, w1t.stride(), w1t.dtype, w1t.get_device(),
                   b1.shape, b1.stride(), b1.dtype, b1.get_device(), w2t.stride(), w2t.dtype, w2t.get_device(),
                   None if b2 is None else (b2.shape, b2.stride(), b2.dtype, b2.get_device()),
                   None if r is None else (r.shape, r.stride(), r.dtype, r.get_device()))
            plan = self._plans.get(key)
            if plan is not None:
                return self._launch_planned(plan, key, x, w1t, b1, w2t, b2, r)
            y = self._launch_checked(x, w1t, b1, w2t, b2, r)
            if self._plan_ok:
                d = _abi.MlpDesc()
                ctypes.memmove(ctypes.byref(d), ctypes.byref(self._desc), ctypes.sizeof(d))
                self._plans[key] = _MlpPlan(d, int(x.shape[0]), int(x.shape[1]), x.dtype, self._plan_pack_bytes)
            return y
        return self._launch_checked(x, w1t, b1, w2t, b2, r)

    def _launch_planned(self, plan: "_MlpPlan", key: tuple, x: torch.Tensor, w1t: torch.Tensor,
                        b1: torch.Tensor, w2t: torch.Tensor, b2: Optional[torch.Tensor],
                        r: Optional[torch.Tensor]) -> torch.Tensor:
        w = plan.words
        w[_MW["x"]] = x.data_ptr()
        w[_MW["w1"]] = w1t.data_ptr()
        w[_MW["b1"]] = b1.data_ptr()
        w[_MW["w2"]] = w2t.data_ptr()
        w[_MW["b2"]] = 0 if b2 is None else b2.data_ptr()
        w[_MW["r"]] = 0 if r is None else r.data_ptr()
        y = torch.empty((plan.M, plan.D), dtype=plan.dtype, device=x.device)
        w[_MW["y"]] = y.data_ptr()
        stream = torch._C._cuda_getCurrentRawStream(x.get_device())
        w[_MW["wpack"]] = self._packed(plan.desc_ref, plan.pack_bytes, x, w1t, w2t, stream) if plan.pack_bytes else 0
        rc = self._lib.fuseml_mlp_block(plan.desc_ref, ctypes.c_void_p(stream))
        if rc != _abi.OK:
            raise _abi.FuseMLHipError(rc, _abi.last_error(self._lib))
        self.launch_count += 1
        return y

    def _packed(self, desc_ref: Any, nbytes: int, x: torch.Tensor, w1t: torch.Tensor, w2t: torch.Tensor,
                stream: int) -> int:
        """The packed weights' address (packed again when W1 or W2 changed)."""
        key = (x.device, nbytes, w1t.data_ptr(), w1t.stride(1), w1t._version, w2t.data_ptr(), w2t.stride(1),
               w2t._version)
        if key != self._pack_key:
            buf = torch.empty(nbytes, dtype=torch.uint8, device=x.device)
            rc = self._lib.fuseml_mlp_pack_weights(desc_ref, ctypes.c_void_p(buf.data_ptr()), ctypes.c_void_p(stream))
            if rc != _abi.OK:
                raise _abi.FuseMLHipError(rc, _abi.last_error(self._lib))
            self._pack, self._pack_key = buf, key
        return self._pack.data_ptr()

    def _launch_checked(self, x: torch.Tensor, w1t: torch.Tensor, b1: torch.Tensor, w2t: torch.Tensor,
                        b2: Optional[torch.Tensor], r: Optional[torch.Tensor]) -> torch.Tensor:
        # whether this call's descriptor may serve later calls of its signature
        # (operands used in place, not copied), and its packed-weight size
        self._plan_ok = False
        self._plan_pack_bytes = 0
        if x.dim() != 2 or w1t.dim() != 2 or w2t.dim() != 2:
            raise _abi.FuseMLHipError(_abi.EUNSUPPORTED, "mlp_block takes 2-D x and weights")
        M, D = x.shape
        I = w1t.shape[1]
        dt = x.dtype
        if dt not in _DTYPES or any(t is not None and t.dtype != dt for t in (w1t, b1, w2t, b2, r)):
            raise _abi.FuseMLHipError(_abi.EUNSUPPORTED, "mlp_block: every tensor must share one bf16/f16 dtype")
        tensors = [t for t in (x, w1t, b1, w2t, b2, r) if t is not None]
        if isinstance(self._lib, ctypes.CDLL) and (x.device.type != "cuda" or
                                                   any(t.device != x.device for t in tensors)):
            # a host pointer (or another device's) would fault in the kernel
            raise _abi.FuseMLHipError(_abi.EINVAL, "mlp_block: every tensor must be on the launch's GPU")
        if tuple(w1t.shape) != (D, I) or tuple(w2t.shape) != (I, D) or b1.shape != (I,) or \
                (b2 is not None and b2.shape != (D,)) or (r is not None and tuple(r.shape) != (M, D)):
            raise _abi.FuseMLHipError(_abi.EUNSUPPORTED, "mlp_block: operand shapes do not chain")
        # K-contiguous operands (the graph's layouts: x row-major, t(W) views).
        in_place = (x.stride(1) == 1 and w1t.stride(0) == 1 and w2t.stride(0) == 1 and b1.is_contiguous()
                    and (b2 is None or b2.is_contiguous()) and (r is None or r.stride(1) == 1))
        if x.stride(1) != 1:
            x = x.contiguous()
        if w1t.stride(0) != 1:
            w1t = w1t.t().contiguous().t()
        if w2t.stride(0) != 1:
            w2t = w2t.t().contiguous().t()
        b1 = b1.contiguous()
        if b2 is not None:
            b2 = b2.contiguous()
        if r is not None and r.stride(1) != 1:
            r = r.contiguous()
        y = torch.empty((M, D), dtype=dt, device=x.device)
        if M == 0:
            return y
        d = self._desc
        d.M, d.D, d.I = M, D, I
        d.x, d.ldx = x.data_ptr(), x.stride(0)
        d.w1, d.ldw1 = w1t.data_ptr(), w1t.stride(1)
        d.b1 = b1.data_ptr()
        d.w2, d.ldw2 = w2t.data_ptr(), w2t.stride(1)
        d.b2 = b2.data_ptr() if b2 is not None else None
        d.r, d.ldr = (r.data_ptr(), r.stride(0)) if r is not None else (None, D)
        d.y, d.ldy = y.data_ptr(), D
        d.dtype = _DTYPES[dt]
        d.gelu = self._gelu
        d.n_post = len(self.post)
        for i, (k, v) in enumerate(self.post):
            d.post_kind[i], d.post_scalar[i] = _POST_KINDS[k], v
        d.wpack = None
        stream = torch.cuda.current_stream(x.device).cuda_stream if x.device.type == "cuda" else 0
        nbytes = 0
        if self.pack_weights and isinstance(self._lib, ctypes.CDLL):
            nbytes = self._lib.fuseml_mlp_pack_bytes(ctypes.byref(d))
            if nbytes > 0:
                d.wpack = self._packed(ctypes.byref(d), nbytes, x, w1t, w2t, stream)
        rc = self._lib.fuseml_mlp_block(ctypes.byref(d), ctypes.c_void_p(stream))
        if rc != _abi.OK:
            raise _abi.FuseMLHipError(rc, _abi.last_error(self._lib))
        self.launch_count += 1
        self._plan_ok, self._plan_pack_bytes = in_place, nbytes
        return y

    def __call__(self, *inputs: Any) -> torch.Tensor:
        if len(inputs) != self.N_INPUTS:
            raise ValueError(f"Expected {self.N_INPUTS} inputs (x, t(W1), b1, t(W2), b2, r), got {len(inputs)}.")
        if self._guard is not None:
            return self._guard.execute(self.launch, inputs)
        return self.launch(*inputs)


# ---------------------------------------------------------------------------
# Group-pair matching (compile time)
# ---------------------------------------------------------------------------


def mlp_first_group(spec: EpilogueSpec) -> Optional[Dict[str, Any]]:
    """G1 = addmm(b1, x, t(W1)) -> gelu [-> scale / add_scalar, at most
    MLP_MAX_POST]: the slots of b1/x/t(W1), the GELU form and the scalar ops."""
    if spec.reductions or spec.extra_dtypes or not spec.store_tile or not 2 <= len(spec.ops) <= 2 + _abi.MLP_MAX_POST \
            or spec.output_shapes or spec.operand_shapes:
        return None
    bias, act, post = spec.ops[0], spec.ops[1], spec.ops[2:]
    if bias.kind != "add" or bias.scalar != 1.0 or act.kind not in ("gelu_erf", "gelu_tanh"):
        return None
    if any(op.kind not in _POST_KINDS for op in post):
        return None
    return {"x": spec.left, "w1t": spec.right, "b1": bias.operand,
            "approximate": "tanh" if act.kind == "gelu_tanh" else "none",
            "post": tuple((op.kind, float(op.scalar)) for op in post)}


def mlp_second_group(spec: EpilogueSpec) -> Optional[Dict[str, Any]]:
    """G2 = addmm(b2, h, t(W2)) -> add(., r): the slots of h/t(W2)/b2/r."""
    if spec.reductions or spec.extra_dtypes or not spec.store_tile or len(spec.ops) != 2 \
            or spec.output_shapes or spec.operand_shapes:
        return None
    bias, res = spec.ops
    if bias.kind != "add" or bias.scalar != 1.0 or res.kind != "add" or res.scalar != 1.0:
        return None
    return {"h": spec.left, "w2t": spec.right, "b2": bias.operand, "r": res.operand}


def mlp_eager_fn(g1_fn: Callable[..., Any], g2_fn: Callable[..., Any], n1: int, n2: int,
                 slots1: Dict[str, int], slots2: Dict[str, int]) -> Callable[..., Any]:
    """The two groups' eager closures chained, with the launcher's input order."""

    def run(x, w1t, b1, w2t, b2, r):
        a1 = [None] * n1
        a1[slots1["x"]], a1[slots1["w1t"]], a1[slots1["b1"]] = x, w1t, b1
        h = g1_fn(*a1)
        a2 = [None] * n2
        a2[slots2["h"]], a2[slots2["w2t"]], a2[slots2["b2"]], a2[slots2["r"]] = h, w2t, b2, r
        return g2_fn(*a2)

    return run
