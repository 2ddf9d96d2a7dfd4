"""Eager fallback for a fused launch that fails at run time.

Same contract as the reference's ``EagerFallbackGuard``
(fuseml/codegen/eager_fallback.py:63-298): try the fused launch; on a
recoverable error (``RuntimeError`` — which includes every non-zero C-ABI
return, see ``_abi.FuseMLHipError`` — eager_fallback.py:147-166) count it, log
it, synchronise the device, release the fused path's buffers (emptying the
allocator cache after an out-of-memory error, 179-265) and return
``eager_fn(*inputs)``.  ``TypeError``/``ValueError`` and signals propagate.

Differences, both deliberate:
* inputs are not cloned before the launch: the HIP kernels never write their
  inputs, so the clone the reference takes on every call (eager_fallback.py:131)
  buys nothing;
* ``FUSEML_HIP_FORCE_FAIL=1`` makes every guarded launch raise before touching
  the device, so the fallback path can be exercised from the host.
"""

from __future__ import annotations

import logging
import os
from typing import Any, Callable, Sequence

import torch

logger = logging.getLogger("fuseml_amd")

FORCE_FAIL_ENV = "FUSEML_HIP_FORCE_FAIL"


class ForcedFailure(RuntimeError):
    """Raised instead of launching when FUSEML_HIP_FORCE_FAIL is set."""


class EagerFallbackGuard:
    def __init__(self, eager_fn: Callable[..., Any], kernel_signature: str) -> None:
        self._eager_fn = eager_fn
        self._kernel_signature = kernel_signature
        self._fallback_count = 0

    @property
    def fallback_count(self) -> int:
        return self._fallback_count

    @property
    def kernel_signature(self) -> str:
        return self._kernel_signature

    @staticmethod
    def is_recoverable(exc: BaseException) -> bool:
        return isinstance(exc, RuntimeError)

    @staticmethod
    def is_oom(exc: BaseException) -> bool:
        return "out of memory" in str(exc).lower()

    def execute(self, launch_fn: Callable[..., Any], inputs: Sequence[Any]) -> Any:
        """``launch_fn(*inputs)``, or the eager path after a recoverable error."""
        try:
            if os.environ.get(FORCE_FAIL_ENV, "") not in ("", "0"):
                raise ForcedFailure(f"{FORCE_FAIL_ENV} set")
            return launch_fn(*inputs)
        except Exception as exc:  # noqa: BLE001 - filtered below
            if not self.is_recoverable(exc):
                raise
            return self._fallback(exc, inputs)

    def _fallback(self, exc: BaseException, inputs: Sequence[Any]) -> Any:
        self._fallback_count += 1
        logger.warning(
            "fused kernel '%s' failed (#%d): %s: %s — running the eager path",
            self._kernel_signature,
            self._fallback_count,
            type(exc).__name__,
            exc,
        )
        for t in inputs:
            if isinstance(t, torch.Tensor) and t.device.type == "cuda":
                torch.cuda.synchronize(t.device)
                if self.is_oom(exc):
                    torch.cuda.empty_cache()
                break
        return self._eager_fn(*inputs)
