"""Launcher cache keyed on what fixes a fused launch.

Replaces the reference's kernel cache (fuseml/codegen/kernel_cache.py:45-531:
``TensorFingerprint``, ``KernelCacheKey``, ``KernelCache``, ``build_cache_key``).
Kernels are compiled ahead of time, so the cache only avoids rebuilding host
launchers; the key is (the group's derived :class:`EpilogueSpec` — op chain
with operand positions and scalars, reductions, escape stores and the order of
the returned values —, per-input shape/stride/dtype fingerprints, output
shape and dtype, device arch).  Keying on the spec rather than on the node
targets keeps two groups whose chains match but whose return signatures
differ (e.g. the same reductions with and without the reduced value escaping)
apart.  Storage offsets and data alignment are checked per call by the C ABI,
so they need not be part of the key.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch


@dataclass(frozen=True)
class LauncherCacheKey:
    spec: Any  # EpilogueSpec (frozen, hashable)
    inputs: Tuple[Tuple[Tuple[int, ...], Tuple[int, ...], str], ...]
    output: Tuple[Tuple[int, ...], str]
    arch: str


def _fingerprint(node: Any) -> Optional[Tuple[Tuple[int, ...], Tuple[int, ...], str]]:
    meta = getattr(node, "meta", {}) or {}
    tm = meta.get("tensor_meta")
    if tm is not None and hasattr(tm, "shape"):
        return tuple(int(s) for s in tm.shape), tuple(int(s) for s in tm.stride), str(tm.dtype)
    val = meta.get("val")
    if val is not None and hasattr(val, "shape"):
        try:
            return tuple(int(s) for s in val.shape), tuple(int(s) for s in val.stride()), str(val.dtype)
        except TypeError:  # symbolic sizes: not cacheable
            return None
    return None


def _arch() -> str:
    if torch.cuda.is_available():
        try:
            return str(getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", ""))
        except Exception:  # pragma: no cover
            return "unknown"
    return "cpu"


def launcher_cache_key(group: Any, spec: Any) -> Optional[LauncherCacheKey]:
    """Key of a group whose spec is `spec`, or None when some metadata is
    missing or symbolic."""
    fps = []
    for n in group.inputs:
        fp = _fingerprint(n)
        if fp is None:
            return None
        fps.append(fp)
    out = getattr(group, "output_metadata", None) or {}
    if "shape" not in out:
        return None
    return LauncherCacheKey(
        spec=spec,
        inputs=tuple(fps),
        output=(tuple(int(s) for s in out["shape"]), str(out["dtype"])),
        arch=_arch(),
    )


class LauncherCache:
    def __init__(self) -> None:
        self._store: Dict[LauncherCacheKey, Any] = {}
        self.hits = 0
        self.misses = 0

    def lookup(self, key: LauncherCacheKey) -> Any:
        v = self._store.get(key)
        if v is None:
            self.misses += 1
        else:
            self.hits += 1
        return v

    def store(self, key: LauncherCacheKey, launcher: Any) -> None:
        self._store[key] = launcher

    def __len__(self) -> int:
        return len(self._store)

    def clear(self) -> None:
        self._store.clear()
        self.hits = self.misses = 0
