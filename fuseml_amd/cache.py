"""Launcher cache keyed on what fixes a fused launch.

Replaces the reference's kernel cache (fuseml/codegen/kernel_cache.py:45-531:
``TensorFingerprint``, ``KernelCacheKey``, ``KernelCache``, ``build_cache_key``).
Kernels are compiled ahead of time, so the cache only avoids rebuilding host
launchers; the key is (op chain with the literal arguments that change the
epilogue, per-input shape/stride/dtype fingerprints, output dtype, device
arch).  Storage offsets and data alignment are checked per call by the C ABI,
so they need not be part of the key.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional, Tuple

import torch


@dataclass(frozen=True)
class LauncherCacheKey:
    op_chain: Tuple[Tuple[str, Tuple[Any, ...]], ...]
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


def _literal(x: Any) -> Any:
    if isinstance(x, torch.fx.Node):
        return ("node",)
    if isinstance(x, (list, tuple)):
        return tuple(_literal(v) for v in x)
    return x


def _arch() -> str:
    if torch.cuda.is_available():
        try:
            return str(getattr(torch.cuda.get_device_properties(torch.cuda.current_device()), "gcnArchName", ""))
        except Exception:  # pragma: no cover
            return "unknown"
    return "cpu"


def launcher_cache_key(group: Any) -> Optional[LauncherCacheKey]:
    """Key of a group, or None when some metadata is missing or symbolic."""
    chain = []
    for n in group.all_nodes:
        args = group.node_args_snapshot.get(n.name, n.args)
        chain.append((str(n.target), _literal(tuple(args)) + tuple(sorted((k, _literal(v)) for k, v in n.kwargs.items()))))
    # where each node's operands come from (input slot or group member) matters too
    index = {id(x): i for i, x in enumerate(group.inputs)}
    members = {id(x) for x in group.all_nodes}
    wiring = []
    for n in group.all_nodes:
        args = group.node_args_snapshot.get(n.name, n.args)
        wiring.append(tuple(("in", index[id(a)]) if id(a) in index else ("grp",) if id(a) in members else ("lit",)
                            for a in args if isinstance(a, torch.fx.Node)))
    fps = []
    for n in group.inputs:
        fp = _fingerprint(n)
        if fp is None:
            return None
        fps.append(fp)
    out = group.output_metadata or {}
    if "shape" not in out:
        return None
    return LauncherCacheKey(
        op_chain=tuple(chain) + (("wiring", tuple(wiring)),),
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
