"""Build the gfx950 HIP kernel library in-tree: ``python -m fuseml_amd.build``.

Each ``fuseml_amd/csrc/*.hip`` is compiled by its own ``hipcc -c`` for
``--offload-arch=gfx950`` only (in parallel: the GEMM kernels are split one
tile variant per translation unit), and the objects are linked into
``fuseml_amd/libfuseml_hip.so``.  The build is ahead-of-time: there is no
runtime JIT (the reference compiles Triton kernels on the first call,
fuseml/codegen/kernel_generator.py:1067-1172).
"""

from __future__ import annotations

import concurrent.futures
import glob
import os
import shutil
import subprocess
import sys

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
INCLUDE_DIR = os.path.join(REPO_DIR, "include")
CSRC_DIR = os.path.join(PKG_DIR, "csrc")
LIB_PATH = os.path.join(PKG_DIR, "libfuseml_hip.so")
OBJ_DIR = os.path.join(PKG_DIR, "_build")

ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for every HIP translation unit.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]
# hipcc's host pass does not know the packed-fp32 feature and says so.
_NOISE = "packed-fp32-ops' is not a recognized feature"


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build fuseml_amd)")


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC_DIR, "*.hip")))


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    err = "\n".join(l for l in proc.stderr.splitlines() if _NOISE not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)


def build(verbose: bool = False, jobs: int | None = None) -> str:
    """Compile every HIP source and link the in-tree shared library; return its path."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    os.makedirs(OBJ_DIR, exist_ok=True)
    cc = hipcc()
    objs = [os.path.join(OBJ_DIR, os.path.splitext(os.path.basename(s))[0] + ".o") for s in srcs]
    cmds = [[cc, *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", "-c", s, "-o", o] for s, o in zip(srcs, objs)]
    workers = jobs or min(len(cmds), max(1, len(os.sched_getaffinity(0))), 16)
    with concurrent.futures.ThreadPoolExecutor(max_workers=workers) as pool:
        for f in [pool.submit(_run, c, verbose) for c in cmds]:
            f.result()
    tmp = LIB_PATH + ".tmp"
    _run([cc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
