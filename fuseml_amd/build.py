"""Build the gfx950 HIP kernel library in-tree: ``python -m fuseml_amd.build``.

One ``hipcc`` invocation compiles ``fuseml_amd/csrc/*.hip`` into
``fuseml_amd/libfuseml_hip.so`` for ``--offload-arch=gfx950`` only.  The build
is ahead-of-time: there is no runtime JIT (the reference compiles Triton
kernels on the first call, fuseml/codegen/kernel_generator.py:1067-1172).
"""

from __future__ import annotations

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

ARCH = "gfx950"

# Packed fp32 VALU ops are disabled for every HIP translation unit.
HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-shared",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and os.path.exists(cand):
            return cand
    raise RuntimeError("hipcc not found (ROCm is required to build fuseml_amd)")


def sources() -> list[str]:
    return sorted(glob.glob(os.path.join(CSRC_DIR, "*.hip")))


def build(verbose: bool = False) -> str:
    """Compile every HIP source into the in-tree shared library; return its path."""
    srcs = sources()
    if not srcs:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    tmp = LIB_PATH + ".tmp"
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE_DIR}", *srcs, "-o", tmp]
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass does not know the packed-fp32 feature and says so; drop that noise.
    noise = "packed-fp32-ops' is not a recognized feature"
    err = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed ({proc.returncode}):\n{err}")
    if err.strip() and verbose:
        print(err, file=sys.stderr)
    os.replace(tmp, LIB_PATH)
    return LIB_PATH


if __name__ == "__main__":
    print(build(verbose=True))
