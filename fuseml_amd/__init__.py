"""fuseml_amd — MI355X (gfx950) fused GEMM+epilogue path behind the FuseML backend API."""

from .epilogue import EpilogueSpec, EpiOp, UnsupportedGroup, spec_from_group

__all__ = ["EpilogueSpec", "EpiOp", "UnsupportedGroup", "spec_from_group"]
