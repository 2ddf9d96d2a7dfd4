"""ctypes binding of ``include/fuseml_hip.h`` (the C ABI of the HIP kernel family).

The structures below mirror the header field for field; ``check_abi`` compares
``sizeof(fuseml_gemm_desc)`` and the ABI version reported by the library with
the Python mirror so a stale ``.so`` is caught at load time rather than as a
garbled launch.

The library is ``fuseml_amd/libfuseml_hip.so``, built in-tree by
``fuseml_amd/build.py`` (``__graft_entry__.build()``).  There is no fallback:
if the library is missing, :func:`load_library` raises.
"""

from __future__ import annotations

import ctypes
import os
import threading
from typing import Optional

ABI_VERSION = 6
MAX_OPS = 16
MAX_OPERANDS = 8
MAX_EXTRA_OUT = 4
MLP_MAX_POST = 4

# Element types.
BF16, F16, F32 = 0, 1, 2

# Epilogue op codes.
OP_ADD = 1
OP_MUL = 2
OP_RELU = 3
OP_GELU_ERF = 4
OP_GELU_TANH = 5
OP_SIGMOID = 6
OP_SCALE = 7
OP_ADD_SCALAR = 8
OP_STORE = 9
OP_ADD_SELF = 10
OP_MUL_SELF = 11

OP_CODES = {
    "add": OP_ADD,
    "mul": OP_MUL,
    "relu": OP_RELU,
    "gelu_erf": OP_GELU_ERF,
    "gelu_tanh": OP_GELU_TANH,
    "sigmoid": OP_SIGMOID,
    "scale": OP_SCALE,
    "add_scalar": OP_ADD_SCALAR,
    "store": OP_STORE,
    "add_self": OP_ADD_SELF,
    "mul_self": OP_MUL_SELF,
}

# Reduction bits and the slot of each reduction's output buffer.
RED_SUM, RED_AMAX, RED_MEAN = 1, 2, 4
RED_BITS = {"sum": RED_SUM, "amax": RED_AMAX, "mean": RED_MEAN}
RED_SLOT = {"sum": 0, "amax": 1, "mean": 2}

# Segment codes of fuseml_split_bf16x3 (2 bits per segment) and the two
# layouts an fp32 group uses: A3 = hi | hf | lo, B3 = hi | lo | hf.
SEG_HI, SEG_LO, SEG_HI_FINITE = 0, 1, 2
SPLIT_A = SEG_HI | (SEG_HI_FINITE << 2) | (SEG_LO << 4)
SPLIT_B = SEG_HI | (SEG_LO << 2) | (SEG_HI_FINITE << 4)

# Error codes.
OK, EINVAL, EUNSUPPORTED, EHIP, EDEVICE = 0, -1, -2, -3, -4

LIBRARY_NAME = "libfuseml_hip.so"

# Every entry point the header declares (the CPU test checks they are exported).
EXPORTED_SYMBOLS = (
    "fuseml_gemm_epilogue",
    "fuseml_gemm_epilogue_supported",
    "fuseml_gemm_epilogue_config",
    "fuseml_gemm_epilogue_force_variant",
    "fuseml_gemm_epilogue_chain",
    "fuseml_last_error",
    "fuseml_device_arch",
    "fuseml_abi_version",
    "fuseml_desc_size",
    "fuseml_mlp_desc_size",
    "fuseml_mfma_peak_probe",
    "fuseml_mlp_block",
    "fuseml_mlp_block_supported",
    "fuseml_mlp_pack_bytes",
    "fuseml_mlp_pack_weights",
    "fuseml_split_bf16x3",
)


class EpiOp(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("operand", ctypes.c_int32),
        ("scalar", ctypes.c_float),
        ("reserved", ctypes.c_int32),
    ]


class Operand(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("stride_m", ctypes.c_int64),
        ("stride_n", ctypes.c_int64),
        ("extent", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class Output(ctypes.Structure):
    _fields_ = [
        ("ptr", ctypes.c_void_p),
        ("ld", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
    ]


class GemmDesc(ctypes.Structure):
    _fields_ = [
        ("M", ctypes.c_int64),
        ("N", ctypes.c_int64),
        ("K", ctypes.c_int64),
        ("a", ctypes.c_void_p),
        ("lda", ctypes.c_int64),
        ("b", ctypes.c_void_p),
        ("ldb", ctypes.c_int64),
        ("ab_dtype", ctypes.c_int32),
        ("n_ops", ctypes.c_int32),
        ("ops", EpiOp * MAX_OPS),
        ("n_operands", ctypes.c_int32),
        ("n_extra", ctypes.c_int32),
        ("operands", Operand * MAX_OPERANDS),
        ("out", Output),
        ("extra", Output * MAX_EXTRA_OUT),
        ("reduce_axis", ctypes.c_int32),
        ("reduce_mask", ctypes.c_uint32),
        ("reduce_out", ctypes.c_void_p * 3),
    ]


class MlpDesc(ctypes.Structure):
    """fuseml_mlp_desc: the single-kernel MLP block (y = post(GELU(x W1^T + b1)) W2^T + b2 + r)."""

    _fields_ = [
        ("M", ctypes.c_int64),
        ("D", ctypes.c_int64),
        ("I", ctypes.c_int64),
        ("x", ctypes.c_void_p),
        ("ldx", ctypes.c_int64),
        ("w1", ctypes.c_void_p),
        ("ldw1", ctypes.c_int64),
        ("b1", ctypes.c_void_p),
        ("w2", ctypes.c_void_p),
        ("ldw2", ctypes.c_int64),
        ("b2", ctypes.c_void_p),
        ("r", ctypes.c_void_p),
        ("ldr", ctypes.c_int64),
        ("y", ctypes.c_void_p),
        ("ldy", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("gelu", ctypes.c_int32),
        ("wpack", ctypes.c_void_p),
        ("n_post", ctypes.c_int32),
        ("post_kind", ctypes.c_int32 * MLP_MAX_POST),
        ("post_scalar", ctypes.c_float * MLP_MAX_POST),
    ]


class FuseMLHipError(RuntimeError):
    """A non-zero return code from the C ABI (recoverable by the eager guard)."""

    def __init__(self, code: int, message: str) -> None:
        super().__init__(f"fuseml_hip error {code}: {message}")
        self.code = code


_lock = threading.Lock()
_lib: Optional[ctypes.CDLL] = None


def library_path() -> str:
    return os.path.join(os.path.dirname(os.path.abspath(__file__)), LIBRARY_NAME)


def _declare(lib: ctypes.CDLL) -> None:
    desc_p = ctypes.POINTER(GemmDesc)
    lib.fuseml_gemm_epilogue.argtypes = [desc_p, ctypes.c_void_p]
    lib.fuseml_gemm_epilogue.restype = ctypes.c_int
    lib.fuseml_gemm_epilogue_supported.argtypes = [desc_p]
    lib.fuseml_gemm_epilogue_supported.restype = ctypes.c_int
    lib.fuseml_gemm_epilogue_config.argtypes = [desc_p, ctypes.POINTER(ctypes.c_int32)]
    lib.fuseml_gemm_epilogue_config.restype = ctypes.c_int
    lib.fuseml_gemm_epilogue_force_variant.argtypes = [ctypes.c_char_p]
    lib.fuseml_gemm_epilogue_force_variant.restype = ctypes.c_int
    lib.fuseml_gemm_epilogue_chain.argtypes = [desc_p]
    lib.fuseml_gemm_epilogue_chain.restype = ctypes.c_int
    lib.fuseml_last_error.argtypes = []
    lib.fuseml_last_error.restype = ctypes.c_char_p
    lib.fuseml_device_arch.argtypes = [ctypes.c_int, ctypes.c_char_p, ctypes.c_int]
    lib.fuseml_device_arch.restype = ctypes.c_int
    lib.fuseml_abi_version.argtypes = []
    lib.fuseml_abi_version.restype = ctypes.c_int
    lib.fuseml_mfma_peak_probe.argtypes = [ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p, ctypes.c_void_p]
    lib.fuseml_mfma_peak_probe.restype = ctypes.c_int
    mlp_p = ctypes.POINTER(MlpDesc)
    lib.fuseml_mlp_block.argtypes = [mlp_p, ctypes.c_void_p]
    lib.fuseml_mlp_block.restype = ctypes.c_int
    lib.fuseml_mlp_block_supported.argtypes = [mlp_p]
    lib.fuseml_mlp_block_supported.restype = ctypes.c_int
    lib.fuseml_mlp_pack_bytes.argtypes = [mlp_p]
    lib.fuseml_mlp_pack_bytes.restype = ctypes.c_int64
    lib.fuseml_mlp_pack_weights.argtypes = [mlp_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.fuseml_mlp_pack_weights.restype = ctypes.c_int
    lib.fuseml_desc_size.argtypes = []
    lib.fuseml_desc_size.restype = ctypes.c_size_t
    lib.fuseml_mlp_desc_size.argtypes = []
    lib.fuseml_mlp_desc_size.restype = ctypes.c_size_t
    i64 = ctypes.c_int64
    lib.fuseml_split_bf16x3.argtypes = [ctypes.c_void_p, i64, i64, i64, i64, ctypes.c_void_p, i64, i64,
                                        ctypes.c_uint32, ctypes.c_void_p]
    lib.fuseml_split_bf16x3.restype = ctypes.c_int


def check_abi(lib: ctypes.CDLL) -> None:
    ver = lib.fuseml_abi_version()
    size = lib.fuseml_desc_size() if ver == ABI_VERSION else -1
    mlp = lib.fuseml_mlp_desc_size() if ver == ABI_VERSION else -1
    if ver != ABI_VERSION or size != ctypes.sizeof(GemmDesc) or mlp != ctypes.sizeof(MlpDesc):
        raise ImportError(
            f"{library_path()} ABI mismatch: library v{ver} desc {size} B mlp desc {mlp} B, "
            f"binding v{ABI_VERSION} desc {ctypes.sizeof(GemmDesc)} B mlp desc {ctypes.sizeof(MlpDesc)} B "
            "— rebuild with `python -m fuseml_amd.build`"
        )


def load_library() -> ctypes.CDLL:
    """Load the HIP kernel library; raise ImportError if it is not built."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        path = library_path()
        if not os.path.exists(path):
            raise ImportError(
                f"{path} is not built — run `python -m fuseml_amd.build` "
                "(or __graft_entry__.build()) first"
            )
        lib = ctypes.CDLL(path)
        check_abi(lib)  # before binding: an older library lacks newer entry points
        _declare(lib)
        _lib = lib
        return lib


VARIANTS = ("large", "deep", "deep3", "small", "narrow64", "narrow32", "large128", "small64")


def force_variant(name: Optional[str]) -> None:
    """Pin the kernel variant for later launches in this process (None: automatic).

    ``FUSEML_HIP_TILE`` gives the initial value and is read once per process;
    this is how tests and tuning sweeps change it afterwards."""
    lib = load_library()
    rc = lib.fuseml_gemm_epilogue_force_variant(None if name is None else name.encode())
    if rc != OK:
        raise ValueError(last_error(lib))


def last_error(lib: ctypes.CDLL) -> str:
    msg = lib.fuseml_last_error()
    return msg.decode("utf-8", "replace") if msg else ""
