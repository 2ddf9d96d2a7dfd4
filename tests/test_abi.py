"""The C-ABI library loads, exports every symbol include/fuseml_hip.h declares,
and agrees with the Python mirror of its structures (no device calls)."""

import ctypes
import os
import re

import pytest

from fuseml_amd import _abi

HEADER = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "include", "fuseml_hip.h")


def _declared_functions():
    text = open(HEADER).read()
    return sorted(set(re.findall(r"^\s*(?:int|int64_t|const char\*|size_t)\s+(fuseml_\w+)\s*\(", text, re.M)))


def test_library_loads_and_abi_matches():
    lib = _abi.load_library()
    assert lib.fuseml_abi_version() == _abi.ABI_VERSION
    assert lib.fuseml_desc_size() == ctypes.sizeof(_abi.GemmDesc)


def test_every_declared_symbol_is_exported():
    lib = _abi.load_library()
    declared = _declared_functions()
    assert set(declared) == set(_abi.EXPORTED_SYMBOLS), declared
    for name in declared:
        assert hasattr(lib, name), name


def test_header_constants_match_binding():
    text = open(HEADER).read()
    consts = dict((k, int(v)) for k, v in re.findall(r"(FUSEML_\w+)\s*=\s*(-?\d+)", text))
    assert consts["FUSEML_OP_ADD"] == _abi.OP_ADD
    assert consts["FUSEML_OP_MUL_SELF"] == _abi.OP_MUL_SELF
    for name, code in _abi.OP_CODES.items():
        assert consts[f"FUSEML_OP_{name.upper()}"] == code, name
    assert consts["FUSEML_RED_MEAN"] == _abi.RED_MEAN
    assert consts["FUSEML_EDEVICE"] == _abi.EDEVICE
    defines = dict(re.findall(r"#define (FUSEML_MAX_\w+) (\d+)", text))
    assert int(defines["FUSEML_MAX_OPS"]) == _abi.MAX_OPS
    assert int(defines["FUSEML_MAX_OPERANDS"]) == _abi.MAX_OPERANDS
    assert int(defines["FUSEML_MAX_EXTRA_OUT"]) == _abi.MAX_EXTRA_OUT
    assert int(re.search(r"#define FUSEML_MLP_MAX_POST (\d+)", text).group(1)) == _abi.MLP_MAX_POST


def _desc(M=256, N=256, K=64):
    d = _abi.GemmDesc()
    d.M, d.N, d.K = M, N, K
    d.a, d.lda, d.b, d.ldb = 0x10000, K, 0x20000, K
    d.ab_dtype = _abi.BF16
    d.out.ptr, d.out.ld, d.out.dtype = 0x30000, N, _abi.BF16
    return d


def test_supported_checks_are_host_only():
    lib = _abi.load_library()
    d = _desc()
    assert lib.fuseml_gemm_epilogue_supported(ctypes.byref(d)) == 1
    d.K = 60  # not a multiple of 8
    assert lib.fuseml_gemm_epilogue_supported(ctypes.byref(d)) == 0
    assert "multiples of 8" in _abi.last_error(lib)
    d = _desc()
    d.ab_dtype = _abi.F32
    assert lib.fuseml_gemm_epilogue_supported(ctypes.byref(d)) == 0
    assert "MFMA" in _abi.last_error(lib)
    d = _desc()
    d.n_ops = 1
    d.ops[0].kind = _abi.OP_ADD
    d.ops[0].operand = 0  # no operands declared
    assert lib.fuseml_gemm_epilogue_supported(ctypes.byref(d)) == 0
    assert "operand index" in _abi.last_error(lib)


def _bias_gelu(d):
    """The descriptor with a bias + GELU(erf) chain (a [N] bias operand)."""
    d.n_operands = 1
    o = d.operands[0]
    o.ptr, o.stride_m, o.stride_n, o.extent, o.dtype = 0x40000, 0, 1, d.N, _abi.BF16
    d.n_ops = 2
    d.ops[0].kind, d.ops[0].operand, d.ops[0].scalar = _abi.OP_ADD, 0, 1.0
    d.ops[1].kind = _abi.OP_GELU_ERF
    return d


def test_tile_config_choice():
    """K = 1024, 4 tiles per CU: a chain with a fixed-chain kernel (here none)
    runs on the one-wave whole-stage variant, bias + GELU(erf) on the ping-pong
    one; below one round of 256x256 tiles, smaller tiles."""
    lib = _abi.load_library()
    cfg = (ctypes.c_int32 * 4)()
    assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_desc(16384, 4096, 1024)), cfg) == 0
    assert tuple(cfg[:3]) == (256, 256, 4)
    assert 128 * 1024 <= cfg[3] <= 160 * 1024
    assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_bias_gelu(_desc(16384, 4096, 1024))), cfg) == 0
    assert tuple(cfg[:3]) == (256, 256, 8)
    assert 128 * 1024 <= cfg[3] <= 160 * 1024
    assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_desc(2048, 2048, 1024)), cfg) == 0
    assert tuple(cfg[:3]) == (64, 128, 4)
    assert 2 * cfg[3] <= 160 * 1024  # two workgroups share one gfx950 CU's LDS


@pytest.mark.parametrize("shape,tile", [
    ((2048, 4096, 1024), (256, 128, 8)),  # 256 ping-pong tiles, one per CU: 384 rows x 1.2
    ((4096, 2048, 1024), (256, 128, 8)),
    ((2048, 1024, 4096), (64, 128, 4)),   # 128 tiles of 128x128: 256 of 64x128, one per CU
    ((2048, 2048, 1024), (64, 128, 4)),   # 256 tiles of 128x128 (one per CU) against 512 of 64x128 (two)
    ((8192, 512, 2048), (64, 128, 4)),
    ((1024, 1024, 1024), (32, 128, 4)),   # 64 tiles of 128x128: 256 of 32x128
    ((128, 256, 1024), (32, 128, 4)),     # the reference's small preset's second GEMM: 8 tiles
    ((1, 4096, 1024), (32, 128, 4)),      # one row
    ((64, 512, 2048), (32, 128, 4)),
    ((2048, 1024, 8192), (64, 128, 4)),   # K > 2048: one 64x128 workgroup per CU (192 rows x 1.4)
    ((128, 16384, 4096), (64, 128, 4)),   # 128 column tiles, fewer than one per CU: not weight streaming
    ((128, 8192, 1024), (32, 128, 4)),
])
def test_partial_round_tile_choice(shape, tile):
    """Below one round of 256x256 tiles the tile with the least K-loop work on
    its busiest CU: ceil(tiles / 256) x (BM + BN) operand rows, weighted 8:5
    (7:5 for K > 2048) for a lock-step tile when no CU holds two workgroups
    and 6:5 for the ping-pong tile, the first listed on a tie; also for M <=
    128 at any N."""
    lib = _abi.load_library()
    cfg = (ctypes.c_int32 * 4)()
    assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_desc(*shape)), cfg) == 0
    assert tuple(cfg[:3]) == tile
    assert cfg[3] <= 160 * 1024 and (tile[2] == 8 or 2 * cfg[3] <= 160 * 1024)


@pytest.mark.parametrize("shape,tile", [
    ((128, 32768, 4096), (128, 128)),  # 65-128 rows: the 128x128 tile at BK = 64
    ((96, 65536, 1024), (128, 128)),
    ((64, 65536, 4096), (64, 128)),    # 33-64 rows
    ((16, 65536, 1024), (32, 128)),    # up to 32 rows
])
def test_weight_streaming_tile_choice(shape, tile):
    """M <= 128 with a 128-column tile per CU or more: one row of tiles, the
    smallest BM >= M, so the weight is read once; 128 rows in K stages of 64
    (130 KB of LDS: one workgroup per CU)."""
    lib = _abi.load_library()
    cfg = (ctypes.c_int32 * 4)()
    assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_desc(*shape)), cfg) == 0
    assert (cfg[0], cfg[1], cfg[2]) == (*tile, 4)
    if tile == (128, 128):
        assert 128 * 1024 < cfg[3] <= 160 * 1024


def test_force_variant_pins_and_releases():
    lib = _abi.load_library()
    cfg = (ctypes.c_int32 * 4)()
    try:
        _abi.force_variant("small")
        assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_desc(16384, 4096, 1024)), cfg) == 0
        assert tuple(cfg[:3]) == (128, 128, 4)
        _abi.force_variant("deep3")
        assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_desc(16384, 4096, 1024)), cfg) == 0
        assert tuple(cfg[:3]) == (256, 256, 4)
        _abi.force_variant("narrow32")
        assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_desc(16384, 4096, 1024)), cfg) == 0
        assert tuple(cfg[:3]) == (32, 128, 4)
        with pytest.raises(ValueError):
            _abi.force_variant("huge")
    finally:
        _abi.force_variant(None)
    assert lib.fuseml_gemm_epilogue_config(ctypes.byref(_bias_gelu(_desc(16384, 4096, 1024))), cfg) == 0
    assert tuple(cfg[:3]) == (256, 256, 8)


def test_operand_span_limit_is_per_tile():
    """Buffer accesses are based at each tile's origin: an operand larger than
    2 GiB is accepted when one tile's elements span less than that."""
    lib = _abi.load_library()
    d = _desc(40000, 32768, 64)
    d.n_operands = 1
    o = d.operands[0]
    o.ptr, o.stride_m, o.stride_n, o.dtype = 0x10000, 32768, 1, _abi.BF16
    o.extent = 40000 * 32768                     # 2.6 GB of bf16
    d.n_ops = 1
    d.ops[0].kind, d.ops[0].operand = _abi.OP_ADD, 0
    assert lib.fuseml_gemm_epilogue_supported(ctypes.byref(d)) == 1, _abi.last_error(lib)
    o.stride_m = 1 << 23                         # 256 rows of this stride span 4 GiB
    o.extent = 39999 * (1 << 23) + 32768
    assert lib.fuseml_gemm_epilogue_supported(ctypes.byref(d)) == 0
    assert "2 GiB" in _abi.last_error(lib)


def test_mlp_pack_bytes_is_host_only():
    """The repacked-weight size: 4 * D * I bytes where the single-kernel MLP
    streams weight fragments (D of 256 or 512, I a multiple of 128), else 0."""
    lib = _abi.load_library()
    d = _abi.MlpDesc()
    d.M, d.D, d.I = 1000, 256, 1024
    d.x, d.ldx, d.w1, d.ldw1, d.b1 = 0x10000, 256, 0x20000, 256, 0x30000
    d.w2, d.ldw2, d.y, d.ldy = 0x40000, 1024, 0x50000, 256
    d.dtype, d.gelu = _abi.BF16, _abi.OP_GELU_ERF
    assert lib.fuseml_mlp_pack_bytes(ctypes.byref(d)) == 4 * 256 * 1024
    d.I, d.ldw2 = 96, 96                      # not a multiple of 128: the D-split kernel, no packing
    assert lib.fuseml_mlp_pack_bytes(ctypes.byref(d)) == 0
    d.D, d.I, d.ldx, d.ldw1, d.ldw2, d.ldy = 1024, 1024, 1024, 1024, 1024, 1024
    assert lib.fuseml_mlp_pack_bytes(ctypes.byref(d)) == 0
    d.D = 300                                 # unsupported width: invalid descriptor
    assert lib.fuseml_mlp_pack_bytes(ctypes.byref(d)) == 0
