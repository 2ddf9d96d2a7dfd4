"""Which epilogue a launch compiles in, decided on the host (no device calls).

``fuseml_gemm_epilogue_chain`` runs the library's own host path (validation,
flag derivation, variant choice, chain matching) on a descriptor whose
pointers are never dereferenced, and returns the fixed chain kernel the launch
would use (0: the generic op loop).  The ids are ``FixedChain`` in
``fuseml_amd/csrc/gemm_epilogue_shared.h``.  The GPU tests check that each
fixed kernel gives bitwise the generic loop's results; these tests pin which
descriptors reach which kernel, including every condition that must keep a
descriptor on the generic path.
"""

import pytest

from fuseml_amd import _abi

NONE, BIAS, GELU, GELU_TANH, BIAS_RELU, BIAS_TILE, ACT_HEAVY, RELU = 1, 2, 3, 4, 5, 6, 7, 8

ROW, TILE, ROW2, COL = 0, 1, 2, 3  # operand slots below


def _desc(M=1024, N=1024, K=1024, ab=_abi.BF16, tile_dtype=_abi.BF16):
    d = _abi.GemmDesc()
    d.M, d.N, d.K = M, N, K
    d.a, d.lda, d.b, d.ldb = 0x100000, K, 0x200000, K
    d.ab_dtype = ab
    d.out.ptr, d.out.ld, d.out.dtype = 0x300000, N, _abi.BF16
    ops = [
        (0x400000, 0, 1, N, _abi.BF16),           # row vector [N]
        (0x500000, N, 1, M * N, tile_dtype),      # 2-D tile [M, N]
        (0x600000, 0, 1, N, _abi.BF16),           # second row vector
        (0x700000, 1, 0, M, _abi.BF16),           # column vector [M, 1]
    ]
    for i, (p, sm, sn, ext, dt) in enumerate(ops):
        o = d.operands[i]
        o.ptr, o.stride_m, o.stride_n, o.extent, o.dtype = p, sm, sn, ext, dt
    d.n_operands = len(ops)
    return d


def _ops(d, chain):
    d.n_ops = len(chain)
    for i, (kind, operand, scalar) in enumerate(chain):
        op = d.ops[i]
        op.kind, op.operand, op.scalar = _abi.OP_CODES[kind], operand, scalar
    return d


@pytest.fixture
def lib():
    lib = _abi.load_library()
    yield lib
    _abi.force_variant(None)


def _chain(lib, d, variant="deep3"):
    _abi.force_variant(variant)
    return lib.fuseml_gemm_epilogue_chain(d)


CASES = {
    "none": ([], NONE),
    "bias": ([("add", ROW, 1.0)], BIAS),
    "bias_alpha": ([("add", ROW, -0.5)], BIAS),
    "bias_gelu": ([("add", ROW, 1.0), ("gelu_erf", -1, 1.0)], GELU),
    "bias_gelu_tanh": ([("add", ROW, 1.0), ("gelu_tanh", -1, 1.0)], GELU_TANH),
    "bias_relu": ([("add", ROW, 1.0), ("relu", -1, 1.0)], BIAS_RELU),
    "bias_residual": ([("add", ROW, 1.0), ("add", TILE, 1.0)], BIAS_TILE),
    "act_heavy": ([("add", ROW, 1.0), ("relu", -1, 1.0), ("mul", TILE, 1.0), ("sigmoid", -1, 1.0),
                   ("add", ROW2, 1.0)], ACT_HEAVY),
    "relu": ([("relu", -1, 1.0)], RELU),
}


@pytest.mark.parametrize("name", sorted(CASES))
def test_each_fixed_chain_is_matched(lib, name):
    chain, want = CASES[name]
    assert _chain(lib, _ops(_desc(), chain)) == want


@pytest.mark.parametrize("name", sorted(CASES))
def test_generic_pin_and_other_variants_keep_the_op_loop(lib, name):
    chain, _ = CASES[name]
    for variant in ("deep3-generic", "large", "deep", "small", "narrow64", "narrow32", "large128", "small64"):
        assert _chain(lib, _ops(_desc(), chain), variant) == 0, variant


def test_relu_with_reductions_is_fixed_other_chains_with_reductions_are_not(lib):
    for chain, want in ((CASES["relu"][0], RELU), (CASES["bias_gelu"][0], 0), (CASES["none"][0], 0)):
        d = _ops(_desc(), chain)
        d.reduce_mask, d.reduce_axis = _abi.RED_SUM | _abi.RED_AMAX, 1
        d.reduce_out[0], d.reduce_out[1] = 0x800000, 0x900000
        assert _chain(lib, d) == want


def test_conditions_that_keep_the_generic_loop(lib):
    gelu = CASES["bias_gelu"][0]
    # f16 GEMM operands: fixed chains are built for bf16 only
    assert _chain(lib, _ops(_desc(ab=_abi.F16), gelu)) == 0
    # an escape store in the chain
    d = _ops(_desc(), [("add", ROW, 1.0), ("store", 0, 1.0), ("gelu_erf", -1, 1.0)])
    d.n_extra = 1
    d.extra[0].ptr, d.extra[0].ld, d.extra[0].dtype = 0xA00000, 1024, _abi.BF16
    assert _chain(lib, d) == 0
    # a column vector ([M, 1]) where the chain expects a row vector
    assert _chain(lib, _ops(_desc(), [("add", COL, 1.0), ("gelu_erf", -1, 1.0)])) == 0
    # the bias is a 2-D tile, not a vector
    assert _chain(lib, _ops(_desc(), [("add", TILE, 1.0), ("gelu_erf", -1, 1.0)])) == 0
    # residual that cannot be LDS-staged: fp32, or N not a multiple of 8
    resid = CASES["bias_residual"][0]
    assert _chain(lib, _ops(_desc(tile_dtype=_abi.F32), resid)) == 0
    assert _chain(lib, _ops(_desc(N=1020), resid)) == 0
    # K % 64 != 0: the deep3 pin falls back to the two-stage one-wave variant
    assert _chain(lib, _ops(_desc(K=1000), gelu)) == 0
    # an op order the fixed kernels do not hold
    assert _chain(lib, _ops(_desc(), [("gelu_erf", -1, 1.0), ("add", ROW, 1.0)])) == 0
    # an invalid descriptor is an error code, not a chain
    bad = _ops(_desc(), gelu)
    bad.M = 0
    assert _chain(lib, bad) == _abi.EINVAL
