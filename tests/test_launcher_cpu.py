"""HipKernelLauncher host logic with the C entry point replaced by a recorder (CPU).

Pins the launcher's calling convention (the reference's KernelLauncher
contract, fuseml/codegen/kernel_launcher.py:640-821): arity check, left/right
operand roles, M/N/K extraction, output allocation, descriptor contents
(strides, op codes, operand slots, broadcast strides), return order, and the
eager fallback (forced from the host).  No device call is made.
"""

import ctypes

import pytest
import torch

from fuseml_amd import _abi
from fuseml_amd.epilogue import EpilogueSpec, EpiOp
from fuseml_amd.fallback import FORCE_FAIL_ENV
from fuseml_amd.launcher import HipKernelLauncher


class Recorder:
    """Stands in for the library: records each descriptor, returns `rc`."""

    def __init__(self, rc=0, msg=b"", split_rc=0):
        self.calls = []
        self.splits = []
        self.rc = rc
        self.split_rc = split_rc
        self.msg = msg

    def fuseml_gemm_epilogue(self, desc_ref, stream):
        d = ctypes.cast(desc_ref, ctypes.POINTER(_abi.GemmDesc)).contents
        snap = {
            "M": d.M, "N": d.N, "K": d.K, "lda": d.lda, "ldb": d.ldb, "ab": d.ab_dtype,
            "ops": [(d.ops[i].kind, d.ops[i].operand, d.ops[i].scalar) for i in range(d.n_ops)],
            "operands": [(d.operands[i].stride_m, d.operands[i].stride_n, d.operands[i].extent,
                          d.operands[i].dtype) for i in range(d.n_operands)],
            "out": (bool(d.out.ptr), d.out.ld, d.out.dtype),
            "n_extra": d.n_extra, "mask": d.reduce_mask, "axis": d.reduce_axis,
            "a": d.a, "b": d.b,
        }
        self.calls.append(snap)
        return self.rc

    def fuseml_split_bf16x3(self, src, rows, K, stride_r, stride_k, dst, ld_dst, k_pad, seg_codes, stream):
        self.splits.append({"src": src.value, "rows": rows, "K": K, "sr": stride_r, "sk": stride_k,
                            "dst": dst.value, "ld": ld_dst, "k_pad": k_pad, "mask": seg_codes})
        return self.split_rc

    def fuseml_last_error(self):
        return self.msg


def make(spec, n, rec, eager=None):
    launcher = HipKernelLauncher(spec, n, eager_fn=eager)
    launcher._lib = rec
    return launcher


BF = torch.bfloat16


def test_descriptor_for_bias_gelu():
    rec = Recorder()
    spec = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("gelu_erf")), BF)
    b, x, w = torch.randn(48, dtype=BF), torch.randn(32, 64, dtype=BF), torch.randn(48, 64, dtype=BF)
    out = make(spec, 3, rec)(b, x, w.t())
    c = rec.calls[0]
    assert (c["M"], c["N"], c["K"]) == (32, 48, 64)
    assert c["lda"] == 64 and c["ldb"] == 64           # t(W) is K-contiguous: no copy
    assert c["b"] == w.data_ptr() and c["a"] == x.data_ptr()
    assert c["ops"] == [(_abi.OP_ADD, 0, 1.0), (_abi.OP_GELU_ERF, -1, 1.0)]
    assert c["operands"] == [(0, 1, 48, _abi.BF16)]     # [N] bias broadcast over M
    assert c["out"] == (True, 48, _abi.BF16) and c["mask"] == 0
    assert out.shape == (32, 48) and out.dtype == BF and out.is_contiguous()


def test_operand_slots_dedupe_and_broadcast_kinds():
    rec = Recorder()
    ops = (EpiOp("add", 0), EpiOp("mul", 3), EpiOp("add", 4, 2.0), EpiOp("mul", 0), EpiOp("add", 5))
    spec = EpilogueSpec(1, 2, ops, BF)
    M, N, K = 8, 16, 24
    b = torch.randn(N, dtype=BF)
    x, wt = torch.randn(M, K, dtype=BF), torch.randn(N, K, dtype=BF).t()
    tile = torch.randn(M, N, dtype=BF)
    col = torch.randn(M, 1, dtype=torch.float16)
    scalar = torch.tensor(3.0)
    make(spec, 6, rec)(b, x, wt, tile, col, scalar)
    c = rec.calls[0]
    # operand 0 appears twice but occupies one slot
    assert [o[1] for o in c["ops"]] == [0, 1, 2, 0, 3]
    assert c["operands"][0] == (0, 1, N, _abi.BF16)
    assert c["operands"][1] == (N, 1, M * N, _abi.BF16)
    assert c["operands"][2] == (1, 0, M, _abi.F16)           # column vector
    assert c["operands"][3] == (0, 0, 1, _abi.F32)           # 0-d tensor
    assert c["ops"][2][2] == 2.0


def test_relayout_of_non_k_contiguous_operands():
    rec = Recorder()
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), BF)
    a = torch.randn(64, 32, dtype=BF).t()           # [32,64] with stride (1,32): not K-contiguous
    b = torch.randn(64, 40, dtype=BF)               # [K,N] row-major: N-contiguous
    make(spec, 2, rec)(a, b)
    c = rec.calls[0]
    assert (c["M"], c["N"], c["K"]) == (32, 40, 64)
    assert c["lda"] == 64 and c["ldb"] == 64


def test_reductions_and_return_order():
    rec = Recorder()
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), BF, store_tile=True, reductions=("sum", "amax", "mean"),
                        reduce_axis=1, reduce_dtypes=(torch.float32, BF, torch.float32),
                        outputs=(("red", "sum"), ("red", "amax"), ("red", "mean"), ("tile",)))
    s, mx, mean, tile = make(spec, 2, rec)(torch.randn(8, 16, dtype=BF), torch.randn(24, 16, dtype=BF).t())
    c = rec.calls[0]
    assert c["mask"] == 7 and c["axis"] == 1
    assert s.shape == (8,) and s.dtype == torch.float32
    assert mx.dtype == BF                         # accumulated in fp32, cast to the node's dtype
    assert tile.shape == (8, 24)


def test_arity_error_is_value_error():
    spec = EpilogueSpec(0, 1, (), BF)
    with pytest.raises(ValueError, match="Expected 2"):
        make(spec, 2, Recorder())(torch.randn(4, 8, dtype=BF))


def test_negative_stride_detection():
    """torch never produces negative strides (flip copies); the guard is checked on stubs,
    as the reference does with fake tensors (tests/test_kernel_launcher.py:379-391)."""
    from fuseml_amd.launcher import _has_negative_stride

    class Stub:
        def __init__(self, st):
            self._st = st

        def stride(self):
            return self._st

    assert _has_negative_stride(Stub((-24, 1)))
    assert not _has_negative_stride(Stub((0, 1)))
    assert not _has_negative_stride(torch.randn(3, 4).t())


def test_error_code_raises_runtime_error_without_guard():
    spec = EpilogueSpec(0, 1, (), BF)
    launcher = make(spec, 2, Recorder(rc=_abi.EUNSUPPORTED, msg=b"no variant"))
    with pytest.raises(_abi.FuseMLHipError, match="no variant"):
        launcher(torch.randn(4, 8, dtype=BF), torch.randn(8, 8, dtype=BF).t())


def test_error_code_falls_back_to_eager():
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), BF)
    eager = lambda a, b: torch.relu(a @ b)  # noqa: E731
    launcher = make(spec, 2, Recorder(rc=_abi.EHIP, msg=b"launch failed"), eager=eager)
    a, b = torch.randn(4, 8, dtype=BF), torch.randn(8, 8, dtype=BF).t()
    out = launcher(a, b)
    assert torch.equal(out, eager(a, b))
    assert launcher.fallback_count == 1


def test_forced_failure_from_host(monkeypatch):
    rec = Recorder()
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), BF)
    eager = lambda a, b: torch.relu(a @ b)  # noqa: E731
    launcher = make(spec, 2, rec, eager=eager)
    monkeypatch.setenv(FORCE_FAIL_ENV, "1")
    a, b = torch.randn(4, 8, dtype=BF), torch.randn(8, 8, dtype=BF).t()
    assert torch.equal(launcher(a, b), eager(a, b))
    assert rec.calls == [] and launcher.fallback_count == 1


def test_value_errors_are_not_swallowed_by_guard():
    spec = EpilogueSpec(0, 1, (), BF)
    launcher = make(spec, 2, Recorder(), eager=lambda *a: None)
    with pytest.raises(ValueError):
        launcher(torch.randn(4, 8, dtype=BF))


def test_unsupported_gemm_dtype_raises():
    spec = EpilogueSpec(0, 1, (), torch.float64)
    launcher = make(spec, 2, Recorder())
    with pytest.raises(_abi.FuseMLHipError, match="bf16, f16 or fp32"):
        launcher(torch.randn(4, 8, dtype=torch.float64), torch.randn(8, 8, dtype=torch.float64).t())
    with pytest.raises(_abi.FuseMLHipError, match="bf16, f16 or fp32"):
        launcher(torch.randn(4, 8), torch.randn(8, 8, dtype=BF).t())


def test_fp32_operands_are_split_then_one_bf16_gemm():
    """fp32 A and t(W): each is split into [M|N, 3 k_pad] bf16 parts (A as
    hi|hi|lo, the weight rows as hi|lo|hi), and the GEMM runs on the parts
    with K' = 3 k_pad; the epilogue and the fp32 output are unchanged."""
    rec = Recorder()
    M, N, K = 6, 20, 13            # K % 8 != 0: padded to 16 per segment
    spec = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("relu")), torch.float32)
    b, x, w = torch.randn(N), torch.randn(M, K), torch.randn(N, K)
    out = make(spec, 3, rec)(b, x, w.t())
    sa, sb = rec.splits
    assert (sa["src"], sa["rows"], sa["K"], sa["sr"], sa["sk"], sa["mask"]) == (x.data_ptr(), M, K, K, 1, _abi.SPLIT_A)
    assert (sb["src"], sb["rows"], sb["K"], sb["sr"], sb["sk"], sb["mask"]) == (w.data_ptr(), N, K, K, 1, _abi.SPLIT_B)
    assert sa["k_pad"] == sb["k_pad"] == 16 and sa["ld"] == sb["ld"] == 48
    c = rec.calls[0]
    assert (c["M"], c["N"], c["K"], c["lda"], c["ldb"], c["ab"]) == (M, N, 48, 48, 48, _abi.BF16)
    assert c["a"] == sa["dst"] and c["b"] == sb["dst"]
    assert c["operands"] == [(0, 1, N, _abi.F32)] and c["out"] == (True, N, _abi.F32)
    assert out.dtype == torch.float32 and out.shape == (M, N)
    # strided K: the split reads the operand in place, whatever its strides
    n_before = len(rec.splits)
    x2 = torch.randn(M, 2 * K)[:, ::2]
    make(spec, 3, rec)(b, x2, w.t())
    sa2 = rec.splits[n_before]
    assert (sa2["src"], sa2["sr"], sa2["sk"]) == (x2.data_ptr(), 2 * K, 2)


def test_fp32_split_error_is_a_hip_error():
    rec = Recorder(split_rc=_abi.EINVAL, msg=b"split_bf16x3: bad sizes")
    spec = EpilogueSpec(0, 1, (), torch.float32)
    with pytest.raises(_abi.FuseMLHipError, match="bad sizes"):
        make(spec, 2, rec)(torch.randn(4, 8), torch.randn(8, 8).t())
    assert rec.calls == []


def test_name_for_fx():
    assert HipKernelLauncher(EpilogueSpec(0, 1, (), BF), 2).__name__ == "fuseml_fused_kernel"


def test_nd_operands_and_output_views():
    """[*lead, N] groups: operands broadcast against the N-D value then merged
    to [M,N]; outputs returned as views of the group's shapes."""
    rec = Recorder()
    B, S, N, K = 2, 4, 16, 8
    ops = (EpiOp("add", 0), EpiOp("add", 3), EpiOp("mul", 4), EpiOp("add", 5))
    shape = (B, S, N)
    spec = EpilogueSpec(1, 2, ops, BF, operand_shapes=((3, shape), (4, shape), (5, shape)),
                        output_shapes=(shape,))
    b = torch.randn(N, dtype=BF)
    x, wt = torch.randn(B * S, K, dtype=BF), torch.randn(N, K, dtype=BF).t()
    resid = torch.randn(B, S, N, dtype=BF)          # contiguous: merges to (N, 1)
    per_batch = torch.randn(B, 1, N, dtype=BF)      # strides do not merge: materialised
    row = torch.randn(1, 1, N, dtype=BF)            # broadcast row: (0, 1)
    out = make(spec, 6, rec)(b, x, wt, resid, per_batch, row)
    c = rec.calls[0]
    assert (c["M"], c["N"], c["K"]) == (B * S, N, K)
    assert c["operands"][0] == (0, 1, N, _abi.BF16)
    assert c["operands"][1] == (N, 1, B * S * N, _abi.BF16)
    assert c["operands"][2] == (N, 1, B * S * N, _abi.BF16)
    assert c["operands"][3] == (0, 1, N, _abi.BF16)
    assert out.shape == shape and out.is_contiguous()


@pytest.mark.parametrize("axis", [1, 0])
def test_empty_reduction_axis_matches_torch(axis):
    """M or N zero: no launch; a reduction over the empty axis is sum 0 and
    mean NaN, and amax raises IndexError like torch.amax."""
    rec = Recorder()
    M, N = (8, 0) if axis == 1 else (0, 8)
    x, w = torch.randn(M, 16, dtype=BF), torch.randn(N, 16, dtype=BF)
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), BF, store_tile=False, reductions=("sum", "mean"),
                        reduce_axis=axis, reduce_dtypes=(torch.float32,) * 2,
                        outputs=(("red", "sum"), ("red", "mean")))
    s, mean = make(spec, 2, rec)(x, w.t())
    h = torch.relu(x.float() @ w.float().t())
    assert rec.calls == []
    assert torch.equal(s, h.sum(axis)) and torch.equal(mean.isnan(), h.mean(axis).isnan())
    spec_max = EpilogueSpec(0, 1, (EpiOp("relu"),), BF, store_tile=False, reductions=("amax",),
                            reduce_axis=axis, reduce_dtypes=(torch.float32,), outputs=(("red", "amax"),))
    with pytest.raises(IndexError):
        make(spec_max, 2, rec)(x, w.t())


def test_empty_rows_give_empty_reductions():
    rec = Recorder()
    x, w = torch.randn(0, 16, dtype=BF), torch.randn(8, 16, dtype=BF)
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), BF, store_tile=True, reductions=("amax",),
                        reduce_axis=1, reduce_dtypes=(torch.float32,), outputs=(("tile",), ("red", "amax")))
    tile, mx = make(spec, 2, rec)(x, w.t())
    assert tile.shape == (0, 8) and mx.shape == (0,) and rec.calls == []


def test_plan_reuse_takes_each_calls_pointers():
    """The descriptor's non-pointer fields are filled once per input signature;
    every call still sets its own input and output pointers."""
    rec = Recorder()
    spec = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("add", 3)), BF)
    M, N, K = 16, 24, 32
    launcher = make(spec, 4, rec)

    def args():
        return (torch.randn(N, dtype=BF), torch.randn(M, K, dtype=BF), torch.randn(N, K, dtype=BF).t(),
                torch.randn(M, N, dtype=BF))

    first, second = args(), args()
    out1 = launcher(*first)
    out2 = launcher(*second)
    assert len(launcher._plans) == 1
    c1, c2 = rec.calls
    assert (c1["a"], c1["b"]) == (first[1].data_ptr(), first[2].data_ptr())
    assert (c2["a"], c2["b"]) == (second[1].data_ptr(), second[2].data_ptr())
    assert c1["operands"] == c2["operands"] == [(0, 1, N, _abi.BF16), (N, 1, M * N, _abi.BF16)]
    assert out1 is not out2 and out1.shape == out2.shape == (M, N)  # fresh outputs per call


def test_plan_rebuilds_converted_operands_every_call():
    """An operand the kernel cannot read in its own dtype (int here) is converted
    per call, and the descriptor points at that call's converted copy."""
    seen = []

    class PtrRecorder(Recorder):
        def fuseml_gemm_epilogue(self, desc_ref, stream):
            d = ctypes.cast(desc_ref, ctypes.POINTER(_abi.GemmDesc)).contents
            seen.append((d.operands[0].ptr, d.operands[0].dtype))
            return super().fuseml_gemm_epilogue(desc_ref, stream)

    rec = PtrRecorder()
    spec = EpilogueSpec(1, 2, (EpiOp("add", 0),), BF)
    M, N, K = 8, 16, 24
    launcher = make(spec, 3, rec)
    x, wt = torch.randn(M, K, dtype=BF), torch.randn(N, K, dtype=BF).t()
    b1, b2 = torch.arange(N, dtype=torch.int32), torch.arange(N, dtype=torch.int32) * 2
    launcher(b1, x, wt)
    launcher(b2, x, wt)
    assert len(launcher._plans) == 1
    assert [dt for _, dt in seen] == [_abi.F32, _abi.F32]
    assert seen[0][0] not in (b1.data_ptr(), b2.data_ptr()) and seen[1][0] not in (b1.data_ptr(), b2.data_ptr())


def test_new_signature_gets_its_own_plan():
    rec = Recorder()
    spec = EpilogueSpec(0, 1, (EpiOp("relu"),), BF)
    launcher = make(spec, 2, rec)
    launcher(torch.randn(8, 16, dtype=BF), torch.randn(24, 16, dtype=BF).t())
    launcher(torch.randn(40, 16, dtype=BF), torch.randn(24, 16, dtype=BF).t())
    assert len(launcher._plans) == 2
    assert [(c["M"], c["N"], c["K"]) for c in rec.calls] == [(8, 24, 16), (40, 24, 16)]


def test_host_tensors_are_refused_before_any_device_call():
    """With the real library bound, CPU tensors (or tensors on different
    devices) raise a recoverable error instead of reaching a kernel that would
    dereference host pointers on the GPU; the eager guard then takes over."""
    spec = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("relu")), BF)
    b, x, w = torch.randn(16, dtype=BF), torch.randn(8, 32, dtype=BF), torch.randn(16, 32, dtype=BF)
    launcher = HipKernelLauncher(spec, 3)                   # the real library (loads without a GPU)
    assert isinstance(launcher._lib, ctypes.CDLL)
    with pytest.raises(_abi.FuseMLHipError, match="must be on the launch's GPU"):
        launcher(b, x, w.t())
    guarded = HipKernelLauncher(spec, 3, eager_fn=lambda bb, xx, ww: torch.relu(torch.addmm(bb, xx, ww)))
    out = guarded(b, x, w.t())
    assert guarded.fallback_count == 1 and torch.equal(out, torch.relu(torch.addmm(b, x, w.t())))
