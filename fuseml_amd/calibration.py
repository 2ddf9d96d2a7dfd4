"""The measurement behind the cost model's two thresholds (fused kernel or eager).

    python -m fuseml_amd.calibration [--out profiles/cost_model_calibration.json]
    python -m fuseml_amd.calibration --mlp [--out profiles/mlp_block_crossover.json]

For each group below, on one GPU, the same inputs run three ways:

* ``fused``: the group through :class:`~fuseml_amd.launcher.HipKernelLauncher`
  (one launch of the gfx950 kernel family, automatic variant);
* ``eager``: the group's PyTorch ops (hipBLASLt's GEMM with the addmm bias in
  its epilogue, then one elementwise kernel per remaining op);
* ``mm``: hipBLASLt's plain GEMM alone (what eager's GEMM costs without the
  epilogue passes).

Each time is the median of HIP-event timed calls (per call: event, launch,
event), the best of two alternating passes.  The groups are the benchmark
configs' six GEMM groups at full size, a K sweep of one- and four-pass chains
at 256+ tiles, a few-tile sweep (fewer 128x128 output tiles than CUs) of a
bias+GELU chain over K, and the few-tile groups of the reference's `small` and
`medium` presets.  They replace the reference's NVIDIA tables
(fuseml/passes/topology.py:286-571), which on ROCm fall to defaults.

Each row records the chain's elementwise passes
(:func:`fuseml_amd.compiler.epilogue_passes`), the 128x128 tile count, the
three times, and which path won; ``tests/test_cost_model_calibration.py``
checks that :func:`fuseml_amd.compiler.fused_beats_eager` and the few-tile
rule of :func:`fuseml_amd.compiler.trigger_is_fusible` pick the measured
winner on every row where the two differ by more than the tie margin.
"""

from __future__ import annotations

import argparse
import json
import statistics
import sys
import time
from typing import Callable, Dict, List, Tuple

import torch
import torch.nn.functional as F

BF = torch.bfloat16

# (label, chain, M, N, K).  Chains: "bias_gelu" (addmm + GELU, 1 pass),
# "bias_residual" (addmm + residual add, 1 pass), "bias_gelu_residual"
# (addmm, GELU, residual add: 2 passes), "act_heavy" (addmm, ReLU, gate
# product, sigmoid, row add: 4 passes), "relu_3red" (mm, ReLU, row sum, amax
# and mean: 4 passes).
CONFIG_GROUPS: List[Tuple[str, str, int, int, int]] = [
    ("C2 G1", "bias_gelu", 16384, 4096, 1024),
    ("C2 G2", "bias_residual", 16384, 1024, 4096),
    ("C3", "act_heavy", 16384, 4096, 1024),
    ("C4", "relu_3red", 8192, 8192, 2048),
    ("C5 G1", "bias_gelu", 8192, 16384, 4096),
    ("C5 G2", "bias_residual", 8192, 4096, 16384),
]
K_SWEEP: List[Tuple[str, str, int, int, int]] = (
    [(f"bias_gelu K={k}", "bias_gelu", 16384, 4096, k) for k in (2048, 4096)]
    + [(f"bias_residual K={k}", "bias_residual", 16384, 1024, k) for k in (1024, 2048)]
    + [(f"bias_gelu_residual K={k}", "bias_gelu_residual", 16384, 4096, k) for k in (2048, 4096, 8192)]
    + [(f"act_heavy K={k}", "act_heavy", 16384, 4096, k) for k in (2048, 4096, 8192)]
    + [(f"relu_3red K={k}", "relu_3red", 8192, 8192, k) for k in (4096, 8192)]
)
FEW_TILES: List[Tuple[str, str, int, int, int]] = [
    (f"few-tile {m}x{n} K={k}", "bias_gelu", m, n, k)
    for (m, n) in ((1024, 1024), (256, 4096), (512, 4096), (2048, 2048))
    for k in (1024, 2048, 4096, 8192)
]
# The reference presets' few-tile groups: `medium`'s and `stacked_memory_bound`'s
# second GEMMs and `small`'s two.
PRESET_GROUPS: List[Tuple[str, str, int, int, int]] = [
    ("medium G2", "bias_residual", 2048, 1024, 4096),
    ("stacked_memory_bound G2", "bias_residual", 8192, 512, 2048),
    ("small G1", "bias_gelu", 128, 1024, 256),
    ("small G2", "bias_residual", 128, 256, 1024),
]
# Decode-sized M against a wide weight (at least 512 128x128 output tiles):
# both paths stream the weight from HBM once.
DECODE: List[Tuple[str, str, int, int, int]] = [
    ("decode 64x65536 K=4096", "bias_gelu", 64, 65536, 4096),
    ("decode 128x65536 K=4096", "bias_residual", 128, 65536, 4096),
    ("decode 128x65536 K=8192", "bias_gelu", 128, 65536, 8192),
    ("decode 16x65536 K=2048", "bias_gelu", 16, 65536, 2048),
]
GROUPS = CONFIG_GROUPS + K_SWEEP + FEW_TILES + PRESET_GROUPS + DECODE

# (M, D, I) MLP blocks (linear2(gelu(linear1(x))) + x) for the single-kernel
# MLP's rule (``--mlp``): the reference's memory-bound widths over M, and C2.
MLP_SWEEP: List[Tuple[int, int, int]] = (
    [(M, 256, 1024) for M in (2048, 4096, 8192, 16384, 32768, 65536)]
    + [(M, 256, 4096) for M in (4096, 8192, 16384, 32768)]
    + [(M, 512, 2048) for M in (8192, 16384, 32768)]
    + [(16384, 1024, 4096)]
)


def _spec(chain: str):
    from .epilogue import EpilogueSpec, EpiOp

    if chain == "bias_gelu":
        return EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("gelu_erf")), BF), 3
    if chain == "bias_residual":
        return EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("add", 3)), BF), 4
    if chain == "bias_gelu_residual":
        return EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("gelu_erf"), EpiOp("add", 3)), BF), 4
    if chain == "act_heavy":
        return EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("relu"), EpiOp("mul", 3), EpiOp("sigmoid"),
                                   EpiOp("add", 4)), BF), 5
    if chain == "relu_3red":
        return EpilogueSpec(0, 1, (EpiOp("relu"),), BF, store_tile=True, reductions=("sum", "amax", "mean"),
                            reduce_axis=1, reduce_dtypes=(torch.float32,) * 3,
                            outputs=(("tile",), ("red", "sum"), ("red", "amax"), ("red", "mean"))), 2
    raise ValueError(chain)


def _inputs(chain: str, M: int, N: int, K: int, dev) -> List[torch.Tensor]:
    g = torch.Generator().manual_seed(M * 31 + N * 7 + K)
    x = torch.randn(M, K, generator=g).to(BF).to(dev)
    wt = (torch.randn(N, K, generator=g) / K ** 0.5).to(BF).to(dev).t()
    b = (torch.rand(N, generator=g) * 0.1 - 0.05).to(BF).to(dev)
    if chain == "bias_gelu":
        return [b, x, wt]
    if chain in ("bias_residual", "bias_gelu_residual"):
        return [b, x, wt, torch.randn(M, N, generator=g).to(BF).to(dev)]
    if chain == "act_heavy":
        gate = torch.rand(M, N, generator=g).to(BF).to(dev)
        return [b, x, wt, gate, (torch.rand(N, generator=g) * 0.06 - 0.03).to(BF).to(dev)]
    return [x, wt]


def _eager(chain: str) -> Callable:
    if chain == "bias_gelu":
        return lambda b, x, wt: F.gelu(torch.addmm(b, x, wt))
    if chain == "bias_residual":
        return lambda b, x, wt, r: torch.addmm(b, x, wt) + r
    if chain == "bias_gelu_residual":
        return lambda b, x, wt, r: F.gelu(torch.addmm(b, x, wt)) + r
    if chain == "act_heavy":
        return lambda b, x, wt, gate, row: torch.sigmoid(torch.relu(torch.addmm(b, x, wt)) * gate) + row

    def relu_3red(x, wt):
        h = torch.relu(x @ wt)
        return h, h.sum(-1, dtype=torch.float32), h.amax(-1), h.mean(-1, dtype=torch.float32)

    return relu_3red


def _median_ms(fn: Callable[[], object], iters: int) -> float:
    for _ in range(5):
        fn()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for e0, e1 in evs:
        e0.record()
        fn()
        e1.record()
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in evs)


def measure(groups=GROUPS, passes: int = 2, dev: str = "cuda") -> List[Dict[str, object]]:
    from .compiler import epilogue_passes, few_tile_verdict, fused_beats_eager, weight_streaming
    from .launcher import HipKernelLauncher

    rows = []
    for label, chain, M, N, K in groups:
        spec, n_in = _spec(chain)
        ins = _inputs(chain, M, N, K, dev)
        L = HipKernelLauncher(spec, n_in)
        eager = _eager(chain)
        x, wt = ins[spec.left], ins[spec.right]
        fns = {"fused": lambda: L(*ins), "eager": lambda: eager(*ins), "mm": lambda: x @ wt}
        iters = max(20, min(400, int(2e12 / (2.0 * M * N * K) * 40)))
        best = {k: float("inf") for k in fns}
        with torch.no_grad():
            for _ in range(passes):
                for k, f in fns.items():
                    best[k] = min(best[k], _median_ms(f, iters))
        tiles = -(-M // 128) * -(-N // 128)
        addmm = chain != "relu_3red"  # the other chains' GEMM is an addmm (bias in hipBLASLt's epilogue)
        p = epilogue_passes(spec, gemm_is_addmm=addmm)
        few = few_tile_verdict(M, N, K) is not None and not weight_streaming(M, N)
        rule = (not few) and fused_beats_eager(spec, K, dtype=BF, gemm_is_addmm=addmm, M=M, N=N)[0]
        rows.append({"group": label, "chain": chain, "M": M, "N": N, "K": K, "passes": p, "tiles_128": tiles,
                     "fused_ms": round(best["fused"], 4), "eager_ms": round(best["eager"], 4),
                     "mm_ms": round(best["mm"], 4), "fused_over_eager": round(best["fused"] / best["eager"], 3),
                     "rule_fuses": bool(rule)})
        print(f"[calibration] {label}: fused {best['fused']:.4f} eager {best['eager']:.4f} mm {best['mm']:.4f} ms",
              file=sys.stderr, flush=True)
        del L, ins
        torch.cuda.empty_cache()
    return rows


def _reference_ms(fn: Callable[[], object], iters: int) -> float:
    """The reference harness's timing: events around one call, a
    synchronisation after each, median."""
    for _ in range(10):
        fn()
    torch.cuda.synchronize()
    ts = []
    for _ in range(iters):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        fn()
        e1.record()
        torch.cuda.synchronize()
        ts.append(e0.elapsed_time(e1))
    return statistics.median(ts)


def measure_mlp(shapes=MLP_SWEEP, passes: int = 2, dev: str = "cuda") -> List[Dict[str, object]]:
    """Per MLP block shape: the compiled module with two launches (the default
    cost model, no single kernel) and with the single-kernel MLP, timed the
    reference's way; best of alternating passes."""
    from .compiler import FuseMLCompiler
    from .mlp import HipMlpLauncher, mlp_block_beats_two_launches
    from .workloads import TransformerMLP

    rows = []
    for M, D, I in shapes:
        torch.manual_seed(0)
        model = TransformerMLP(D, I).to(dev, BF).eval()
        x = torch.randn(M, D, device=dev, dtype=BF)
        fns = {}
        with torch.no_grad():
            for label, kw in (("two", dict(fuse_mlp_block=False)),
                              ("single", dict(fuse_mlp_block=True, k_per_epilogue_pass=0, min_tiles_long_k=0,
                                              min_output_elements=0))):
                torch._dynamo.reset()
                be = FuseMLCompiler(**kw)
                c = torch.compile(model, backend=be)
                c(x)
                if label == "single" and not any(isinstance(L, HipMlpLauncher) for L in be.launchers):
                    raise RuntimeError(f"M={M} D={D} I={I}: the single-kernel MLP did not bind")
                fns[label] = c
            iters = max(50, min(300, int(3e10 / (4.0 * M * D * I) * 50)))
            best = {k: float("inf") for k in fns}
            for _ in range(passes):
                for k, f in fns.items():
                    best[k] = min(best[k], _reference_ms(lambda: f(x), iters))
        rows.append({"M": M, "D": D, "I": I, "two_ms": round(best["two"], 4), "single_ms": round(best["single"], 4),
                     "single_over_two": round(best["single"] / best["two"], 3),
                     "rule_binds": bool(mlp_block_beats_two_launches(M, D, I)[0])})
        print(f"[calibration] mlp M={M} D={D} I={I}: two {best['two']:.4f} single {best['single']:.4f} ms",
              file=sys.stderr, flush=True)
        del fns, model, x
        torch._dynamo.reset()
        torch.cuda.empty_cache()
    return rows


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--out", default="", help="write the JSON here (default: stdout)")
    ap.add_argument("--passes", type=int, default=2)
    ap.add_argument("--mlp", action="store_true",
                    help="measure the single-kernel MLP against two launches (MLP_SWEEP) instead of the GEMM groups")
    args = ap.parse_args(argv)
    if not torch.cuda.is_available():
        print("calibration needs a GPU", file=sys.stderr)
        return 2
    t0 = time.perf_counter()
    if args.mlp:
        rows = measure_mlp(passes=args.passes)
        method = ("compiled TransformerMLP (bf16), events around one forward and a synchronisation after each "
                  "(the reference harness's method), median, best of alternating passes; two = default cost model "
                  "without the single kernel, single = the single-kernel MLP bound")
    else:
        rows = measure(passes=args.passes)
        method = "median HIP-event time per call, best of alternating passes; same inputs for all three paths"
    arch = getattr(torch.cuda.get_device_properties(0), "gcnArchName", "")
    doc = {"device": arch, "cus": torch.cuda.get_device_properties(0).multi_processor_count,
           "seconds": round(time.perf_counter() - t0, 1), "method": method, "rows": rows}
    text = json.dumps(doc, indent=1)
    if args.out:
        with open(args.out, "w") as f:
            f.write(text + "\n")
    else:
        print(text)
    return 0


if __name__ == "__main__":
    sys.exit(main())
