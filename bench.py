"""Benchmark of the fused MLP-block hot path on one MI355X.

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--workload C2|C3|C4|C5]

A step is one forward of the workload through the fused HIP kernels (for the
default C2 MLP block: GEMM1+bias+GELU and GEMM2+bias+residual, two launches of
the gfx950 kernel family through the C ABI), on synthetic seeded inputs that are
resident in HBM before timing starts.  W untimed steps, then K timed steps
bracketed by ``torch.cuda.synchronize()``.  Rank 0 prints one JSON line:

* ``value``/``ms_per_step`` — fused block latency in ms (lower is better);
* ``roofline`` — the dominant kernel's algorithmic FLOPs per launch divided by
  its average launch duration, measured with HIP events on the launch stream
  inside the timed region, against the bf16 dense MFMA peak (every config is
  MFMA-bound on MI355X: arithmetic intensity 443-2184 FLOP/B vs a ridge of
  ~315 FLOP/B);
* ``eager_ms`` / ``speedup_vs_eager`` — the same module run by PyTorch eager on
  the same GPU (hipBLASLt GEMMs + elementwise kernels);
* ``cpu_baseline`` — the CPU oracle (numpy float32, ``oracle/workloads.py``)
  timed on this host on a bounded row sample and scaled to the full batch
  (reported, not a target).

One GPU only: ``--gpus`` above 1 exits with an explanation.
"""

from __future__ import annotations

import argparse
import json
import os
import sys
import time

REPO = os.path.dirname(os.path.abspath(__file__))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

import torch  # noqa: E402

MFMA_BF16_PEAK_TFLOPS = 2500.0  # MI355X dense bf16
HBM_PEAK_GBS = 8000.0

WORKLOAD_DESC = {
    "C2": "MLP block memory_bound bf16: x[16384,1024] -> addmm(1024->4096)+b1 -> GELU -> addmm(4096->1024)+b2 + residual x",
    "C3": "Activation-heavy bf16: x[16384,1024] -> addmm(1024->4096)+b -> ReLU -> *g[16384,4096] -> Sigmoid -> +row[4096]",
    "C4": "GEMM + fused row reductions bf16: x[8192,2048] @ W[8192,2048]^T -> ReLU -> tile + row sum/amax/mean fp32",
    "C5": "Stacked MLP x4 bf16: x[8192,4096], 4 x (addmm(4096->16384)+GELU -> addmm(16384->4096)+b2+residual)",
}


def _parse():
    p = argparse.ArgumentParser()
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=50)
    p.add_argument("--warmup", type=int, default=10)
    p.add_argument("--workload", default="C2", choices=sorted(WORKLOAD_DESC))
    p.add_argument("--no-cpu", action="store_true", help="skip the CPU oracle baseline")
    p.add_argument("--no-eager", action="store_true", help="skip the eager GPU comparison")
    p.add_argument("--eager-only", action="store_true",
                   help="run only the eager leg and print its call count (rocprof counter runs of the eager module)")
    p.add_argument("--cpu-seconds", type=float, default=12.0)
    p.add_argument("--calib-copy-mb", type=int, default=0,
                   help="after timing, run device copies of this size (rocprof counter calibration)")
    return p.parse_args()


# ---------------------------------------------------------------------------
# Fused pipelines: one list of (launcher, arg-builder) per workload
# ---------------------------------------------------------------------------


def _build_pipeline(name: str, wl, dev):
    from fuseml_amd.epilogue import EpilogueSpec, EpiOp
    from fuseml_amd.launcher import HipKernelLauncher

    dt = wl.dtype
    m = wl.model
    stages = []  # (label, launcher, fn(state)->args, gemm (M,N,K))

    def mlp_block(prefix, blk, gemms):
        g1 = HipKernelLauncher(EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("gelu_erf")), dt), 3)
        g2 = HipKernelLauncher(EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("add", 3)), dt), 4)
        w1t, b1 = blk.linear1.weight.t(), blk.linear1.bias
        w2t, b2 = blk.linear2.weight.t(), blk.linear2.bias
        stages.append((f"{prefix}G1 addmm+bias+gelu", g1, lambda s: (b1, s["x"], w1t), "h", gemms[0]))
        stages.append((f"{prefix}G2 addmm+bias+residual", g2, lambda s: (b2, s["h"], w2t, s["x"]), "x", gemms[1]))

    if name == "C2":
        mlp_block("", m, wl.gemms)
    elif name == "C5":
        for i, blk in enumerate(m.blocks):
            mlp_block(f"B{i} ", blk, wl.gemms[2 * i: 2 * i + 2])
    elif name == "C3":
        lin = m.linear
        spec = EpilogueSpec(1, 2, (EpiOp("add", 0), EpiOp("relu"), EpiOp("mul", 3), EpiOp("sigmoid"), EpiOp("add", 4)), dt)
        g = HipKernelLauncher(spec, 5)
        stages.append(("addmm+bias+relu*g+sigmoid+row", g,
                       lambda s: (lin.bias, s["x"], lin.weight.t(), s["g"], m.row), "y", wl.gemms[0]))
    elif name == "C4":
        # the spec FuseMLCompiler(fuse_sibling_reductions=True) derives for this module
        spec = EpilogueSpec(0, 1, (EpiOp("relu"),), dt, store_tile=True,
                            reductions=("sum", "amax", "mean"), reduce_axis=1,
                            reduce_dtypes=(torch.float32,) * 3,
                            outputs=(("red", "sum"), ("red", "amax"), ("red", "mean"), ("tile",)))
        g = HipKernelLauncher(spec, 2)
        wt = m.linear.weight.t()
        stages.append(("mm+relu+rowsum/amax/mean", g, lambda s: (s["x"], wt), "y", wl.gemms[0]))
    return stages


def _run_pipeline(stages, state, events=None, io=None):
    for i, (_, launcher, args, out_key, _) in enumerate(stages):
        if events is not None:
            events[i][0].record()
        a = args(state)
        out = launcher(*a)
        if events is not None:
            events[i][1].record()
        if io is not None:
            io.append((a, out))
        state[out_key] = out
    return state


def _algorithmic_bytes(args, out):
    """HBM bytes a launch must move at least: every distinct input tensor read
    once (a [K,N] weight view counts its K*N elements) and every output written
    once."""
    seen, total = set(), 0
    outs = out if isinstance(out, (tuple, list)) else (out,)
    for t in list(args) + list(outs):
        if isinstance(t, torch.Tensor) and (t.data_ptr(), t.numel()) not in seen:
            seen.add((t.data_ptr(), t.numel()))
            total += t.numel() * t.element_size()
    return total


def _initial_state(name, wl):
    st = {"x": wl.inputs[0]}
    if name == "C3":
        st["g"] = wl.inputs[1]
    return st


# ---------------------------------------------------------------------------
# HBM traffic per launch, from the committed rocprofv3 counter summary
# ---------------------------------------------------------------------------

TRAFFIC_SUMMARY = os.path.join(REPO, "profiles", "traffic_{workload}.md")


def _traffic(workload, launch):
    """Bytes per launch of the step's launch number `launch` (issue order within
    a step, as `python -m fuseml_amd.profiling traffic --per-step N` numbers
    them), or None."""
    data = _json_block(TRAFFIC_SUMMARY.format(workload=workload))
    if data is None:
        return None
    for k in data.get("kernels", []):
        if (str(k.get("kernel", "")).startswith("gemm_epilogue_kernel") and k.get("launch") == launch
                and k.get("fetch_bytes") is not None and k.get("write_bytes") is not None):
            return int(k["fetch_bytes"] + k["write_bytes"])
    return None


EAGER_TRAFFIC_SUMMARY = os.path.join(REPO, "profiles", "traffic_eager_{workload}.md")


def _json_block(path):
    if not os.path.exists(path):
        return None
    text = open(path).read()
    if "```json" not in text:
        return None
    return json.loads(text.split("```json", 1)[1].split("```", 1)[0])


def _hbm_traffic(workload, gemms):
    """Fused step against the eager module, both from committed counter summaries.

    Final-output bytes are what any implementation must write (the last GEMM's
    bf16 tile, plus C4's three fp32 reduction vectors); written bytes beyond
    them are intermediates.  Each intermediate is written once and read back at
    least once, so the share of intermediate writes removed is the share of
    intermediate traffic removed."""
    fused, eager = _json_block(TRAFFIC_SUMMARY.format(workload=workload)), _json_block(
        EAGER_TRAFFIC_SUMMARY.format(workload=workload))
    if fused is None or eager is None:
        return None
    gemm_entries = [k for k in fused["kernels"] if str(k["kernel"]).startswith("gemm_epilogue_kernel")]
    if not gemm_entries or any(k.get("fetch_bytes") is None or k.get("write_bytes") is None
                               for k in fused["kernels"]):
        return None
    # the summaries number a step's launches modulo their count of distinct shapes
    reps = len(gemms) / len(gemm_entries)
    f_fetch = f_write = 0.0
    for k in fused["kernels"]:
        r = reps if k in gemm_entries else 1.0
        f_fetch += k["fetch_bytes"] * r
        f_write += k["write_bytes"] * r
    M, N, _ = gemms[-1]
    out_bytes = M * N * 2 + (3 * M * 4 if workload == "C4" else 0)
    e_fetch, e_write = eager["fetch_bytes_per_call"], eager["write_bytes_per_call"]
    e_int, f_int = e_write - out_bytes, max(f_write - out_bytes, 0.0)
    return {
        "eager_bytes": int(e_fetch + e_write),
        "fused_bytes": int(f_fetch + f_write),
        "saved_frac": round(1.0 - (f_fetch + f_write) / (e_fetch + e_write), 4),
        "eager_write_bytes": int(e_write),
        "fused_write_bytes": int(f_write),
        "final_output_bytes": int(out_bytes),
        "intermediate_eliminated_frac": round(1.0 - f_int / e_int, 4) if e_int > 0 else None,
        "source": f"profiles/traffic_{workload}.md, profiles/traffic_eager_{workload}.md",
    }


# ---------------------------------------------------------------------------
# CPU oracle baseline (bounded sample, scaled to the full batch)
# ---------------------------------------------------------------------------


def _cpu_baseline(name, wl, seconds):
    import numpy as np
    from threadpoolctl import threadpool_info, threadpool_limits

    from oracle import workloads as ora_w

    cores = len(os.sched_getaffinity(0))
    f32 = lambda t: t.detach().float().cpu().numpy()  # noqa: E731
    m = wl.model
    x = f32(wl.inputs[0])
    M = x.shape[0]
    rows = np.arange(min(M, 256))
    if name in ("C2",):
        args = (f32(m.linear1.weight), f32(m.linear1.bias), f32(m.linear2.weight), f32(m.linear2.bias))
        fn = lambda: ora_w.transformer_mlp(x, *args, rows=rows, dtype=np.float32)  # noqa: E731
    elif name == "C3":
        g = f32(wl.inputs[1])
        args = (f32(m.linear.weight), f32(m.linear.bias), g, f32(m.row))
        fn = lambda: ora_w.activation_heavy(x, *args, rows=rows, dtype=np.float32)  # noqa: E731
    elif name == "C4":
        w = f32(m.linear.weight)
        fn = lambda: ora_w.gemm_row_reductions(x, w, rows=rows, dtype=np.float32)  # noqa: E731
    else:
        blocks = [(f32(b.linear1.weight), f32(b.linear1.bias), f32(b.linear2.weight), f32(b.linear2.bias))
                  for b in m.blocks]
        rows = np.arange(min(M, 64))
        fn = lambda: ora_w.stacked_mlp(x, blocks, rows=rows, dtype=np.float32)  # noqa: E731
    with threadpool_limits(limits=cores):
        threads = max((i.get("num_threads", 1) for i in threadpool_info()), default=1)
        fn()  # warm-up
        t0 = time.perf_counter()
        reps = 0
        while True:
            fn()
            reps += 1
            if time.perf_counter() - t0 >= seconds:
                break
        dt = (time.perf_counter() - t0) / reps
    ms_full = dt * 1e3 * (M / len(rows))
    return {
        "value": round(ms_full, 3),
        "unit": "ms per full-batch forward (extrapolated from a row sample)",
        "cores": int(threads),
        "kind": "port",
        "sample": f"oracle/workloads.py numpy float32 forward of {len(rows)} of {M} rows, "
                  f"{reps} repetitions in {dt * reps:.1f} s, scaled by {M / len(rows):.0f}",
    }


# ---------------------------------------------------------------------------


def _calib_copy(mb, dev):
    """Device copies of `mb` MiB, the known-size reference for the rocprof
    FETCH_SIZE / WRITE_SIZE scale factors."""
    if mb <= 0:
        return
    src = torch.empty(mb * 1024 * 1024, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    torch.cuda.synchronize()
    del src, dst


def _run_eager(wl, warmup, steps):
    """The workload's module under PyTorch eager: (forward calls made, ms per timed call)."""
    with torch.no_grad():
        n_warm = max(3, warmup)
        for _ in range(n_warm):
            wl.model(*wl.inputs)
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for _ in range(steps):
            wl.model(*wl.inputs)
        torch.cuda.synchronize()
    return n_warm + steps, (time.perf_counter() - t0) * 1e3 / steps


def main():
    args = _parse()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build runs the fused kernels on a single MI355X "
              "(rows shard across GPUs with no exchange, so N GPUs run N independent copies). "
              "Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(2)

    from fuseml_amd.workloads import WORKLOADS

    name = args.workload
    dev = torch.device("cuda:0")
    wl = WORKLOADS[name]()
    wl.to(dev)
    torch.backends.cuda.matmul.allow_tf32 = False

    if args.eager_only:
        _calib_copy(args.calib_copy_mb, dev)
        calls, eager_ms = _run_eager(wl, args.warmup, args.steps)
        print(json.dumps({"workload": name, "eager_ms": round(eager_ms, 4), "eager_calls": calls}), flush=True)
        return

    stages = _build_pipeline(name, wl, dev)
    with torch.no_grad():
        state = _initial_state(name, wl)
        for _ in range(args.warmup):
            _run_pipeline(stages, dict(state))
        torch.cuda.synchronize()

        events = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True))
                   for _ in stages] for _ in range(args.steps)]
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        for k in range(args.steps):
            ev = [events[k][i] for i in range(len(stages))]
            _run_pipeline(stages, dict(state), ev)
        torch.cuda.synchronize()
        wall = time.perf_counter() - t0
    ms_per_step = wall * 1e3 / args.steps

    per_kernel = []
    for i, (label, _, _, _, gemm) in enumerate(stages):
        durs = [events[k][i][0].elapsed_time(events[k][i][1]) for k in range(args.steps)]
        avg = sum(durs) / len(durs)
        Mg, Ng, Kg = gemm
        flops = 2.0 * Mg * Ng * Kg
        per_kernel.append({"kernel": label, "avg_ms": round(avg, 4), "gemm_MNK": [Mg, Ng, Kg],
                           "tflops": round(flops / (avg * 1e-3) / 1e12, 1)})
    # one more (untimed) pass to read each launch's operands and outputs
    io = []
    with torch.no_grad():
        _run_pipeline(stages, dict(state), io=io)
    torch.cuda.synchronize()
    for pk, (a, out) in zip(per_kernel, io):
        pk["algorithmic_bytes"] = _algorithmic_bytes(a, out)
        pk["GBps"] = round(pk["algorithmic_bytes"] / (pk["avg_ms"] * 1e-3) / 1e9, 1)
    dom = max(range(len(per_kernel)), key=lambda i: per_kernel[i]["avg_ms"])
    dk = per_kernel[dom]
    Mg, Ng, Kg = dk["gemm_MNK"]
    achieved = 2.0 * Mg * Ng * Kg / (dk["avg_ms"] * 1e-3) / 1e12

    _calib_copy(args.calib_copy_mb, dev)

    eager_ms = None
    if not args.no_eager:
        _, eager_ms = _run_eager(wl, args.warmup, args.steps)

    cpu = None
    if not args.no_cpu:
        cpu = _cpu_baseline(name, wl, args.cpu_seconds)

    line = {
        "metric": "fused MLP-block latency (ms), % HBM/MFMA roofline, speedup vs eager",
        "value": round(ms_per_step, 4),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded torch.Generator inputs, random-init nn.Linear weights)",
        "config": {"workload": f"{name}: {WORKLOAD_DESC[name]}", "gemms_MNK": wl.gemms,
                   "parallelism": "single GPU"},
        "tflops_per_step": round(wl.flops / (ms_per_step * 1e-3) / 1e12, 1),
        "eager_ms": None if eager_ms is None else round(eager_ms, 4),
        "speedup_vs_eager": None if eager_ms is None else round(eager_ms / ms_per_step, 3),
        "kernels": per_kernel,
        "roofline": {
            "bound": "mfma",
            "kernel": dk["kernel"],
            "achieved": round(achieved, 1),
            "peak": MFMA_BF16_PEAK_TFLOPS,
            "unit": "TFLOP/s",
            "frac": round(achieved / MFMA_BF16_PEAK_TFLOPS, 4),
            "traffic": _traffic(name, dom),
        },
        # the same dominant kernel against the HBM roofline: algorithmic bytes
        # (inputs and outputs once) over its event-timed duration
        "hbm_roofline": {"kernel": dk["kernel"], "algorithmic_bytes": dk["algorithmic_bytes"],
                         "achieved": dk["GBps"], "peak": HBM_PEAK_GBS, "unit": "GB/s",
                         "frac": round(dk["GBps"] / HBM_PEAK_GBS, 4)},
        "hbm_traffic": _hbm_traffic(name, wl.gemms),
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
