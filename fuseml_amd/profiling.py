"""Summaries of rocprofv3 output for the fused kernels.

    python -m fuseml_amd.profiling trace <kernel_trace.csv> [--per-step N]
    python -m fuseml_amd.profiling traffic <fetch counter_collection.csv> <write counter_collection.csv> \
        --copy-mib 512 [--per-step N]

``trace`` groups dispatches by (kernel, grid size, launch) and prints call
count and average / min / max duration.  The GEMMs of one step are often the
same template at the same grid (the 256-wide variants launch one workgroup per
CU whatever the tile count), so ``--per-step N`` (N launches of the kernel per
step, as ``bench.py`` prints in ``config.gemms_MNK``) numbers a kernel's
dispatches in issue order and groups dispatch i as launch i % N.

``traffic`` turns the per-dispatch ``FETCH_SIZE`` and ``WRITE_SIZE`` counters
(KiB) into bytes per launch.  The counters are scaled by what they read for a
device-to-device copy of known size run in the same process
(``bench.py --calib-copy-mb``): factor = copy bytes / counter bytes.

``mfma-busy`` turns one counter pass of ``SQ_VALU_MFMA_BUSY_CYCLES`` and
``GRBM_GUI_ACTIVE`` into the MFMA-busy fraction of each launch: the ratio of
the two counters, divided by the same ratio read for the MFMA-only probe
(``fuseml_mfma_peak_probe``, which ``bench.py`` runs in the same process and
which keeps every SIMD's MFMA pipe busy), so the normalisation (counter
aggregation over XCDs, CUs and SIMDs) cancels.  It also reports each launch's
clock, GRBM_GUI_ACTIVE per XCD over the traced duration when a kernel trace
of the same run is given.

``counters`` averages every counter of one ``--pmc`` pass per launch, also per
wave of the dispatch (instruction counts, LDS bank conflicts, active cycles).

``step-traffic`` sums the same counters over every dispatch of a run (the
calibration copy aside) and divides by ``--calls``, the number of times the
run called the module (``bench.py --eager-only`` prints it): HBM bytes per
call of the eager module, whatever kernels the library picks.
"""

from __future__ import annotations

import argparse
import csv
import json
import re
import statistics
import sys
from collections import defaultdict
from typing import Dict, List, Tuple

COPY_KERNEL_HINT = "copyBuffer"
PROBE_KERNEL_HINT = "mfma_peak_kernel"


def _short(name: str) -> str:
    """gemm_epilogue_kernel<BM,BN,BK,S,WM,WN,SCHED,dtype[,red][,chN]> from the
    mangled name (",red": the instantiation that carries the reductions;
    ",chN": fixed epilogue chain N, absent for the generic op loop, chain 0)."""
    m = re.search(r"gemm_epilogue_kernelI((?:Li\d+E)+)(DF16b|DF16_)(?:Lb([01])E)?(?:Li(\d+)E)?E", name)
    if m:
        ints = ",".join(re.findall(r"Li(\d+)E", m.group(1)))
        dtype = {"DF16b": "bf16", "DF16_": "f16"}[m.group(2)]
        ch = f",ch{m.group(4)}" if m.group(4) not in (None, "0") else ""
        return f"gemm_epilogue_kernel<{ints},{dtype}{',red' if m.group(3) == '1' else ''}{ch}>"
    # Demangled by the profiler: "void ns::gemm_epilogue_kernel<256, 256, ..., __bf16, true, 3>(...)".
    # rocprofv3 demangles some instantiations with a garbled type tail (the
    # __bf16 mangling); then only the seven tile integers are kept.
    m = re.search(r"gemm_epilogue_kernel<((?:\d+, ){6}\d+), ([^()]*)>\(", name)
    if m:
        ints = m.group(1).replace(" ", "")
        tail = [t.strip() for t in m.group(2).split(",")]
        dtype = {"__bf16": "bf16", "_Float16": "f16"}.get(tail[0]) if tail else None
        if dtype is None or len(tail) not in (2, 3) or tail[1] not in ("true", "false") or \
                (len(tail) == 3 and not tail[2].isdigit()):
            return f"gemm_epilogue_kernel<{ints},...>"
        ch = f",ch{tail[2]}" if len(tail) == 3 and tail[2] != "0" else ""
        return f"gemm_epilogue_kernel<{ints},{dtype}{',red' if tail[1] == 'true' else ''}{ch}>"
    return name[:60]


def _launch_positions(rows: List[Dict[str, str]], per_step: int) -> List[int]:
    """Position (dispatch index mod per_step) of each row among the fused
    kernel's dispatches in issue order (Dispatch_Id); 0 for other kernels."""
    order = sorted((int(r.get("Dispatch_Id") or 0), i) for i, r in enumerate(rows)
                   if "gemm_epilogue_kernel" in r["Kernel_Name"])
    pos = [0] * len(rows)
    for n, (_, i) in enumerate(order):
        pos[i] = n % max(per_step, 1)
    return pos


def trace_summary(path: str, per_step: int = 1) -> List[Dict[str, object]]:
    rows = list(csv.DictReader(open(path)))
    pos = _launch_positions(rows, per_step)
    groups: Dict[Tuple[str, int, int], List[float]] = defaultdict(list)
    for r, p in zip(rows, pos):
        grid = int(r.get("Grid_Size_X") or r.get("Grid_Size") or 0)
        dur = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3  # us
        groups[(r["Kernel_Name"], grid, p)].append(dur)
    out = []
    for (name, grid, p), durs in sorted(groups.items(), key=lambda kv: (kv[0][0], kv[0][2], -sum(kv[1]))):
        out.append({"kernel": _short(name), "grid": grid, "launch": p, "calls": len(durs),
                    "avg_us": round(statistics.mean(durs), 2), "min_us": round(min(durs), 2),
                    "max_us": round(max(durs), 2)})
    return out


def counter_by_dispatch(path: str, counter: str, per_step: int = 1) -> Dict[Tuple[str, int, int], List[float]]:
    rows = [r for r in csv.DictReader(open(path)) if r["Counter_Name"] == counter]
    pos = _launch_positions(rows, per_step)
    acc: Dict[Tuple[str, int, int], List[float]] = defaultdict(list)
    for r, p in zip(rows, pos):
        acc[(r["Kernel_Name"], int(r.get("Grid_Size") or r.get("Grid_Size_X") or 0), p)].append(
            float(r["Counter_Value"]))
    return acc


def _copy_factor(table: Dict[Tuple[str, int, int], List[float]], copy_bytes: float):
    """copy bytes / counter bytes read for the calibration copy, or None."""
    vals = [v for (n, _, _), vs in table.items() if COPY_KERNEL_HINT in n for v in vs]
    # FETCH_SIZE reads a device copy at about half its bytes: keep every dispatch
    # of at least a quarter of the copy size.
    big = [v for v in vals if v * 1024 >= 0.25 * copy_bytes]
    if not big:
        return None
    return copy_bytes / (statistics.median(big) * 1024)


def traffic_summary(fetch_csv: str, write_csv: str, copy_mib: float, per_step: int = 1) -> Dict[str, object]:
    fetch = counter_by_dispatch(fetch_csv, "FETCH_SIZE", per_step)
    write = counter_by_dispatch(write_csv, "WRITE_SIZE", per_step)
    copy_bytes = copy_mib * 1024 * 1024
    ff, wf = _copy_factor(fetch, copy_bytes), _copy_factor(write, copy_bytes)
    kernels = []
    for key in sorted(set(fetch) | set(write)):
        name, grid, p = key
        if COPY_KERNEL_HINT in name:
            continue
        f = statistics.mean(fetch.get(key, [0.0])) * 1024
        w = statistics.mean(write.get(key, [0.0])) * 1024
        kernels.append({
            "kernel": _short(name), "grid": grid, "launch": p,
            "fetch_bytes_raw": f, "write_bytes_raw": w,
            "fetch_bytes": None if ff is None else f * ff,
            "write_bytes": None if wf is None else w * wf,
        })
    return {"copy_mib": copy_mib, "fetch_factor": ff, "write_factor": wf, "kernels": kernels}


def mfma_busy_summary(pmc_csv: str, per_step: int = 1, xcds: int = 8) -> Dict[str, object]:
    busy = counter_by_dispatch(pmc_csv, "SQ_VALU_MFMA_BUSY_CYCLES", per_step)
    gui = counter_by_dispatch(pmc_csv, "GRBM_GUI_ACTIVE", per_step)
    ratio = {k: statistics.mean(busy[k]) / statistics.mean(gui[k]) for k in busy if k in gui and
             statistics.mean(gui[k]) > 0}
    probe = [r for (n, _, _), r in ratio.items() if PROBE_KERNEL_HINT in n]
    ref = statistics.median(probe) if probe else None
    kernels = []
    for key in sorted(ratio):
        name, grid, p = key
        if COPY_KERNEL_HINT in name:
            continue
        kernels.append({
            "kernel": "mfma_peak_kernel (probe)" if PROBE_KERNEL_HINT in name else _short(name),
            "grid": grid, "launch": p, "dispatches": len(busy[key]),
            "mfma_busy_cycles": statistics.mean(busy[key]), "grbm_gui_active": statistics.mean(gui[key]),
            "gui_active_per_xcd": statistics.mean(gui[key]) / xcds,
            "mfma_busy_frac": None if ref is None else round(ratio[key] / ref, 4),
        })
    return {"probe_ratio": ref, "kernels": kernels}


def counter_summary(pmc_csv: str, per_step: int = 1) -> Dict[str, object]:
    """Mean of every counter of one ``--pmc`` pass per (kernel, launch), and
    per wave of the dispatch (grid / 64): e.g. VALU and LDS instruction counts,
    LDS bank-conflict cycles, active-VALU cycles of the fused kernels."""
    rows = list(csv.DictReader(open(pmc_csv)))
    names = sorted({r["Counter_Name"] for r in rows})
    out: Dict[Tuple[str, int, int], Dict[str, object]] = {}
    for c in names:
        for key, vals in counter_by_dispatch(pmc_csv, c, per_step).items():
            name, grid, p = key
            if COPY_KERNEL_HINT in name:
                continue
            e = out.setdefault(key, {"kernel": "mfma_peak_kernel (probe)" if PROBE_KERNEL_HINT in name else _short(name),
                                     "grid": grid, "launch": p, "dispatches": len(vals), "counters": {},
                                     "per_wave": {}})
            e["counters"][c] = statistics.mean(vals)
            if grid:
                e["per_wave"][c] = round(statistics.mean(vals) / (grid / 64), 1)
    return {"counters": names, "kernels": [out[k] for k in sorted(out)]}


def step_traffic(fetch_csv: str, write_csv: str, copy_mib: float, calls: int) -> Dict[str, object]:
    """HBM bytes per call of a whole module (every dispatch but the calibration
    copy), for a run that called the module ``calls`` times: totals over the
    kernels dispatched at least once per call, scaled by the copy factors,
    divided by ``calls``.  Used for the
    eager leg, whose kernels (library GEMMs, elementwise ops) vary in name and
    count from one torch build to the next."""
    fetch = counter_by_dispatch(fetch_csv, "FETCH_SIZE")
    write = counter_by_dispatch(write_csv, "WRITE_SIZE")
    copy_bytes = copy_mib * 1024 * 1024
    ff, wf = _copy_factor(fetch, copy_bytes), _copy_factor(write, copy_bytes)
    kernels = []
    for key in sorted(set(fetch) | set(write)):
        name, grid, _ = key
        if COPY_KERNEL_HINT in name:
            continue
        f, w = fetch.get(key, []), write.get(key, [])
        kernels.append({
            "kernel": _short(name), "grid": grid, "dispatches": max(len(f), len(w)),
            "fetch_bytes_per_call": None if ff is None else sum(f) * 1024 * ff / calls,
            "write_bytes_per_call": None if wf is None else sum(w) * 1024 * wf / calls,
        })
    # A kernel dispatched fewer times than the module was called is one-off work
    # (library workspace fills, first-call set-up), not part of a call.
    per_call = [x for x in kernels if x["dispatches"] >= calls]
    tot = lambda k: None if any(x[k] is None for x in per_call) else sum(x[k] for x in per_call)  # noqa: E731
    for x in kernels:
        x["per_call"] = x["dispatches"] >= calls
    return {"copy_mib": copy_mib, "fetch_factor": ff, "write_factor": wf, "calls": calls,
            "fetch_bytes_per_call": tot("fetch_bytes_per_call"),
            "write_bytes_per_call": tot("write_bytes_per_call"), "kernels": kernels}


def main(argv=None) -> int:
    ap = argparse.ArgumentParser()
    sub = ap.add_subparsers(dest="cmd", required=True)
    t = sub.add_parser("trace")
    t.add_argument("csv")
    t.add_argument("--per-step", type=int, default=1)
    tr = sub.add_parser("traffic")
    tr.add_argument("fetch_csv")
    tr.add_argument("write_csv")
    tr.add_argument("--copy-mib", type=float, required=True)
    tr.add_argument("--per-step", type=int, default=1)
    mb = sub.add_parser("mfma-busy")
    mb.add_argument("csv")
    mb.add_argument("--per-step", type=int, default=1)
    cs = sub.add_parser("counters")
    cs.add_argument("csv")
    cs.add_argument("--per-step", type=int, default=1)
    st = sub.add_parser("step-traffic")
    st.add_argument("fetch_csv")
    st.add_argument("write_csv")
    st.add_argument("--copy-mib", type=float, required=True)
    st.add_argument("--calls", type=int, required=True)
    a = ap.parse_args(argv)
    if a.cmd == "trace":
        for row in trace_summary(a.csv, a.per_step):
            print(json.dumps(row))
    elif a.cmd == "traffic":
        print(json.dumps(traffic_summary(a.fetch_csv, a.write_csv, a.copy_mib, a.per_step), indent=1))
    elif a.cmd == "mfma-busy":
        print(json.dumps(mfma_busy_summary(a.csv, a.per_step), indent=1))
    elif a.cmd == "counters":
        print(json.dumps(counter_summary(a.csv, a.per_step), indent=1))
    else:
        print(json.dumps(step_traffic(a.fetch_csv, a.write_csv, a.copy_mib, a.calls), indent=1))
    return 0


if __name__ == "__main__":
    sys.exit(main())
