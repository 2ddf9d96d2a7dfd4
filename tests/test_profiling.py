"""The rocprofv3 summaries used for the committed profiles (CPU only)."""

import csv

from fuseml_amd.profiling import step_traffic, trace_summary, traffic_summary

GEMM = "_ZN12_GLOBAL__N_120gemm_epilogue_kernelILi256ELi256ELi32ELi4ELi2ELi4ELi1EDF16bEEv16fuseml_gemm_desc"
COPY = "__amd_rocclr_copyBuffer"


def _write(path, fields, rows):
    with open(path, "w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=fields)
        w.writeheader()
        w.writerows(rows)


def test_trace_launches_grouped_by_position(tmp_path):
    # Three steps of two launches at the same grid (G1 100 us, G2 50 us), with
    # another kernel in between; rows out of dispatch order.
    rows = []
    did = 0
    for step in range(3):
        for pos, dur in ((0, 100_000), (1, 50_000)):
            did += 1
            rows.append({"Dispatch_Id": did, "Kernel_Name": GEMM, "Grid_Size_X": 131072,
                         "Start_Timestamp": 1000 * did, "End_Timestamp": 1000 * did + dur + step})
            did += 1
            rows.append({"Dispatch_Id": did, "Kernel_Name": "other", "Grid_Size_X": 64,
                         "Start_Timestamp": 1000 * did, "End_Timestamp": 1000 * did + 7000})
    rows.reverse()
    p = tmp_path / "t_kernel_trace.csv"
    _write(p, ["Dispatch_Id", "Kernel_Name", "Grid_Size_X", "Start_Timestamp", "End_Timestamp"], rows)

    merged = [r for r in trace_summary(str(p)) if r["kernel"].startswith("gemm_epilogue_kernel")]
    assert len(merged) == 1 and merged[0]["calls"] == 6

    split = {r["launch"]: r for r in trace_summary(str(p), per_step=2)
             if r["kernel"] == "gemm_epilogue_kernel<256,256,32,4,2,4,1,bf16>"}
    assert sorted(split) == [0, 1]
    assert split[0]["calls"] == 3 and split[0]["avg_us"] == 100.0 and split[0]["max_us"] == 100.0
    assert split[1]["calls"] == 3 and split[1]["avg_us"] == 50.0 and split[1]["min_us"] == 50.0


def test_traffic_scaled_by_copy_and_split_by_launch(tmp_path):
    fields = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    # Copy of 512 MiB read as 409.6 MiB by the counter: factor 1.25.
    copy_kib = 512 * 1024 / 1.25
    fetch = [{"Dispatch_Id": 1, "Kernel_Name": COPY, "Grid_Size": 512, "Counter_Name": "FETCH_SIZE",
              "Counter_Value": copy_kib}]
    write = [{"Dispatch_Id": 1, "Kernel_Name": COPY, "Grid_Size": 512, "Counter_Name": "WRITE_SIZE",
              "Counter_Value": copy_kib}]
    for i, (f, w) in enumerate([(10.0, 1.0), (20.0, 2.0)] * 2):
        fetch.append({"Dispatch_Id": 2 + i, "Kernel_Name": GEMM, "Grid_Size": 131072,
                      "Counter_Name": "FETCH_SIZE", "Counter_Value": f})
        write.append({"Dispatch_Id": 2 + i, "Kernel_Name": GEMM, "Grid_Size": 131072,
                      "Counter_Name": "WRITE_SIZE", "Counter_Value": w})
    pf, pw = tmp_path / "f.csv", tmp_path / "w.csv"
    _write(pf, fields, fetch)
    _write(pw, fields, write)
    t = traffic_summary(str(pf), str(pw), 512, per_step=2)
    assert abs(t["fetch_factor"] - 1.25) < 1e-12 and abs(t["write_factor"] - 1.25) < 1e-12
    k = {r["launch"]: r for r in t["kernels"]}
    assert abs(k[0]["fetch_bytes"] - 10.0 * 1024 * 1.25) < 1e-6 and abs(k[0]["write_bytes"] - 1.0 * 1024 * 1.25) < 1e-6
    assert abs(k[1]["fetch_bytes"] - 20.0 * 1024 * 1.25) < 1e-6 and abs(k[1]["write_bytes"] - 2.0 * 1024 * 1.25) < 1e-6


def test_step_traffic_totals_every_kernel_per_call(tmp_path):
    fields = ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"]
    copy_kib = 512 * 1024 / 2.0  # factor 2
    rows = {"FETCH_SIZE": [], "WRITE_SIZE": []}
    for c in rows:
        rows[c].append({"Dispatch_Id": 1, "Kernel_Name": COPY, "Grid_Size": 512, "Counter_Name": c,
                        "Counter_Value": copy_kib})
    # three calls of a module with two kernels of different names (one launched twice per call)
    d = 2
    for _ in range(3):
        for name, grid, f, w in [("Cijk_gemm", 1024, 100.0, 10.0), ("elementwise", 4096, 7.0, 7.0),
                                 ("Cijk_gemm", 1024, 50.0, 5.0)]:
            rows["FETCH_SIZE"].append({"Dispatch_Id": d, "Kernel_Name": name, "Grid_Size": grid,
                                       "Counter_Name": "FETCH_SIZE", "Counter_Value": f})
            rows["WRITE_SIZE"].append({"Dispatch_Id": d, "Kernel_Name": name, "Grid_Size": grid,
                                       "Counter_Name": "WRITE_SIZE", "Counter_Value": w})
            d += 1
    # a one-off fill (fewer dispatches than calls) stays out of the per-call totals
    for c in rows:
        rows[c].append({"Dispatch_Id": d, "Kernel_Name": "fillBuffer", "Grid_Size": 64, "Counter_Name": c,
                        "Counter_Value": 999.0})
    pf, pw = tmp_path / "f.csv", tmp_path / "w.csv"
    _write(pf, fields, rows["FETCH_SIZE"])
    _write(pw, fields, rows["WRITE_SIZE"])
    t = step_traffic(str(pf), str(pw), 512, calls=3)
    assert abs(t["fetch_bytes_per_call"] - 157.0 * 1024 * 2) < 1e-6
    assert abs(t["write_bytes_per_call"] - 22.0 * 1024 * 2) < 1e-6
    k = {r["kernel"]: r for r in t["kernels"]}
    assert not k["fillBuffer"]["per_call"] and k["elementwise"]["per_call"]
    assert k["Cijk_gemm"]["dispatches"] == 6 and abs(k["Cijk_gemm"]["fetch_bytes_per_call"] - 150.0 * 2048) < 1e-6


def test_kernel_names_with_the_reduction_flag():
    """The kernel template carries a bool (launch with reductions): the short
    name keeps the shape and dtype, and marks the reduction instantiation."""
    from fuseml_amd.profiling import _short

    base = "_ZN12_GLOBAL__N_120gemm_epilogue_kernelILi256ELi256ELi64ELi2ELi2ELi2ELi6E"
    assert _short(base + "DF16bLb0EEEv16fuseml_gemm_desc") == "gemm_epilogue_kernel<256,256,64,2,2,2,6,bf16>"
    assert _short(base + "DF16_Lb1EEEv16fuseml_gemm_desc") == "gemm_epilogue_kernel<256,256,64,2,2,2,6,f16,red>"
    assert _short(GEMM) == "gemm_epilogue_kernel<256,256,32,4,2,4,1,bf16>"
    assert _short("__amd_rocclr_copyBuffer") == "__amd_rocclr_copyBuffer"
    # the epilogue-chain template argument: chain 0 (generic loop) is not shown
    assert _short(base + "DF16bLb0ELi0EEEv16fuseml_gemm_desc") == "gemm_epilogue_kernel<256,256,64,2,2,2,6,bf16>"
    assert _short(base + "DF16bLb0ELi3EEEv16fuseml_gemm_desc") == "gemm_epilogue_kernel<256,256,64,2,2,2,6,bf16,ch3>"
    assert _short(base + "DF16bLb1ELi8EEEv16fuseml_gemm_desc") == \
        "gemm_epilogue_kernel<256,256,64,2,2,2,6,bf16,red,ch8>"


def test_kernel_names_demangled_by_the_profiler():
    """rocprofv3 demangles some instantiations (named namespace): the short name
    is the same as for the mangled form, and a garbled type tail keeps only the
    tile integers."""
    from fuseml_amd.profiling import _short

    named = "_ZN11fuseml_gemm20gemm_epilogue_kernelILi256ELi256ELi32ELi4ELi2ELi4ELi1EDF16bLb0EEEv16fuseml_gemm_desc"
    assert _short(named) == "gemm_epilogue_kernel<256,256,32,4,2,4,1,bf16>"
    dem = "void fuseml_gemm::gemm_epilogue_kernel<256, 256, 64, 2, 2, 2, 6, __bf16, true>(fuseml_gemm_desc)"
    assert _short(dem) == "gemm_epilogue_kernel<256,256,64,2,2,2,6,bf16,red>"
    dem_ch = "void fuseml_gemm::gemm_epilogue_kernel<256, 256, 64, 2, 2, 2, 6, __bf16, false, 7>(fuseml_gemm_desc)"
    assert _short(dem_ch) == "gemm_epilogue_kernel<256,256,64,2,2,2,6,bf16,ch7>"
    garbled = "void fuseml_gemm::gemm_epilogue_kernel<256, 256, 64, 2, 2, 2, 6, bool _Accum, bool, E>(fuseml_gemm_desc)"
    assert _short(garbled) == "gemm_epilogue_kernel<256,256,64,2,2,2,6,...>"


def test_counter_summary_means_per_launch_and_wave(tmp_path):
    """`counters` averages each counter per (kernel, launch) and per wave of the grid."""
    from fuseml_amd.profiling import counter_summary

    rows = []
    did = 0
    for step in range(2):
        for pos, vals in ((0, (100.0, 4.0)), (1, (300.0, 0.0))):
            did += 1
            for c, v in zip(("SQ_INSTS_VALU", "SQ_LDS_BANK_CONFLICT"), vals):
                rows.append({"Dispatch_Id": did, "Kernel_Name": GEMM, "Grid_Size": 128,
                             "Counter_Name": c, "Counter_Value": v + step})
    p = tmp_path / "c_counter_collection.csv"
    _write(p, ["Dispatch_Id", "Kernel_Name", "Grid_Size", "Counter_Name", "Counter_Value"], rows)
    out = counter_summary(str(p), per_step=2)
    assert out["counters"] == ["SQ_INSTS_VALU", "SQ_LDS_BANK_CONFLICT"]
    k = {e["launch"]: e for e in out["kernels"]}
    assert k[0]["counters"]["SQ_INSTS_VALU"] == 100.5 and k[1]["counters"]["SQ_INSTS_VALU"] == 300.5
    assert k[0]["per_wave"]["SQ_INSTS_VALU"] == 50.2 or k[0]["per_wave"]["SQ_INSTS_VALU"] == 50.3
    assert k[1]["counters"]["SQ_LDS_BANK_CONFLICT"] == 0.5 and k[0]["dispatches"] == 2
