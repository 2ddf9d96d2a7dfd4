"""CPU checks of bench.py's figures that do not need a GPU: algorithmic bytes
per launch and the fused-against-eager traffic from the committed summaries."""

import importlib.util
import os

import torch

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _bench():
    spec = importlib.util.spec_from_file_location("bench_under_test", os.path.join(REPO, "bench.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod


def test_algorithmic_bytes_counts_each_tensor_once():
    b = _bench()
    M, N, K = 64, 48, 32
    x = torch.zeros(M, K, dtype=torch.bfloat16)
    w = torch.zeros(N, K, dtype=torch.bfloat16)
    bias = torch.zeros(N, dtype=torch.bfloat16)
    out = torch.zeros(M, N, dtype=torch.bfloat16)
    # G2-style call: the residual is x itself, passed twice
    got = b._algorithmic_bytes((bias, x, w.t(), x), out)
    assert got == 2 * (N + M * K + N * K + M * N)
    # tuple outputs (reductions in fp32 plus the tile)
    red = torch.zeros(M, dtype=torch.float32)
    assert b._algorithmic_bytes((x, w.t()), (red, red.clone(), out)) == 2 * (M * K + N * K + M * N) + 8 * M


def test_hbm_traffic_from_committed_summaries():
    b = _bench()
    c2 = b._hbm_traffic("C2", [[16384, 4096, 1024], [16384, 1024, 4096]])
    # the fused step writes the two group outputs (h and y); the counters are
    # KiB per dispatch scaled by a copy kernel's reading, so a run can be off
    # by a few bytes
    def near(got, want):
        return abs(got - want) <= 1e-6 * want
    assert near(c2["fused_write_bytes"], 16384 * 4096 * 2 + 16384 * 1024 * 2)
    assert c2["final_output_bytes"] == 16384 * 1024 * 2
    assert 0.5 < c2["intermediate_eliminated_frac"] < 0.6
    c3 = b._hbm_traffic("C3", [[16384, 4096, 1024]])
    assert c3["intermediate_eliminated_frac"] == 1.0 and c3["saved_frac"] > 0.6
    c5 = b._hbm_traffic("C5", [[8192, 16384, 4096], [8192, 4096, 16384]] * 4)
    assert near(c5["fused_write_bytes"], 4 * (8192 * 16384 * 2 + 8192 * 4096 * 2))
    assert b._hbm_traffic("nope", [[1, 1, 1]]) is None


def test_mfma_busy_from_committed_summaries():
    b = _bench()
    for w, launches in (("C2", 2), ("C3", 1), ("C4", 1), ("C5", 8)):
        for i in range(launches):
            f = b._mfma_busy(w, i)
            assert f is not None and 0.1 < f < 1.0, (w, i, f)
    assert b._mfma_busy("nope", 0) is None


def test_preset_traffic_matches_the_c2_table():
    """The MLP block at C2's shape (16384; 1024 -> 4096) counted from shapes:
    721.4 MB eager, 385.9 MB with two fused launches, 83.9 MB compulsory, so
    the two launches remove 52.6% of the intermediate traffic (46.5% of all of
    it) and a single-kernel block all of it."""
    bench = _bench()

    t = bench.preset_traffic("mlp_block", 16384, 1024, 4096, 1)
    assert round(t["eager_bytes"] / 1e6, 1) == 721.4
    assert round(t["fused_bytes"] / 1e6, 1) == 385.9
    assert round(t["compulsory_bytes"] / 1e6, 1) == 83.9
    assert t["fused_eliminated"] == 0.5263 and t["fused_total_saved"] == 0.4651
    assert t["single_kernel_eliminated"] == 1.0


def test_preset_traffic_activation_heavy_and_stacked():
    """The activation-heavy block adds two [M, I] round trips to eager only
    (its scale and shift run inside either fused path); a stack of blocks keeps
    the blocks' outputs as intermediates."""
    bench = _bench()

    M, D, I = 16384, 256, 1024
    mlp = bench.preset_traffic("mlp_block", M, D, I, 1)
    act = bench.preset_traffic("activation_heavy", M, D, I, 1)
    assert act["eager_bytes"] - mlp["eager_bytes"] == 2 * 2 * M * I * 2
    assert act["fused_bytes"] == mlp["fused_bytes"] and act["single_kernel_bytes"] == mlp["single_kernel_bytes"]
    assert act["fused_eliminated"] > mlp["fused_eliminated"] and act["single_kernel_eliminated"] == 1.0
    st = bench.preset_traffic("stacked_mlp", M, D, I, 4)
    assert st["eager_bytes"] == 4 * mlp["eager_bytes"] and st["fused_bytes"] == 4 * mlp["fused_bytes"]
    # 4 blocks: compulsory = input + 4 blocks' weights + output
    assert st["compulsory_bytes"] == (2 * M * D + 4 * (2 * D * I + I + D)) * 2


def test_preset_roofline_names_the_binding_roofline():
    """Both fractions from one device time; the bound is the roofline with the
    longer floor, which changes sides at 312.5 flops per compulsory byte (the
    2.5 PFLOP/s : 8 TB/s ridge)."""
    bench = _bench()
    B = 10 ** 6
    above = bench.preset_roofline(0.1, 320.0 * B, B)
    below = bench.preset_roofline(0.1, 300.0 * B, B)
    assert above["bound"] == "mfma" and below["bound"] == "hbm"
    assert above["tflops"] == 3.2 and above["frac_mfma"] == round(3.2 / 2500.0, 4)
    assert above["GBps"] == 10.0 and above["frac_hbm"] == round(10.0 / 8000.0, 4)
    # frac_of_bound = the bound's floor over the measured time
    assert abs(above["frac_of_bound"] - 320.0 * B / 2.5e15 / 1e-4) <= 1e-4
    assert abs(below["frac_of_bound"] - B / 8e12 / 1e-4) <= 1e-4
    # the reference's memory_bound preset (16384 rows, 256 -> 1024) is MFMA-bound on this GPU
    M, D, I = 16384, 256, 1024
    t = bench.preset_traffic("mlp_block", M, D, I, 1)
    r = bench.preset_roofline(0.03, 2 * 2.0 * M * D * I, t["compulsory_bytes"])
    assert r["bound"] == "mfma"
