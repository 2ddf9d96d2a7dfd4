"""The cost model's thresholds against the committed measurement they come from.

``profiles/cost_model_calibration.json`` is the output of
``python -m fuseml_amd.calibration`` on one MI355X: per GEMM group, the fused
kernel, the eager ops and hipBLASLt's plain GEMM on the same inputs.
``profiles/mlp_block_crossover.json`` (``--mlp``) times compiled MLP blocks with
two launches and with the single-kernel MLP; the default
``fuse_mlp_block="auto"`` rule must pick the faster one.  For every
row whose fused and eager times differ by more than the tie margin, the rules
the compiler applies today (:func:`fused_beats_eager` and the few-tile rule of
:func:`trigger_is_fusible`) must pick the measured winner; a row within the
margin may go either way.  The test recomputes the decision from the current
code, so changing a threshold without re-measuring fails here.
"""

import json
import os

import pytest
import torch

from fuseml_amd import calibration as cal
from fuseml_amd.compiler import (MIN_TILES_LONG_K, epilogue_passes, few_tile_verdict, fused_beats_eager,
                                 weight_streaming)
from fuseml_amd.mlp import mlp_block_beats_two_launches

PROFILES = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "profiles")
PATH = os.path.join(PROFILES, "cost_model_calibration.json")
MLP_PATH = os.path.join(PROFILES, "mlp_block_crossover.json")
# |fused / eager - 1| below this is a tie: the same rows measured on two boxes
# of the pool differ by 1-2%, and near the crossover the linear rule may give
# up a few per cent (bias + residual at K = 2048: fused 3.4% faster, sent to
# eager; a 2048x2048 bias + GELU at the same K: fused 4.6% slower).
TIE = 0.04
# Few-tile groups take 10-50 us, where eager's time per call sits on its host
# floor, which moves between boxes (1024x1024 at K = 4096: eager 24.1 us on one
# box, 26.8 on another, fused 25.4-25.8 on both): within 8% they are ties.
FEW_TILE_TIE = 0.08
# The MLP crossover's near-ties move further between boxes: M = 16384, D = 512
# measured single/two 1.06 on one box and 0.94-0.96 in three runs on another.
MLP_TIE = 0.07


def _rows():
    with open(PATH) as f:
        return json.load(f)["rows"]


def _decision(row):
    spec, _ = cal._spec(row["chain"])
    addmm = row["chain"] != "relu_3red"
    if few_tile_verdict(row["M"], row["N"], row["K"]) is not None and not weight_streaming(row["M"], row["N"]):
        return False
    return fused_beats_eager(spec, row["K"], dtype=torch.bfloat16, gemm_is_addmm=addmm, M=row["M"], N=row["N"])[0]


def test_calibration_covers_the_config_groups_and_both_rules():
    rows = _rows()
    labels = {r["group"] for r in rows}
    assert {g[0] for g in cal.CONFIG_GROUPS} <= labels
    few = [r for r in rows if r["tiles_128"] < MIN_TILES_LONG_K]
    # the few-tile rule is exercised on both sides
    assert any(few_tile_verdict(r["M"], r["N"], r["K"]) is None for r in few)
    assert any(few_tile_verdict(r["M"], r["N"], r["K"]) is not None for r in few)
    assert {1, 2, 4} <= {r["passes"] for r in rows}                       # several pass counts
    for r in rows:
        spec, _ = cal._spec(r["chain"])
        assert r["passes"] == epilogue_passes(spec, gemm_is_addmm=r["chain"] != "relu_3red")


@pytest.mark.parametrize("row", _rows(), ids=lambda r: r["group"])
def test_rule_picks_the_measured_winner(row):
    ratio = row["fused_ms"] / row["eager_ms"]
    if abs(ratio - 1.0) < (FEW_TILE_TIE if row["tiles_128"] < MIN_TILES_LONG_K else TIE):
        pytest.skip(f"tie: fused/eager = {ratio:.3f}")
    assert _decision(row) == (ratio < 1.0), (
        f"{row['group']}: fused {row['fused_ms']} ms, eager {row['eager_ms']} ms, rule fuses={_decision(row)}")


def _mlp_rows():
    with open(MLP_PATH) as f:
        return json.load(f)["rows"]


def test_mlp_crossover_covers_both_outcomes():
    rows = _mlp_rows()
    assert any(r["single_over_two"] < 1 - MLP_TIE for r in rows) and any(r["single_over_two"] > 1 + MLP_TIE for r in rows)
    assert {256, 512, 1024} <= {r["D"] for r in rows}


@pytest.mark.parametrize("row", _mlp_rows(), ids=lambda r: f"M{r['M']}-D{r['D']}-I{r['I']}")
def test_mlp_rule_picks_the_measured_winner(row):
    ratio = row["single_over_two"]
    if abs(ratio - 1.0) < MLP_TIE:
        pytest.skip(f"tie: single/two = {ratio:.3f}")
    binds = mlp_block_beats_two_launches(row["M"], row["D"], row["I"])[0]
    assert binds == (ratio < 1.0), f"{row}: rule binds={binds}"
