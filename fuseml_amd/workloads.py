"""Synthetic inputs and eager modules of the five benchmark configurations.

C1..C5 are the entries of the benchmark's config list (the reference's
preset workloads, benchmarks/bench_mlp_block.py:64-220, at the shapes the
MI355X benchmark is quoted on).  Inputs are generated on the CPU from seeded
``torch.Generator``s and cast to the config dtype, so the GPU path, the eager
path and the CPU oracle all see bit-identical values.  Weights follow
``nn.Linear`` storage ``W[out, in]``; a traced graph sees ``t(W)``.

``scale`` shrinks the row count M (and nothing else) for quick tests; rows are
independent in every workload.
"""

from __future__ import annotations

from dataclasses import dataclass, field
from typing import Dict, List, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F


class TransformerMLP(nn.Module):
    """Linear -> GELU -> Linear [+ residual] (bench_mlp_block.py:160-182)."""

    def __init__(self, d_model: int, d_inter: int, approximate: str = "none", residual: bool = True):
        super().__init__()
        self.linear1 = nn.Linear(d_model, d_inter)
        self.gelu = nn.GELU(approximate=approximate)
        self.linear2 = nn.Linear(d_inter, d_model)
        self.residual = residual

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = self.linear2(self.gelu(self.linear1(x)))
        return y + x if self.residual else y


class ActivationHeavy(nn.Module):
    """sigmoid(relu(Linear(x)) * g) + r — five pointwise ops after one GEMM."""

    def __init__(self, d_model: int, d_inter: int):
        super().__init__()
        self.linear = nn.Linear(d_model, d_inter)
        self.row = nn.Parameter(torch.zeros(d_inter), requires_grad=False)

    def forward(self, x: torch.Tensor, g: torch.Tensor) -> torch.Tensor:
        return torch.sigmoid(torch.relu(self.linear(x)) * g) + self.row


class GemmRowReductions(nn.Module):
    """h = relu(x W^T); returns h and its fp32 row sum, amax and mean."""

    def __init__(self, d_model: int, d_out: int):
        super().__init__()
        self.linear = nn.Linear(d_model, d_out, bias=False)

    def forward(self, x: torch.Tensor):
        h = torch.relu(self.linear(x))
        return h, h.sum(-1, dtype=torch.float32), h.amax(-1).float(), h.mean(-1, dtype=torch.float32)


class ActivationHeavyMLP(nn.Module):
    """Linear -> GELU -> * 0.5 -> + 0.125 -> Linear -> + residual: the
    reference's activation-heavy preset block (bench_mlp_block.py:185-207),
    two more pointwise ops absorbed into the first group."""

    def __init__(self, d_model: int, d_inter: int):
        super().__init__()
        self.linear1 = nn.Linear(d_model, d_inter)
        self.gelu = nn.GELU()
        self.linear2 = nn.Linear(d_inter, d_model)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        h = self.gelu(self.linear1(x)) * 0.5 + 0.125
        return self.linear2(h) + x


class StackedMLP(nn.Module):
    """Blocks of TransformerMLP (bench_mlp_block.py:210-220)."""

    def __init__(self, d_model: int, d_inter: int, num_blocks: int):
        super().__init__()
        self.blocks = nn.ModuleList([TransformerMLP(d_model, d_inter) for _ in range(num_blocks)])

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        for blk in self.blocks:
            x = blk(x)
        return x


@dataclass
class Workload:
    name: str
    model: nn.Module
    inputs: Tuple[torch.Tensor, ...]
    dtype: torch.dtype
    flops: float  # algorithmic FLOPs of one forward (2*M*N*K per GEMM)
    gemms: List[Tuple[int, int, int]] = field(default_factory=list)  # (M, N, K) per GEMM

    def to(self, device) -> "Workload":
        self.model = self.model.to(device)
        self.inputs = tuple(t.to(device) for t in self.inputs)
        return self


def _gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def c1_transformer_mlp_small(scale: float = 1.0) -> Workload:
    M = max(1, int(64 * scale))
    torch.manual_seed(0)
    model = TransformerMLP(512, 2048, approximate="tanh", residual=False).eval()
    x = torch.randn(M, 512, generator=_gen(0))
    g = [(M, 2048, 512), (M, 512, 2048)]
    return Workload("C1_transformer_mlp_small_fp32", model, (x,), torch.float32,
                    sum(2.0 * m * n * k for m, n, k in g), g)


def c2_mlp_block(scale: float = 1.0, dtype=torch.bfloat16) -> Workload:
    M = max(1, int(16384 * scale))
    D, I = 1024, 4096
    torch.manual_seed(0)
    model = TransformerMLP(D, I)
    with torch.no_grad():
        model.linear1.bias.copy_(torch.empty(I).uniform_(-0.03, 0.03, generator=_gen(1)))
    model = model.to(dtype).eval()
    x = torch.randn(M, D, generator=_gen(0)).to(dtype)
    g = [(M, I, D), (M, D, I)]
    return Workload("C2_mlp_block_memory_bound_bf16", model, (x,), dtype,
                    sum(2.0 * m * n * k for m, n, k in g), g)


def c3_activation_heavy(scale: float = 1.0, dtype=torch.bfloat16) -> Workload:
    M = max(1, int(16384 * scale))
    D, I = 1024, 4096
    torch.manual_seed(0)
    model = ActivationHeavy(D, I)
    with torch.no_grad():
        model.row.copy_(torch.empty(I).uniform_(-0.03, 0.03, generator=_gen(2)))
    model = model.to(dtype).eval()
    x = torch.randn(M, D, generator=_gen(0)).to(dtype)
    gate = torch.rand(M, I, generator=_gen(1)).to(dtype)
    g = [(M, I, D)]
    return Workload("C3_activation_heavy_bf16", model, (x, gate), dtype, 2.0 * M * I * D, g)


def c4_gemm_row_reductions(scale: float = 1.0, dtype=torch.bfloat16) -> Workload:
    M = max(1, int(8192 * scale))
    D, N = 2048, 8192
    torch.manual_seed(0)
    model = GemmRowReductions(D, N).to(dtype).eval()
    x = torch.randn(M, D, generator=_gen(0)).to(dtype)
    g = [(M, N, D)]
    return Workload("C4_gemm_row_reductions_bf16", model, (x,), dtype, 2.0 * M * N * D, g)


def c5_stacked_mlp(scale: float = 1.0, dtype=torch.bfloat16, num_blocks: int = 4) -> Workload:
    M = max(1, int(8192 * scale))
    D, I = 4096, 16384
    torch.manual_seed(1)
    model = StackedMLP(D, I, num_blocks)
    with torch.no_grad():
        for blk in model.blocks:
            nn.init.xavier_uniform_(blk.linear1.weight)
            nn.init.xavier_uniform_(blk.linear2.weight)
    model = model.to(dtype).eval()
    x = (torch.randn(M, D, generator=_gen(0)) * 0.5).to(dtype)
    g = [(M, I, D), (M, D, I)] * num_blocks
    return Workload("C5_stacked_mlp_x4_bf16", model, (x,), dtype,
                    sum(2.0 * m * n * k for m, n, k in g), g)


# The reference benchmark's presets (bench_mlp_block.py:64-153): M = batch x
# seq rows of a [M, d_model] input, d_model -> d_intermediate; the speedups the
# reference publishes (README.md:85-96) are quoted on these.
REFERENCE_PRESETS: Dict[str, Tuple[str, int, int, int, int]] = {
    # name: (workload, M, d_model, d_intermediate, blocks)
    "small": ("mlp_block", 128, 256, 1024, 1),
    "memory_bound": ("mlp_block", 16384, 256, 1024, 1),
    "medium": ("mlp_block", 2048, 1024, 4096, 1),
    "activation_heavy_memory_bound": ("activation_heavy", 16384, 256, 1024, 1),
    "activation_heavy_medium": ("activation_heavy", 2048, 1024, 4096, 1),
    "stacked_memory_bound": ("stacked_mlp", 8192, 512, 2048, 4),
    "stacked_medium": ("stacked_mlp", 2048, 1024, 4096, 4),
}


def reference_preset(name: str, dtype=torch.bfloat16, seed: int = 0) -> Workload:
    """One of the reference benchmark's presets in bf16: default nn.Linear
    init after ``manual_seed(seed)``, x ~ N(0, 1) (bench_mlp_block.py:959-968)."""
    kind, M, D, I, blocks = REFERENCE_PRESETS[name]
    torch.manual_seed(seed)
    if kind == "mlp_block":
        model: nn.Module = TransformerMLP(D, I)
    elif kind == "activation_heavy":
        model = ActivationHeavyMLP(D, I)
    else:
        model = StackedMLP(D, I, blocks)
    model = model.to(dtype).eval()
    x = torch.randn(M, D, generator=_gen(seed)).to(dtype)
    g = [(M, I, D), (M, D, I)] * blocks
    return Workload(f"preset_{name}", model, (x,), dtype, sum(2.0 * m * n * k for m, n, k in g), g)


WORKLOADS = {
    "C1": c1_transformer_mlp_small,
    "C2": c2_mlp_block,
    "C3": c3_activation_heavy,
    "C4": c4_gemm_row_reductions,
    "C5": c5_stacked_mlp,
}
