"""Generate the golden fixtures in tests/golden/*.npz.

Each fixture holds seeded inputs (bf16-representable values stored as
float32, or plain float32 for the fp32 case) and the outputs of the same
computation run by PyTorch eager in float32 on the CPU — the reference's eager
path (benchmarks/bench_mlp_block.py:160-220 module definitions).  Shapes are
small and deliberately ragged (N % 4 != 0, K % 64 != 0) so the fixtures
exercise the kernel's edge paths.

    python tests/golden/make_golden.py      # rewrites the .npz files
"""

import os

import numpy as np
import torch
import torch.nn.functional as F

HERE = os.path.dirname(os.path.abspath(__file__))


def _bf(t):
    return t.to(torch.bfloat16).float()


def _save(name, **arrays):
    np.savez_compressed(os.path.join(HERE, name + ".npz"),
                        **{k: v.detach().float().numpy() for k, v in arrays.items()})


def main():
    g = torch.Generator().manual_seed(20261201)

    # C2-shaped MLP block: l2(gelu(l1(x))) + x
    x = _bf(torch.randn(96, 64, generator=g))
    w1, b1 = _bf(torch.randn(160, 64, generator=g) / 8), _bf(torch.rand(160, generator=g) * 0.06 - 0.03)
    w2, b2 = _bf(torch.randn(64, 160, generator=g) / 12), _bf(torch.randn(64, generator=g) / 10)
    h = F.gelu(F.linear(x, w1, b1))
    y = F.linear(h, w2, b2) + x
    _save("mlp_block", x=x, w1=w1, b1=b1, w2=w2, b2=b2, h=h, y=y)

    # C3-shaped activation-heavy: sigmoid(relu(x W^T + b) * g) + r
    x = _bf(torch.randn(77, 48, generator=g))
    w, b = _bf(torch.randn(200, 48, generator=g) / 7), _bf(torch.randn(200, generator=g) / 10)
    gate, r = _bf(torch.rand(77, 200, generator=g)), _bf(torch.rand(200, generator=g) * 0.06 - 0.03)
    y = torch.sigmoid(torch.relu(F.linear(x, w, b)) * gate) + r
    _save("act_heavy", x=x, w=w, b=b, g=gate, r=r, y=y)

    # C4-shaped: h = relu(x W^T); fp32 row sum / amax / mean (N = 257)
    x = _bf(torch.randn(130, 40, generator=g))
    w = _bf(torch.randn(257, 40, generator=g) / 6)
    hh = torch.relu(F.linear(x, w))
    _save("row_reductions", x=x, w=w, h=hh, sum=hh.sum(-1), amax=hh.amax(-1), mean=hh.mean(-1))

    # column reductions of sigmoid(x W^T + b) (reduction over M)
    x = _bf(torch.randn(70, 24, generator=g))
    w, b = _bf(torch.randn(132, 24, generator=g) / 5), _bf(torch.randn(132, generator=g))
    v = torch.sigmoid(F.linear(x, w, b))
    _save("col_reductions", x=x, w=w, b=b, sum=v.sum(0), amax=v.amax(0), mean=v.mean(0))

    # C1-shaped fp32 TransformerMLP with GELU(tanh), no residual
    x = torch.randn(64, 32, generator=g)
    w1, b1 = torch.randn(128, 32, generator=g) / 6, torch.randn(128, generator=g) / 10
    w2, b2 = torch.randn(32, 128, generator=g) / 11, torch.randn(32, generator=g) / 10
    y = F.linear(F.gelu(F.linear(x, w1, b1), approximate="tanh"), w2, b2)
    _save("transformer_mlp_tanh_fp32", x=x, w1=w1, b1=b1, w2=w2, b2=b2, y=y)

    # C5-shaped stack of three MLP blocks
    x = _bf(torch.randn(64, 32, generator=g) * 0.5)
    arrays = {"x": x}
    y = x
    for i in range(3):
        w1, b1 = _bf(torch.randn(96, 32, generator=g) / 6), _bf(torch.randn(96, generator=g) / 10)
        w2, b2 = _bf(torch.randn(32, 96, generator=g) / 10), _bf(torch.randn(32, generator=g) / 10)
        arrays.update({f"w1_{i}": w1, f"b1_{i}": b1, f"w2_{i}": w2, f"b2_{i}": b2})
        y = F.linear(F.gelu(F.linear(y, w1, b1)), w2, b2) + y
    arrays["y"] = y
    _save("stacked_mlp", **arrays)


if __name__ == "__main__":
    with torch.no_grad():
        main()
