"""Write the golden fixtures under tests/golden/ (run from the repo root:
``python tests/golden/make_fixtures.py``).

The reference holds no stored vectors for this path: its correctness gates
compare against PyTorch at run time (kernels/warp_tiled_ampere.py:909-987,
benchmark/check_dk_fp64_comparison.py:29-46). These fixtures freeze that
comparison: inputs from a seeded CPU torch.Generator in the order x, w, dY
(x, dY ~ N(0,1), w ~ N(0,1/K)), outputs from PyTorch CPU autograd through the
reference's PyTorch boundary (benchmark/benchmark_shape_sweep_ampere.py:
220-239: F.pad(x, (K//2, K-1-K//2)) + F.conv1d(groups=H)).

  c1_b64_h16_l48_k48.npz   BASELINE config 1 (CPU plumbing case): x, w, dy;
                           y, dx, dk from float32 autograd; dk64 from float64
                           autograd.
  edge_cases.npz           small edge shapes (K > L, odd K, K = 1, L = 1,
                           L not a multiple of 4, K = 47): inputs and float64
                           autograd outputs, keys "<case>/<name>".
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch
import torch.nn.functional as F

HERE = Path(__file__).resolve().parent

C1 = (64, 16, 48, 48)
C1_SEED = 42

EDGE_CASES = {
    "k_gt_l": (3, 4, 5, 9, 101),
    "odd_k": (2, 3, 16, 7, 102),
    "k1": (2, 5, 12, 1, 103),
    "l1": (4, 3, 1, 5, 104),
    "l37_k48": (5, 6, 37, 48, 105),
    "l48_k47": (3, 4, 48, 47, 106),
    "l16_k48": (3, 2, 16, 48, 107),
    "l48_k4": (6, 5, 48, 4, 108),
}


def pytorch_depthwise_same(x, k):
    K = int(k.shape[1])
    left = K // 2
    x_pad = F.pad(x, (left, K - 1 - left))
    return F.conv1d(x_pad, k.unsqueeze(1), groups=int(x.shape[1]))


def inputs(B, H, L, K, seed):
    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, H, L, generator=g, dtype=torch.float32)
    w = torch.randn(H, K, generator=g, dtype=torch.float32) / math.sqrt(K)
    dy = torch.randn(B, H, L, generator=g, dtype=torch.float32)
    return x, w, dy


def autograd(x, w, dy):
    xr = x.clone().requires_grad_(True)
    wr = w.clone().requires_grad_(True)
    y = pytorch_depthwise_same(xr, wr)
    gx, gw = torch.autograd.grad(y, (xr, wr), dy)
    return y.detach().numpy(), gx.numpy(), gw.numpy()


def main() -> int:
    torch.set_num_threads(1)
    B, H, L, K = C1
    x, w, dy = inputs(B, H, L, K, C1_SEED)
    y, dx, dk = autograd(x, w, dy)
    _, _, dk64 = autograd(x.double(), w.double(), dy.double())
    np.savez_compressed(
        HERE / "c1_b64_h16_l48_k48.npz",
        x=x.numpy(), w=w.numpy(), dy=dy.numpy(), y=y, dx=dx, dk=dk, dk64=dk64,
        shape=np.array(C1), seed=np.array(C1_SEED),
    )
    edge = {}
    for name, (B, H, L, K, seed) in EDGE_CASES.items():
        x, w, dy = inputs(B, H, L, K, seed)
        y64, dx64, dk64 = autograd(x.double(), w.double(), dy.double())
        edge.update({
            f"{name}/x": x.numpy(), f"{name}/w": w.numpy(),
            f"{name}/dy": dy.numpy(), f"{name}/y64": y64,
            f"{name}/dx64": dx64, f"{name}/dk64": dk64,
            f"{name}/shape": np.array((B, H, L, K)),
        })
    np.savez_compressed(HERE / "edge_cases.npz", **edge)
    return 0


if __name__ == "__main__":
    sys.exit(main())
