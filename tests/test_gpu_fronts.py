"""The VALU tile kernel's fronts (marked ``gpu``).

The persistent grid walks the tiles in fronts (PATHTILE_ROWS_FRONTS, two by
default on grids of more than one round): each front covers one contiguous
chunk of tiles with an equal share of the waves. Whatever the front count,
every tile must be computed exactly once and every output must be the
reference's FP32 fmaf chain (kernels/warp_tiled_ampere.py:404-433 FWD,
:472-501 dX), so the outputs start as NaN and are compared in full, bit for
bit, against the oracle's restatement of that chain.

Shapes: several rounds of tiles with a ragged last tile, a channel period
that forces the host to round the grid (H = 37, H = 96), rows of at most 16
columns (8 waves per CU), and rows that are not whole float4s (the dword
path).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

SHAPES = [
    (2048, 64, 48, 4),    # 2048 tiles, 2 rounds at 1024 waves
    (3000, 64, 48, 4),    # ragged: 3000 * 64 rows, 3 rounds
    (4100, 37, 32, 8),    # channel period 37 tiles, grid rounded to it
    (8192, 64, 16, 3),    # L <= 16: 8 waves per CU, 4 rounds
    (5000, 96, 37, 4),    # L % 4 != 0: dword path, period 3 tiles
]


@pytest.fixture(scope="module")
def rt():
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime()
    yield r
    r.close()


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "b{}_h{}_l{}_k{}".format(*s))
def test_fronts_cover_every_tile_bit_exact(rt, shape, monkeypatch):
    B, H, L, K = shape
    print(f"[case] fronts B={B} H={H} L={L} K={K}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=B + H + L + K)
    y_ref = oracle.fwd_f32_refchain(x, w)
    dx_ref = oracle.dx_f32_refchain(dy, w)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    # the tile kernel even where the channel period would hand the call to
    # the streaming kernel
    monkeypatch.setenv("PATHTILE_ROWS_ALGO", "tile")
    for fronts in (1, 2, 4, 8):
        monkeypatch.setenv("PATHTILE_ROWS_FRONTS", str(fronts))
        y = torch.full_like(xd, float("nan"))
        dx = torch.full_like(dyd, float("nan"))
        rt.launch_fwd(xd, wd, y)
        rt.launch_bwd_input(dyd, wd, dx)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().numpy(), y_ref), fronts
        assert np.array_equal(dx.cpu().numpy(), dx_ref), fronts
