"""Channels-last dK through the Flash-DWC bridge ABI on the GPU (marked
``gpu``).

x and dy are [B, 1, L, H] and dw is [1, K, H]
(benchmark/flashdwc_fp32_bridge.cu:21-22). The reference's own check permutes
[B, H, L] tensors into that layout and compares dw[0].T with the FP64 sum
(benchmark/check_dk_fp64_comparison.py:27-65). Bars here:
* within 1e-4 max-abs-scaled of the oracle's FP64 dK (the dK bar);
* accumulation into a non-zero dw (the bridge's "caller must zero dw"
  contract);
* at P, layout invariance: the channels-last result equals the row-major
  dK of the same data to 1e-5.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

DK_TOL = 1e-4


@pytest.fixture(scope="module")
def rt():
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime()
    runtime.install_runtime(r)
    yield r


def _cl(t: torch.Tensor) -> torch.Tensor:
    """[B, H, L] -> [B, 1, L, H] (the reference's permute, :42-43)."""
    return t.permute(0, 2, 1).unsqueeze(1).contiguous()


CASES = [
    (64, 32, 48, 48, 1),
    (64, 32, 48, 48, 4),
    (32, 64, 37, 48, 2),    # ragged L, K > L
    (16, 96, 16, 48, 1),    # K > L
    (48, 32, 44, 5, 3),
    (128, 256, 32, 9, 8),
    (16, 32, 4, 3, 1),      # tiny rows
    (1008, 64, 40, 24, 63),
    (400, 32, 48, 1, 25),   # K = 1
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}H{}L{}K{}GZ{}".format(*c))
def test_channels_last_dk_against_fp64(rt, case):
    B, H, L, K, gz = case
    print(f"[case] channels-last dK B={B} H={H} L={L} K={K} GZ={gz}", flush=True)
    x, _, dy = oracle.make_inputs(B, H, L, K, seed=13000 + B + L + K)
    ref = oracle.dk_f64(dy, x, K)                       # [H, K]
    dw = torch.empty(1, K, H, device="cuda")
    rt.launch_bwd_weight_channels_last(_cl(x).cuda(), _cl(dy).cuda(), dw, gz, zero_first=True)
    got = dw[0].T.double().cpu().numpy()
    assert np.isfinite(got).all()
    assert oracle.normalized_max_abs(got, ref) < DK_TOL
    for j in range(K):
        lo, hi = oracle.valid_tap_range(L, K, j)
        if hi <= lo:
            assert np.all(got[:, j] == 0)


def test_channels_last_dk_accumulates(rt):
    """dw is added to, not overwritten (the caller zeroes it)."""
    B, H, L, K = 64, 64, 48, 17
    x, _, dy = oracle.make_inputs(B, H, L, K, seed=14)
    ref = oracle.dk_f64(dy, x, K)
    dw = torch.full((1, K, H), 1.5, device="cuda")
    rt.launch_bwd_weight_channels_last(_cl(x).cuda(), _cl(dy).cuda(), dw, 1)
    got = dw[0].T.double().cpu().numpy() - 1.5
    assert oracle.normalized_max_abs(got, ref) < DK_TOL


def test_channels_last_dk_primary_shape_matches_row_major(rt):
    """B16384 H128 L48 K48 (the reference's check shape, :23): the
    channels-last dK of the permuted tensors equals the row-major
    deterministic dK of the originals to 1e-5 (the same sums in another
    order), and dK's FP64 adjoint identity holds on a random probe:
    sum_hj dk[h,j] v[h,j] = sum_bht dy[b,h,t] (x conv v)[b,h,t]."""
    B, H, L, K = 16384, 128, 48, 48
    print(f"[case] channels-last dK at P B={B} H={H} L={L} K={K}", flush=True)
    x, _, dy = oracle.make_inputs(B, H, L, K, seed=42)
    xd, dyd = x.cuda(), dy.cuda()
    gk = torch.empty(H, K, device="cuda")
    rt.launch_bwd_weight_deterministic(dyd, xd, gk, K)
    dw = torch.zeros(1, K, H, device="cuda")
    rt.launch_bwd_weight_channels_last(_cl(xd), _cl(dyd), dw, 4096 // 16 * 4)
    got = dw[0].T.contiguous()
    scale = float(gk.abs().max())
    assert float((got - gk).abs().max()) / scale < 1e-5
    v = torch.randn(H, K, generator=torch.Generator().manual_seed(7), dtype=torch.float64)
    lhs = float((got.double().cpu() * v).sum())
    # (x conv v)[b,h,t] = sum_j v[h,j] x[b,h,t+j-p] evaluated in FP64 on the GPU
    p = K // 2
    xp = torch.nn.functional.pad(xd.double(), (p, K - 1 - p))
    conv = torch.zeros_like(xd, dtype=torch.float64)
    vd = v.cuda()
    for j in range(K):
        conv += vd[None, :, j:j + 1] * xp[:, :, j:j + L]
    rhs = float((dyd.double() * conv).sum())
    assert abs(lhs - rhs) <= 1e-5 * float((got.double().cpu().abs() * v.abs()).sum())


def test_channels_last_dk_runtime_errors(rt):
    x = torch.zeros(16, 1, 8, 48, device="cuda")
    with pytest.raises(ValueError, match="flash_dk_fp32"):
        rt.launch_bwd_weight_channels_last(x, x.clone(), torch.zeros(1, 3, 48, device="cuda"))
    x = torch.zeros(16, 1, 8, 32, device="cuda")
    with pytest.raises(ValueError, match="flash_dk_fp32"):   # B / GZ = 8
        rt.launch_bwd_weight_channels_last(x, x.clone(), torch.zeros(1, 3, 32, device="cuda"), 2)
    with pytest.raises(ValueError, match=r"\[1,K,H\]"):
        rt.launch_bwd_weight_channels_last(x, x.clone(), torch.zeros(3, 32, device="cuda"))
    with pytest.raises(ValueError, match=r"\[B,1,L,H\]"):
        rt.launch_bwd_weight_channels_last(x[:, 0], x[:, 0].clone(), torch.zeros(1, 3, 32, device="cuda"))


def _random_cl_cases(n: int, seed: int):
    """Seeded cases inside the bridge's contract (H % 32 == 0, B / GZ a
    multiple of 16): any L up to 48, K up to 48, several sample groups."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        gz = int(rng.choice([1, 2, 3, 5, 8]))
        B = gz * 16 * int(rng.integers(1, 5))
        H = 32 * int(rng.integers(1, 5))
        L = int(rng.integers(1, 49))
        K = int(rng.integers(1, 49) if i % 2 else rng.integers(24, 49))
        out.append((B, H, L, K, gz))
    return out


@pytest.mark.parametrize("case", _random_cl_cases(16, 20261204),
                         ids=lambda c: "B{}H{}L{}K{}GZ{}".format(*c))
def test_channels_last_dk_random_cases(rt, case):
    test_channels_last_dk_against_fp64(rt, case)
