"""BF16 I/O on the GPU (marked ``gpu``): bfloat16 activations and gradients,
FP32 taps and dK, FP32 accumulation on the matrix cores. No counterpart in
the reference (FP32 only).

Bars: the inputs are BF16 values, so the exact result is the FP64 sum over
those values (oracle.fwd_f64 / dx_f64 / dk_f64 of the widened inputs).
FWD/dX run on the BF16 matrix cores with each FP32 tap as a hi + lo BF16
pair (|w - hi - lo| <= 2^-16 |w|) and FP32 accumulation, then one round to
BF16: every element within one BF16 ulp of the FP64 sum plus 2^-16 of the
largest output (the tap split and the accumulation), and at least 99% of
elements equal to the FP64 sum rounded to BF16 (they differ only where those
small errors moved a value across a rounding boundary). dK is FP32: within
1e-4 max-abs-scaled of FP64, and the deterministic variant bitwise
reproducible.
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


def _inputs(B, H, L, K, seed):
    print(f"[case] bf16 B={B} H={H} L={L} K={K} seed={seed}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed)
    return x.to(torch.bfloat16), w, dy.to(torch.bfloat16)


def _check_rounded(out_bf16: torch.Tensor, ref64: np.ndarray) -> None:
    out = out_bf16.float().double().cpu().numpy()
    ref_t = torch.from_numpy(ref64)
    ref_bf = ref_t.to(torch.bfloat16).double().numpy()
    # one BF16 ulp at the reference's magnitude (2^(e - 7)); subnormal floor
    ulp = np.exp2(np.floor(np.log2(np.maximum(np.abs(ref64), 1e-30))) - 7)
    assert np.all(np.abs(out - ref64) <= ulp + 2.0 ** -16 * np.abs(ref64).max())
    assert np.mean(out == ref_bf) >= 0.99


SHAPES = [
    (64, 16, 48, 48),
    (300, 8, 48, 47),
    (129, 24, 32, 9),
    (77, 8, 16, 48),
    (33, 16, 44, 5),
    (1, 8, 4, 3),
    (4097, 64, 40, 24),
]


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_bf16_fwd_dx_against_fp64(rt, shape):
    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=9000 + B + L + K)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    y = torch.empty_like(xd)
    dx = torch.empty_like(dyd)
    rt.launch_fwd_bf16(xd, wd, y)
    rt.launch_bwd_input_bf16(dyd, wd, dx)
    _check_rounded(y, oracle.fwd_f64(x.float(), w))
    _check_rounded(dx, oracle.dx_f64(dy.float(), w))


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_bf16_dk_against_fp64(rt, shape):
    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=9500 + B + L + K)
    xd, dyd = x.cuda(), dy.cuda()
    ref = oracle.dk_f64(dy.float(), x.float(), K)
    ga = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_bf16(dyd, xd, ga, K, zero_first=True)
    g1 = torch.full((H, K), float("nan"), device="cuda")
    g2 = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_deterministic_bf16(dyd, xd, g1, K)
    rt.launch_bwd_weight_deterministic_bf16(dyd, xd, g2, K)
    assert oracle.normalized_max_abs(ga.cpu().numpy(), ref) < DK_TOL
    assert oracle.normalized_max_abs(g1.cpu().numpy(), ref) < DK_TOL
    assert torch.equal(g1, g2)
    for j in range(K):
        lo, hi = oracle.valid_tap_range(L, K, j)
        if hi <= lo:
            assert torch.all(ga[:, j] == 0) and torch.all(g1[:, j] == 0)


@pytest.mark.parametrize("threads", [64, 128, 256, 512])
def test_bf16_dk_every_block_size(threads):
    from pathtile_amd import runtime

    B, H, L, K = 1000, 32, 48, 48
    x, w, dy = _inputs(B, H, L, K, seed=11)
    ref = oracle.dk_f64(dy.float(), x.float(), K)
    r = runtime.HipWarpRuntime(bwdk_block=threads)
    g = torch.empty(H, K, device="cuda")
    r.launch_bwd_weight_bf16(dy.cuda(), x.cuda(), g, K, zero_first=True)
    assert oracle.normalized_max_abs(g.cpu().numpy(), ref) < DK_TOL


@pytest.mark.parametrize("shape", [
    (16384, 128, 48, 48),   # 192 MiB per tensor: 8-channel groups, plain loads
    (22016, 128, 48, 40),   # 258 MiB per tensor: 16-channel groups, non-temporal loads
    (16384, 136, 48, 48),   # 204 MiB, H % 16 != 0
])
def test_bf16_large_shape_sampled_rows(rt, shape):
    """Large BF16 calls on both sides of the 256 MiB load-policy boundary:
    sampled rows of FWD/dX against FP64 (the first and the last sample among
    them) and dK over the full batch."""
    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=12)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    y = torch.empty_like(xd)
    dx = torch.empty_like(dyd)
    rt.launch_fwd_bf16(xd, wd, y)
    rt.launch_bwd_input_bf16(dyd, wd, dx)
    idx = np.sort(np.random.default_rng(3).choice(B, 128, replace=False))
    idx[0], idx[-1] = 0, B - 1
    idx = torch.from_numpy(idx)
    _check_rounded(y[idx.cuda()], oracle.fwd_f64(x[idx].float(), w))
    _check_rounded(dx[idx.cuda()], oracle.dx_f64(dy[idx].float(), w))
    g = torch.empty(H, K, device="cuda")
    rt.launch_bwd_weight_deterministic_bf16(dyd, xd, g, K)
    assert oracle.normalized_max_abs(g.cpu().numpy(), oracle.dk_f64(dy.float(), x.float(), K)) < DK_TOL


def test_bf16_layout_and_dtype_errors(rt):
    x = torch.zeros(4, 8, 18, device="cuda", dtype=torch.bfloat16)
    w = torch.zeros(8, 5, device="cuda")
    with pytest.raises(ValueError, match="unsupported launch configuration"):
        rt.launch_fwd_bf16(x, w, torch.empty_like(x))  # L % 4 != 0
    x = torch.zeros(4, 12, 16, device="cuda", dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="unsupported launch configuration"):
        rt.launch_fwd_bf16(x, torch.zeros(12, 5, device="cuda"), torch.empty_like(x))  # H % 8
    with pytest.raises(ValueError, match="x must be bfloat16"):
        rt.launch_fwd_bf16(x.float(), torch.zeros(12, 5, device="cuda"), torch.empty_like(x))
    with pytest.raises(ValueError, match="k must be float32"):
        rt.launch_fwd_bf16(x, torch.zeros(12, 5, device="cuda", dtype=torch.bfloat16),
                           torch.empty_like(x))


def test_bf16_autograd(rt):
    from pathtile_amd import runtime

    B, H, L, K = 96, 16, 48, 48
    x, w, dy = _inputs(B, H, L, K, seed=13)
    xd = x.cuda().requires_grad_(True)
    wd = w.cuda().requires_grad_(True)
    y = runtime.depthwise_conv_bf16(xd, wd)
    assert y.dtype == torch.bfloat16
    gx, gk = torch.autograd.grad(y, (xd, wd), dy.cuda())
    assert gx.dtype == torch.bfloat16 and gk.dtype == torch.float32
    _check_rounded(y.detach(), oracle.fwd_f64(x.float(), w))
    _check_rounded(gx, oracle.dx_f64(dy.float(), w))
    assert oracle.normalized_max_abs(gk.cpu().numpy(), oracle.dk_f64(dy.float(), x.float(), K)) < DK_TOL


def _random_bf16_shapes(n: int, seed: int):
    """Seeded shapes inside the BF16 path's layout (H % 8 == 0, L % 4 == 0)."""
    rng = np.random.default_rng(seed)
    out = []
    for i in range(n):
        B = int(rng.choice([1, 15, 16, 17, 64, 129, 300, 700]))
        H = int(8 * rng.integers(1, 9))
        L = int(4 * rng.integers(1, 13))
        K = int(rng.integers(1, 49) if i % 2 else rng.integers(24, 49))
        out.append((B, H, L, K))
    return out


@pytest.mark.parametrize("shape", _random_bf16_shapes(24, 20261203), ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_bf16_random_shapes(rt, shape):
    """FWD/dX within one BF16 rounding of FP64, atomic and deterministic dK
    within 1e-4 of FP64 with a bitwise repeat, on seeded random shapes."""
    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=9700 + B + 3 * H + 5 * L + 7 * K)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    y = torch.empty_like(xd)
    dx = torch.empty_like(dyd)
    rt.launch_fwd_bf16(xd, wd, y)
    rt.launch_bwd_input_bf16(dyd, wd, dx)
    _check_rounded(y, oracle.fwd_f64(x.float(), w))
    _check_rounded(dx, oracle.dx_f64(dy.float(), w))
    ref = oracle.dk_f64(dy.float(), x.float(), K)
    ga = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_bf16(dyd, xd, ga, K, zero_first=True)
    g1 = torch.full((H, K), float("nan"), device="cuda")
    g2 = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_deterministic_bf16(dyd, xd, g1, K)
    rt.launch_bwd_weight_deterministic_bf16(dyd, xd, g2, K)
    assert oracle.normalized_max_abs(ga.cpu().numpy(), ref) < DK_TOL
    assert oracle.normalized_max_abs(g1.cpu().numpy(), ref) < DK_TOL
    assert torch.equal(g1, g2)
