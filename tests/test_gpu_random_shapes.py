"""Parity on seeded random shapes (B <= 700, H <= 64, L, K <= 48), with the
library's own kernel choice (no environment override): FWD and dX against
FP64 within 1e-5 and bit-exact with the reference's fmaf chain wherever the
VALU kernels serve, atomic and deterministic dK against FP64 within 1e-4
with exact zeros for taps that never meet the row and a bitwise repeat.
Every fourth case stores its tensors 4-byte but not 16-byte aligned, which
sends FWD/dX to the VALU kernels' dword path and dK to its dword staging.

The draw favours the places where the dispatch changes: channel counts that
are multiples of 8 and 16, rows of every length, and taps on both sides of
the matrix-core thresholds."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pathtile_amd import runtime as _runtime

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-5
DK_TOL = 1e-4


def _draw(n: int, seed: int = 20261202):
    rng = np.random.default_rng(seed)
    cases = []
    for i in range(n):
        B = int(rng.choice([1, 2, 15, 16, 17, 63, 64, 65, 129, 300, 513, 700]))
        H = int(rng.choice([1, 3, 5, 8, 12, 16, 24, 32, 40, 48, 64]))
        L = int(rng.integers(1, 49))
        K = int(rng.integers(1, 49) if i % 2 else rng.integers(24, 49))
        cases.append((B, H, L, K, i % 4 == 3))
    return cases


CASES = _draw(48)


@pytest.fixture(scope="module")
def rt():
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime()
    yield r
    r.close()


def _place(t: torch.Tensor, misaligned: bool) -> torch.Tensor:
    if not misaligned:
        return t.to("cuda:0").contiguous()
    flat = torch.zeros(t.numel() + 1, device="cuda:0")
    flat[1:] = t.reshape(-1).to("cuda:0")
    v = flat[1:].view(t.shape)
    assert v.data_ptr() % 16 != 0
    return v


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}H{}L{}K{}{}".format(*c[:4], "m" if c[4] else ""))
def test_random_shape(rt, case):
    B, H, L, K, mis = case
    print(f"[case] random B={B} H={H} L={L} K={K} misaligned={mis}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, 7000 + B + 3 * H + 5 * L + 7 * K)
    xd, dyd = _place(x, mis), _place(dy, mis)
    wd = w.to("cuda:0")
    y = torch.empty_like(xd)
    rt.launch_fwd(xd, wd, y)
    dx = torch.empty_like(dyd)
    rt.launch_bwd_input(dyd, wd, dx)
    y, dx = y.cpu().numpy(), dx.cpu().numpy()
    assert oracle.normalized_max_abs(y, oracle.fwd_f64(x, w)) < FWD_TOL
    assert oracle.normalized_max_abs(dx, oracle.dx_f64(dy, w)) < FWD_TOL
    if mis or not _runtime.rows_on_matrix_cores(B, H, L, K):
        assert np.array_equal(y, oracle.fwd_f32_refchain(x, w))
        assert np.array_equal(dx, oracle.dx_f32_refchain(dy, w))

    ref = oracle.dk_f64(dy, x, K)
    ga = torch.full((H, K), float("nan"), device="cuda:0")
    rt.launch_bwd_weight(dyd, xd, ga, K, zero_first=True)
    gd1 = torch.full((H, K), float("nan"), device="cuda:0")
    rt.launch_bwd_weight_deterministic(dyd, xd, gd1, K)
    gd2 = torch.full((H, K), float("nan"), device="cuda:0")
    rt.launch_bwd_weight_deterministic(dyd, xd, gd2, K)
    ga, gd1, gd2 = ga.cpu().numpy(), gd1.cpu().numpy(), gd2.cpu().numpy()
    assert oracle.normalized_max_abs(ga, ref) < DK_TOL
    assert oracle.normalized_max_abs(gd1, ref) < DK_TOL
    assert np.array_equal(gd1, gd2)
    for j in range(K):
        lo, hi = oracle.valid_tap_range(L, K, j)
        if hi <= lo:
            assert np.all(ga[:, j] == 0.0) and np.all(gd1[:, j] == 0.0)


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}H{}L{}K{}".format(c[0], 8 * -(-c[1] // 8), *c[2:4]))
def test_random_shape_matrix_cores_forced(rt, case, monkeypatch):
    """The same draws with H rounded up to a multiple of 8 and 16-byte aligned
    tensors, FWD/dX forced onto the matrix cores: FP64 within 1e-5."""
    B, H, L, K, _ = case
    H = 8 * -(-H // 8)
    monkeypatch.setenv("PATHTILE_ROWS_ALGO", "mfma")
    print(f"[case] random, matrix cores forced B={B} H={H} L={L} K={K}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, 9000 + B + 3 * H + 5 * L + 7 * K)
    xd, wd, dyd = x.to("cuda:0"), w.to("cuda:0"), dy.to("cuda:0")
    y = torch.empty_like(xd)
    rt.launch_fwd(xd, wd, y)
    dx = torch.empty_like(dyd)
    rt.launch_bwd_input(dyd, wd, dx)
    assert oracle.normalized_max_abs(y.cpu().numpy(), oracle.fwd_f64(x, w)) < FWD_TOL
    assert oracle.normalized_max_abs(dx.cpu().numpy(), oracle.dx_f64(dy, w)) < FWD_TOL
