"""Pins for the CPU oracle (oracle/), CPU only.

Each oracle function is checked against something it does not restate:
PyTorch's own conv1d/autograd (the library routine the reference validates
against, kernels/warp_tiled_ampere.py:909-987), the committed golden fixtures,
an exact-arithmetic emulation of the reference's fmaf chain, brute-force sums
on tiny shapes, math.fsum, and closed forms (delta taps, shifts, K = 1, L = 1,
linearity, the adjoint identity <FWD(x), dY> = <x, DX(dY)>, dK as a sum of
FWD outputs, exactly-zero taps). test_mutants_are_caught plants plausible
mistakes in a CPU restatement and shows each is rejected by these checks.
"""

from __future__ import annotations

import math
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle

GOLDEN = Path(__file__).resolve().parent / "golden"


def _np(t):
    return t.detach().cpu().numpy()


# ---------------------------------------------------------------------------
# Exact fmaf emulation (one rounding of a*b + c to float32, ties to even)
# ---------------------------------------------------------------------------
def _fmaf(a: np.float32, b: np.float32, c: np.float32) -> np.float32:
    exact = Fraction(float(a)) * Fraction(float(b)) + Fraction(float(c))
    f = np.float32(float(exact))
    cands = (np.nextafter(f, np.float32(-np.inf)), f, np.nextafter(f, np.float32(np.inf)))

    def key(v):
        lsb = int(np.array(v, dtype=np.float32).view(np.uint32)) & 1
        return (abs(Fraction(float(v)) - exact), lsb)

    return np.float32(min(cands, key=key))


def _refchain_fwd_emulated(x, w):
    B, H, L = x.shape
    K = w.shape[1]
    pad = K // 2
    y = np.zeros_like(x)
    for b in range(B):
        for h in range(H):
            for t in range(L):
                acc = np.float32(0.0)
                for kk in range(K):
                    xi = t + kk - pad
                    if 0 <= xi < L:
                        acc = _fmaf(x[b, h, xi], w[h, kk], acc)
                y[b, h, t] = acc
    return y


def _refchain_dx_emulated(dy, w):
    B, H, L = dy.shape
    K = w.shape[1]
    pad = K // 2
    dx = np.zeros_like(dy)
    for b in range(B):
        for h in range(H):
            for t in range(L):
                acc = np.float32(0.0)
                for kk in range(K):
                    tout = t - kk + pad
                    if 0 <= tout < L:
                        acc = _fmaf(dy[b, h, tout], w[h, kk], acc)
                dx[b, h, t] = acc
    return dx


@pytest.mark.parametrize("shape", [(2, 2, 9, 5), (1, 3, 7, 8), (2, 1, 12, 12)])
def test_refchain_is_the_reference_fmaf_chain(shape):
    B, H, L, K = shape
    x, w, dy = (_np(t) for t in oracle.make_inputs(B, H, L, K, seed=sum(shape)))
    y = oracle.fwd_f32_refchain(x, w)
    dx = oracle.dx_f32_refchain(dy, w)
    assert np.array_equal(y, _refchain_fwd_emulated(x, w))
    assert np.array_equal(dx, _refchain_dx_emulated(dy, w))


# ---------------------------------------------------------------------------
# Golden fixtures (PyTorch CPU autograd through the reference's boundary)
# ---------------------------------------------------------------------------
def test_c1_fixture_fp32_and_fp64():
    d = np.load(GOLDEN / "c1_b64_h16_l48_k48.npz")
    x, w, dy = d["x"], d["w"], d["dy"]
    K = w.shape[1]
    # FP32 chains in different orders agree to a few ulps of the output scale.
    assert oracle.normalized_max_abs(oracle.fwd_f32_refchain(x, w), d["y"]) < 1e-6
    assert oracle.normalized_max_abs(oracle.dx_f32_refchain(dy, w), d["dx"]) < 1e-6
    assert oracle.normalized_max_abs(oracle.fwd_f64(x, w), d["y"]) < 1e-6
    assert oracle.normalized_max_abs(oracle.dx_f64(dy, w), d["dx"]) < 1e-6
    assert oracle.normalized_max_abs(oracle.dk_f64(dy, x, K), d["dk64"]) < 1e-12
    assert oracle.normalized_max_abs(d["dk"], d["dk64"]) < 1e-5


def _edge_cases():
    d = np.load(GOLDEN / "edge_cases.npz")
    names = sorted({k.split("/")[0] for k in d.files})
    return d, names


def test_edge_fixtures_fp64():
    d, names = _edge_cases()
    assert len(names) >= 8
    for n in names:
        x, w, dy = d[f"{n}/x"], d[f"{n}/w"], d[f"{n}/dy"]
        K = w.shape[1]
        assert oracle.normalized_max_abs(oracle.fwd_f64(x, w), d[f"{n}/y64"]) < 1e-12, n
        assert oracle.normalized_max_abs(oracle.dx_f64(dy, w), d[f"{n}/dx64"]) < 1e-12, n
        assert oracle.normalized_max_abs(oracle.dk_f64(dy, x, K), d[f"{n}/dk64"]) < 1e-12, n


def test_torch_library_agreement_random_shapes():
    rng = np.random.default_rng(7)
    for _ in range(12):
        B = int(rng.integers(1, 6))
        H = int(rng.integers(1, 7))
        L = int(rng.integers(1, 49))
        K = int(rng.integers(1, 49))
        x, w, dy = oracle.make_inputs(B, H, L, K, seed=int(rng.integers(1 << 30)))
        y64, dx64, dk64 = oracle.torch_grads(x.double(), w.double(), dy.double())
        assert oracle.normalized_max_abs(oracle.fwd_f64(x, w), _np(y64)) < 1e-12
        assert oracle.normalized_max_abs(oracle.dx_f64(dy, w), _np(dx64)) < 1e-12
        assert oracle.normalized_max_abs(oracle.dk_f64(dy, x, K), _np(dk64)) < 1e-12
        # The reference's other PyTorch form (symmetric pad + crop) is the same op.
        yr = oracle.reference_depthwise_conv(x.double(), w.double())
        assert oracle.normalized_max_abs(_np(yr), _np(y64)) < 1e-14


# ---------------------------------------------------------------------------
# Brute force and fsum
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("shape", [(2, 3, 5, 9), (3, 2, 11, 4), (1, 1, 1, 1), (2, 2, 8, 3)])
def test_brute_force(shape):
    B, H, L, K = shape
    x, w, dy = (_np(t) for t in oracle.make_inputs(B, H, L, K, seed=11))
    assert np.array_equal(oracle.fwd_f64(x, w), oracle.brute_fwd(x, w))
    assert np.array_equal(oracle.dx_f64(dy, w), oracle.brute_dx(dy, w))
    assert oracle.normalized_max_abs(oracle.dk_f64(dy, x, K), oracle.brute_dk(dy, x, K)) < 1e-14


def test_dk_fsum_coefficients():
    B, H, L, K = 16, 3, 48, 47
    x, w, dy = (_np(t) for t in oracle.make_inputs(B, H, L, K, seed=5))
    dk = oracle.dk_f64(dy, x, K)
    scale = np.abs(dk).max()
    for h, j in [(0, 0), (1, 23), (2, 46), (0, 11), (2, 35)]:
        ref = oracle.fsum_dk_coefficient(dy, x, K, h, j)
        assert abs(dk[h, j] - ref) <= 1e-13 * scale


# ---------------------------------------------------------------------------
# Closed forms
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("L,K", [(48, 48), (48, 47), (16, 48), (37, 8), (5, 9), (1, 3)])
def test_delta_and_shift_taps(L, K):
    B, H = 3, 2
    x, _, dy = (_np(t) for t in oracle.make_inputs(B, H, L, K, seed=3))
    p = K // 2
    for j in range(K):
        w = np.zeros((H, K), dtype=np.float32)
        w[:, j] = 1.0
        s = j - p  # y[t] = x[t + s]
        expect = np.zeros_like(x)
        for t in range(L):
            if 0 <= t + s < L:
                expect[..., t] = x[..., t + s]
        assert np.array_equal(oracle.fwd_f32_refchain(x, w), expect)
        assert np.array_equal(oracle.fwd_f64(x, w), expect.astype(np.float64))
        # DX is the transpose: dx[s'] = dy[s' - s].
        expect_dx = np.zeros_like(dy)
        for t in range(L):
            if 0 <= t - s < L:
                expect_dx[..., t] = dy[..., t - s]
        assert np.array_equal(oracle.dx_f32_refchain(dy, w), expect_dx)


def test_k1_and_l1():
    x, w, dy = (_np(t) for t in oracle.make_inputs(4, 3, 12, 1, seed=9))
    assert np.array_equal(oracle.fwd_f32_refchain(x, w), x * w[None, :, 0:1])
    assert np.array_equal(oracle.dx_f32_refchain(dy, w), dy * w[None, :, 0:1])
    assert np.allclose(oracle.dk_f64(dy, x, 1)[:, 0], (dy.astype(np.float64) * x).sum(axis=(0, 2)), rtol=1e-13)
    x, w, dy = (_np(t) for t in oracle.make_inputs(4, 3, 1, 5, seed=10))
    p = 5 // 2
    assert np.array_equal(oracle.fwd_f32_refchain(x, w), x * w[None, :, p:p + 1])
    dk = oracle.dk_f64(dy, x, 5)
    assert np.all(dk[:, [0, 1, 3, 4]] == 0.0)


def test_linearity_and_adjoint():
    B, H, L, K = 5, 4, 48, 48
    x1, w, dy = (_np(t) for t in oracle.make_inputs(B, H, L, K, seed=21))
    x2 = _np(oracle.make_inputs(B, H, L, K, seed=22)[0])
    a, b = 0.75, -1.5
    lhs = oracle.fwd_f64(a * x1.astype(np.float64) + b * x2, w)
    # fwd_f64 takes float32 inputs: use exactly representable combinations.
    xs = (np.float32(a) * x1 + np.float32(b) * x2).astype(np.float32)
    lhs = oracle.fwd_f64(xs, w)
    rhs = a * oracle.fwd_f64(x1, w) + b * oracle.fwd_f64(x2, w)
    assert oracle.normalized_max_abs(lhs, rhs) < 1e-6  # xs itself is rounded
    # <FWD(x), dY> == <x, DX(dY)> exactly up to FP64 summation error.
    left = float(np.sum(oracle.fwd_f64(x1, w) * dy.astype(np.float64)))
    right = float(np.sum(x1.astype(np.float64) * oracle.dx_f64(dy, w)))
    assert abs(left - right) <= 1e-12 * max(abs(left), 1.0) * 100
    # <FWD(x), dY> == sum_j w[h,j] dK[h,j]  (dK is the gradient w.r.t. w).
    dk = oracle.dk_f64(dy, x1, K)
    assert abs(left - float(np.sum(dk * w.astype(np.float64)))) <= 1e-10 * abs(left)


def test_dk_equals_sum_of_fwd_with_delta_taps():
    B, H, L, K = 6, 3, 20, 9
    x, _, dy = (_np(t) for t in oracle.make_inputs(B, H, L, K, seed=33))
    dk = oracle.dk_f64(dy, x, K)
    for j in range(K):
        e = np.zeros((H, K), dtype=np.float32)
        e[:, j] = 1.0
        yj = oracle.fwd_f64(x, e)  # y_j[t] = x[t + j - p]
        col = (yj * dy.astype(np.float64)).sum(axis=(0, 2))
        assert np.allclose(dk[:, j], col, rtol=1e-12, atol=1e-12)


def test_dk_zero_overlap_taps_are_exactly_zero():
    L, K = 16, 48
    x, _, dy = (_np(t) for t in oracle.make_inputs(4, 3, L, K, seed=44))
    dk = oracle.dk_f64(dy, x, K)
    for j in range(K):
        lo, hi = oracle.valid_tap_range(L, K, j)
        if hi <= lo:
            assert np.all(dk[:, j] == 0.0), j
        else:
            assert np.all(dk[:, j] != 0.0), j
    empty = [j for j in range(K) if oracle.valid_tap_range(L, K, j)[1] <= oracle.valid_tap_range(L, K, j)[0]]
    assert empty == list(range(0, 9)) + list(range(40, 48))


def test_useful_fma_counts():
    # Primary shape: 7.248 GFLOP of useful work (2 flops per FMA) per path.
    per_row = oracle.useful_fma_per_row(48, 48)
    assert per_row == 1728
    assert 2 * 16384 * 128 * per_row == 7_247_757_312
    assert oracle.useful_fma_per_row(48, 4) == 4 * 48 - (2 + 1) - 1  # taps 0,1 lose 2,1; tap 3 loses 1
    # Closed form: a row of length L and a K-tap window with L >= K.
    for L, K in [(48, 8), (32, 16), (40, 3)]:
        p = K // 2
        assert oracle.useful_fma_per_row(L, K) == L * K - p * (p + 1) // 2 - (K - 1 - p) * (K - p) // 2


def test_rejects_out_of_range():
    """The FP64 sums serve L, K <= 256; beyond that, and for L or K < 1, the
    oracle refuses the shape."""
    x = np.zeros((1, 1, 257), dtype=np.float32)
    with pytest.raises(ValueError):
        oracle.fwd_f64(x, np.zeros((1, 3), dtype=np.float32))
    with pytest.raises(ValueError):
        oracle.fwd_f64(np.zeros((1, 1, 8), dtype=np.float32), np.zeros((1, 257), dtype=np.float32))
    with pytest.raises(ValueError):
        oracle.dk_f64(np.zeros((1, 1, 8), dtype=np.float32), np.zeros((1, 1, 8), dtype=np.float32), 0)


# ---------------------------------------------------------------------------
# Planted mistakes: each must be rejected by at least one of the pins above.
# ---------------------------------------------------------------------------
def _conv_np(x, w, *, pad=None, flip=False, drop_last=False, adjoint=False):
    x = x.astype(np.float64)
    w = w.astype(np.float64)
    B, H, L = x.shape
    K = w.shape[1]
    p = K // 2 if pad is None else pad
    if flip:
        w = w[:, ::-1]
    out = np.zeros_like(x)
    for j in range(K - (1 if drop_last else 0)):
        s = (p - j) if adjoint else (j - p)
        lo, hi = max(0, -s), min(L, L - s)
        if hi > lo:
            out[..., lo:hi] += w[None, :, j:j + 1] * x[..., lo + s:hi + s]
    return out


MUTANTS = {
    "symmetric_pad": dict(pad="sym"),
    "flipped_taps": dict(flip=True),
    "dropped_last_tap": dict(drop_last=True),
    "dx_sign": dict(adjoint_sign=True),
}


@pytest.mark.parametrize("name", sorted(MUTANTS))
def test_mutants_are_caught(name):
    B, H, L, K = 3, 2, 12, 6
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=77)
    xn, wn, dyn = _np(x), _np(w), _np(dy)
    y64, dx64, _ = oracle.torch_grads(x.double(), w.double(), dy.double())
    good_fwd = _conv_np(xn, wn)
    good_dx = _conv_np(dyn, wn, adjoint=True)
    assert oracle.normalized_max_abs(good_fwd, _np(y64)) < 1e-12
    assert oracle.normalized_max_abs(good_dx, _np(dx64)) < 1e-12
    m = MUTANTS[name]
    if "adjoint_sign" in m:
        bad_dx = _conv_np(dyn, wn, adjoint=False)
        left = float(np.sum(good_fwd * dyn))
        right = float(np.sum(xn.astype(np.float64) * bad_dx))
        assert abs(left - right) > 1e-6 * abs(left)  # adjoint identity fails
        assert oracle.normalized_max_abs(bad_dx, _np(dx64)) > 1e-3
        return
    kw = dict(m)
    if kw.get("pad") == "sym":
        kw["pad"] = (K - 1) // 2
    bad = _conv_np(xn, wn, **kw)
    assert oracle.normalized_max_abs(bad, _np(y64)) > 1e-3  # library check fails
    # and the delta-tap closed form fails as well for the index mistakes
    if name in ("symmetric_pad", "flipped_taps"):
        e = np.zeros((H, K), dtype=np.float32)
        e[:, 0] = 1.0
        assert not np.array_equal(_conv_np(xn, e, **kw), oracle.fwd_f64(xn, e))


@pytest.mark.parametrize("L,K", [(192, 192), (100, 37), (64, 256), (200, 256), (1, 256), (49, 49)])
def test_fp64_sums_on_long_rows_match_numpy_correlate(L, K):
    """The FP64 sums on long rows (L, K up to 256, the reference's
    kernels/shared_l192.py regime) against numpy.correlate, a library
    routine independent of the oracle's loops:
    FWD y[t] = corr(pad(x, (p, K-1-p)), w)[t]; dX dx[s] = corr(pad(dy,
    (K-1-p, p)), w[::-1])[s]; dK dk[j] = sum_b corr(pad(x, (p, K-1-p)),
    dy)[j]."""
    B, H = 3, 2
    g = np.random.default_rng(L * 1000 + K)
    x = g.standard_normal((B, H, L)).astype(np.float32)
    dy = g.standard_normal((B, H, L)).astype(np.float32)
    w = g.standard_normal((H, K)).astype(np.float32)
    p = K // 2
    y_ref = np.empty((B, H, L))
    dx_ref = np.empty((B, H, L))
    dk_ref = np.zeros((H, K))
    for b in range(B):
        for h in range(H):
            xp = np.pad(x[b, h].astype(np.float64), (p, K - 1 - p))
            y_ref[b, h] = np.correlate(xp, w[h].astype(np.float64), "valid")
            dyp = np.pad(dy[b, h].astype(np.float64), (K - 1 - p, p))
            dx_ref[b, h] = np.correlate(dyp, w[h, ::-1].astype(np.float64), "valid")
            dk_ref[h] += np.correlate(xp, dy[b, h].astype(np.float64), "valid")
    scale = lambda a: np.abs(a).max() + 1.0  # noqa: E731
    np.testing.assert_allclose(oracle.fwd_f64(x, w), y_ref, rtol=0, atol=1e-12 * scale(y_ref))
    np.testing.assert_allclose(oracle.dx_f64(dy, w), dx_ref, rtol=0, atol=1e-12 * scale(dx_ref))
    np.testing.assert_allclose(oracle.dk_f64(dy, x, K), dk_ref, rtol=0, atol=1e-12 * scale(dk_ref))


def test_reference_chains_keep_the_reference_kernel_range():
    """The FP32 fmaf chains restate kernels limited to L, K <= 48
    (kernels/warp_tiled_ampere.py:715-716) and refuse longer rows."""
    x = np.zeros((1, 1, 49), dtype=np.float32)
    with pytest.raises(ValueError, match="<= 48"):
        oracle.fwd_f32_refchain(x, np.zeros((1, 3), dtype=np.float32))
    with pytest.raises(ValueError, match="<= 48"):
        oracle.dx_f32_refchain(x[:, :, :8], np.zeros((1, 49), dtype=np.float32))
    with pytest.raises(ValueError, match="<= 256"):
        oracle.fwd_f64(np.zeros((1, 1, 257), dtype=np.float32), np.zeros((1, 3), dtype=np.float32))
