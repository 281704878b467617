"""GPU parity of the HIP kernels against the CPU oracle (marked ``gpu``).

Bars (stated per test):
* FWD / dX, VALU kernel (PATHTILE_ROWS_ALGO=valu, and every shape the
  matrix-core kernel does not serve): bit-exact against the oracle's
  restatement of the reference's FP32 fmaf chain (oracle.fwd_f32_refchain /
  dx_f32_refchain) and within 1e-5 max-abs-scaled of FP64;
* FWD / dX, channel-group matrix-core kernel (the default for long FMA
  chains with H % 8 == 0 and 16-byte aligned tensors, any L): within 1e-5
  max-abs-scaled of FP64 (the matrix cores sum in their own order);
* dK (atomic and deterministic): within 1e-4 max-abs-scaled of FP64
  (atomic order is not fixed); the deterministic variant is also bitwise
  reproducible run to run; taps that meet no element are exactly 0.
Large shapes are checked on sampled batch rows (FWD/dX) and in full (dK).
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from pathtile_amd import rows_rule
from pathtile_amd import runtime as _runtime

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-5
DK_TOL = 1e-4


@pytest.fixture(scope="module")
def rt():
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime()
    yield r
    r.close()


def _dev(*ts):
    return [t.to("cuda:0") for t in ts]


def _inputs(B, H, L, K, seed):
    print(f"[case] B={B} H={H} L={L} K={K} seed={seed}", flush=True)
    return oracle.make_inputs(B, H, L, K, seed)


def _fwd(rt, x, w):
    y = torch.empty_like(x)
    rt.launch_fwd(x, w, y)
    return y


def _dx(rt, dy, w):
    dx = torch.empty_like(dy)
    rt.launch_bwd_input(dy, w, dx)
    return dx


def _dk_atomic(rt, dy, x, K, zero_first=True):
    gk = torch.full((x.shape[1], K), float("nan"), device=x.device) if zero_first \
        else torch.zeros((x.shape[1], K), device=x.device)
    rt.launch_bwd_weight(dy, x, gk, K, zero_first=zero_first)
    return gk


def _dk_det(rt, dy, x, K):
    gk = torch.full((x.shape[1], K), float("nan"), device=x.device)
    rt.launch_bwd_weight_deterministic(dy, x, gk, K)
    return gk


SHAPES = [
    (64, 16, 48, 48),     # C1
    (1000, 96, 37, 48),   # E1: B not a multiple of 64, K > L, L % 4 != 0
    (300, 16, 48, 47),    # odd K (E2 family)
    (257, 8, 48, 4),      # short filter (S family)
    (70, 5, 16, 48),      # K > L, zero-overlap taps
    (3, 7, 1, 5),         # L = 1
    (65, 3, 17, 13),      # reference dK edge case (benchmark_dk_packing.py:276-289)
    (1, 1, 1, 1),         # reference dK edge case
    (33, 9, 24, 8),
    (128, 64, 32, 32),
    (40, 4, 40, 24),
    (17, 2, 8, 3),
    (5, 3, 48, 1),
    (129, 2, 45, 40),
    (64, 128, 48, 48),
    (8000, 64, 48, 48),   # several tiles per wave, ragged last chunk group
    (8000, 64, 37, 8),    # same, dword row path
    # rows of 16 and 20-28 columns below 256 MiB: the matrix cores from
    # 9.5 x 16 (L = 16) and 12.5 L (L = 20-28) useful FMAs per row
    (64, 32, 24, 16),     # 320 >= 300: matrix cores
    (40, 8, 24, 14),      # 287 < 300: VALU, bit-exact
    (50, 16, 20, 24),     # 336 >= 250: matrix cores
    (33, 8, 16, 12),      # 156 >= 152: matrix cores
    (33, 8, 16, 10),      # 135 < 152: VALU, bit-exact
]


def _mfma_serves(B, H, L, K, algo):
    """Whether the channel-group matrix-core FWD/DX kernel serves a 16-byte
    aligned call: the layout must allow it (H % 8 == 0, any L) and, unless
    forced, the library's dispatch must pick it (pt_rows_kernel_id)."""
    if algo in ("valu", "tile", "stream") or H % 8:
        return False
    if algo == "mfma":
        return True
    return _runtime.rows_on_matrix_cores(B, H, L, K)


@pytest.mark.parametrize("algo", ["auto", "valu", "tile", "stream", "mfma"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_fwd_dx_bit_exact_and_fp64(rt, shape, algo, monkeypatch):
    """Both FWD/DX kernels; the library reads PATHTILE_ROWS_ALGO on every
    call. The VALU kernel is bit-exact with the reference's fmaf chain."""
    if algo != "auto":
        monkeypatch.setenv("PATHTILE_ROWS_ALGO", algo)
    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=1000 + B + H + L + K)
    xd, wd, dyd = _dev(x, w, dy)
    y = _fwd(rt, xd, wd).cpu().numpy()
    dx = _dx(rt, dyd, wd).cpu().numpy()
    assert np.isfinite(y).all() and np.isfinite(dx).all()
    if not _mfma_serves(B, H, L, K, algo):
        y_ref = oracle.fwd_f32_refchain(x, w)
        dx_ref = oracle.dx_f32_refchain(dy, w)
        assert np.array_equal(y, y_ref), oracle.normalized_max_abs(y, y_ref)
        assert np.array_equal(dx, dx_ref), oracle.normalized_max_abs(dx, dx_ref)
    assert oracle.normalized_max_abs(y, oracle.fwd_f64(x, w)) < FWD_TOL
    assert oracle.normalized_max_abs(dx, oracle.dx_f64(dy, w)) < FWD_TOL


@pytest.mark.parametrize("shape", [
    (1, 8, 48, 48),       # one sample: a single ragged 16-sample step
    (15, 16, 44, 48),     # L < row bucket (48): columns of the next channel masked
    (33, 8, 36, 32),      # L in the 48 bucket, ragged last step
    (100, 24, 20, 17),    # L in the 32 bucket, odd K
    (77, 8, 12, 40),      # K > L
    (50, 16, 4, 9),       # L = 4: three quarters of each MFMA input masked
    (513, 8, 8, 3),       # short filter, forced onto the matrix cores
    (4096, 8, 48, 48),    # one channel group, many interleaved ranges
    (40, 4800, 16, 16),   # 600 channel groups, more than two per CU: one range each
    # rows of 33-48 columns, H % 16 == 0: the 16-channel workgroups (one input
    # stage) where forced or the call is large
    (1, 16, 48, 48),      # a single ragged step
    (33, 32, 36, 32),     # L below the bucket, ragged last step
    (4096, 16, 48, 48),   # one channel group, many interleaved ranges
    (100, 48, 40, 24),    # three channel groups, odd-ish K
    (257, 16, 44, 47),    # odd K, ragged
    # rows that are not whole float4s (L % 4 != 0): element-wise LDS operands
    (1, 8, 37, 48),       # a single ragged step
    (1000, 96, 37, 48),   # E1, ragged last step
    (33, 16, 45, 40),     # L three short of the bucket
    (100, 8, 31, 16),     # 32 bucket
    (50, 8, 13, 9),       # 16 bucket
    (77, 24, 5, 7),       # L = 5: a row ends inside the first float4 of the next
    (20, 8, 1, 1),        # L = 1
    (100, 8, 2, 5),       # L = 2, K > L
    (33, 16, 3, 48),      # L = 3, K far above L
    (64, 24, 7, 7),
])
@pytest.mark.parametrize("channels", ["auto", "8", "16"])
def test_fwd_dx_matrix_core_kernel(rt, shape, channels, monkeypatch):
    """The channel-group matrix-core kernel (forced) against FP64 on the
    layouts it serves, with infinities in the next channel's rows: its
    masked columns must not leak into this channel's outputs. channels:
    the library's choice, or 8 / 16 channels per workgroup forced
    (PATHTILE_ROWS_CHANNELS; 16 needs rows of 33-48 columns and H % 16 == 0,
    else the library keeps 8)."""
    monkeypatch.setenv("PATHTILE_ROWS_ALGO", "mfma")
    if channels != "auto":
        monkeypatch.setenv("PATHTILE_ROWS_CHANNELS", channels)
    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=4000 + B + H + L + K)
    x[:, 1::2, :] = float("inf")
    dy[:, 1::2, :] = float("inf")
    xd, wd, dyd = _dev(x, w, dy)
    y = _fwd(rt, xd, wd).cpu().numpy()[:, 0::2]
    dx = _dx(rt, dyd, wd).cpu().numpy()[:, 0::2]
    xe, we, dye = x[:, 0::2].contiguous(), w[0::2].contiguous(), dy[:, 0::2].contiguous()
    assert np.isfinite(y).all() and np.isfinite(dx).all()
    assert oracle.normalized_max_abs(y, oracle.fwd_f64(xe, we)) < FWD_TOL
    assert oracle.normalized_max_abs(dx, oracle.dx_f64(dye, we)) < FWD_TOL


def _same_bits_or_both_nan(a, b):
    return bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))


@pytest.mark.parametrize("algo", ["auto", "valu", "tile", "stream", "mfma"])
@pytest.mark.parametrize("shape", [
    (64, 16, 48, 48),     # C1: the matrix-core kernel by default
    (40, 8, 44, 48),      # L < row bucket
    (33, 8, 32, 17),      # 32 bucket, ragged last step
    (50, 16, 48, 4),      # short filter (VALU by default, matrix cores forced)
    (40, 8, 37, 48),      # L % 4 != 0 (the matrix-core kernel's element-wise form)
    (33, 16, 45, 32),     # same, H % 16 == 0
])
@pytest.mark.parametrize("channels", ["auto", "16"])
def test_nonfinite_values_reach_only_the_reference_window(rt, shape, algo, channels, monkeypatch):
    """Inf, -Inf and NaN in x / dY (same channel as finite rows) and in one
    channel's taps. The reference's fmaf chain touches an element only
    through the taps whose window holds it (kernels/warp_tiled_ampere.py:
    411-430, 479-498), so non-finite values reach exactly the outputs in that
    window. On every kernel: every row with a non-finite input equals the
    oracle's FP32 chain bit for bit (NaN where it has NaN); in the channel
    with the non-finite tap, the non-finite outputs are exactly the chain's
    (same NaN positions, same signed infinities) and the finite ones within
    1e-5 of it; every other row stays within 1e-5 of FP64."""
    if algo != "auto":
        monkeypatch.setenv("PATHTILE_ROWS_ALGO", algo)
    if channels != "auto":
        monkeypatch.setenv("PATHTILE_ROWS_CHANNELS", channels)
    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=6000 + B + H + L + K)
    rng = np.random.default_rng(B + L + K)
    bad_rows = set()
    for t, v in zip((x, dy), (float("inf"), float("nan"))):
        for val in (v, -float("inf"), float("nan")):
            # channels other than hb, the one that gets a non-finite tap
            b, h, s = int(rng.integers(B)), int(rng.integers(H - 1)), int(rng.integers(L))
            t[b, h, s] = val
            bad_rows.add((b, h))
    hb = H - 1
    w[hb, K // 3] = float("inf")
    xd, wd, dyd = _dev(x, w, dy)
    y = _fwd(rt, xd, wd).cpu().numpy()
    dx = _dx(rt, dyd, wd).cpu().numpy()
    y_ref, dx_ref = oracle.fwd_f32_refchain(x, w), oracle.dx_f32_refchain(dy, w)
    for got, ref, src in ((y, y_ref, x), (dx, dx_ref, dy)):
        exact = ~np.isfinite(src.numpy()).all(axis=2)
        exact[:, hb] = False
        assert exact.sum() >= 2
        assert _same_bits_or_both_nan(got[exact], ref[exact])
        gc, rc = got[:, hb], ref[:, hb]
        assert np.array_equal(np.isnan(gc), np.isnan(rc))
        assert np.array_equal(np.where(np.isinf(gc), gc, 0), np.where(np.isinf(rc), rc, 0))
        fr = np.isfinite(rc)
        assert fr.any() and (~fr).any()
        assert oracle.normalized_max_abs(gc[fr], rc[fr]) < FWD_TOL
        other = ~exact
        other[:, hb] = False
        assert np.isfinite(got[other]).all()
    fin = np.ones((B, H), dtype=bool)
    fin[:, hb] = False
    for b, h in bad_rows:
        fin[b, h] = False
    xs = x.clone(); xs[~torch.from_numpy(fin)] = 0.0
    dys = dy.clone(); dys[~torch.from_numpy(fin)] = 0.0
    ws = w.clone(); ws[hb] = 0.0
    assert oracle.normalized_max_abs(y[fin], oracle.fwd_f64(xs, ws)[fin]) < FWD_TOL
    assert oracle.normalized_max_abs(dx[fin], oracle.dx_f64(dys, ws)[fin]) < FWD_TOL


def _sprinkle_nonfinite(t, n, seed):
    """n non-finite values (Inf, -Inf, NaN in turn) at seeded positions."""
    rng = np.random.default_rng(seed)
    flat = t.view(-1)
    for i, pos in enumerate(rng.integers(0, flat.numel(), size=n)):
        flat[int(pos)] = (float("inf"), -float("inf"), float("nan"))[i % 3]


STREAM_SHAPES = [
    (3, 1, 4, None),        # L = 4: every neighbour float4 is another row
    (70, 5, 16, None),      # one partial span
    (257, 8, 48, None),     # S family
    (33, 9, 24, None),
    (100, 131, 44, None),   # H prime: a channel period of 1441 float4s
    (40, 3, 12, None),      # period of 9 float4s, many per span
]


@pytest.mark.parametrize("K", list(range(1, 10)))
@pytest.mark.parametrize("shape", STREAM_SHAPES, ids=lambda s: "B{}H{}L{}".format(*s[:3]))
def test_stream_kernel_is_the_reference_chain_for_any_values(rt, shape, K, monkeypatch):
    """The short-tap streaming kernel (forced; K <= 9, L % 4 == 0): its
    neighbour float4s come from other lanes, other registers and the span's
    halo loads, and the terms that reach past the row are skipped, so every
    output is the reference's fmaf chain bit for bit, non-finite inputs and
    taps included (NaN where the chain gives NaN)."""
    monkeypatch.setenv("PATHTILE_ROWS_ALGO", "stream")
    B, H, L, _ = shape
    x, w, dy = _inputs(B, H, L, K, seed=9000 + B + H + L + K)
    _sprinkle_nonfinite(x, 5, seed=K)
    _sprinkle_nonfinite(dy, 5, seed=K + 50)
    w[H // 2, (K - 1) // 2] = float("inf")
    xd, wd, dyd = _dev(x, w, dy)
    y = _fwd(rt, xd, wd).cpu().numpy()
    dx = _dx(rt, dyd, wd).cpu().numpy()
    assert _same_bits_or_both_nan(y, oracle.fwd_f32_refchain(x, w))
    assert _same_bits_or_both_nan(dx, oracle.dx_f32_refchain(dy, w))


@pytest.mark.parametrize("K", [1, 4, 9])
@pytest.mark.parametrize("shape", [
    (2048, 256, 48),   # S family: 6144 spans, a 12-wave channel period, several spans per wave
    (2000, 131, 44),   # H prime: more workgroups than fit at once
    (9000, 37, 32),    # period of 296 float4s
], ids=lambda s: "B{}H{}L{}".format(*s))
def test_stream_kernel_multi_span_grids(rt, shape, K, monkeypatch):
    """Grids whose waves take several spans: every lane keeps its column and
    channel from span to span (the grid advances by whole channel periods),
    so the outputs are still the reference's chain bit for bit."""
    monkeypatch.setenv("PATHTILE_ROWS_ALGO", "stream")
    B, H, L = shape
    x, w, dy = _inputs(B, H, L, K, seed=9500 + B + H + L + K)
    xd, wd, dyd = _dev(x, w, dy)
    assert np.array_equal(_fwd(rt, xd, wd).cpu().numpy(), oracle.fwd_f32_refchain(x, w))
    assert np.array_equal(_dx(rt, dyd, wd).cpu().numpy(), oracle.dx_f32_refchain(dy, w))


@pytest.mark.parametrize("wpb,L", [(1, 48), (2, 48), (4, 48), (8, 48), (16, 32)])
@pytest.mark.parametrize("algo", ["stream", "valu"])
def test_stream_kernel_every_waves_per_block(wpb, L, algo, monkeypatch):
    """Every waves_per_block gives the reference's bits on the streaming
    kernel (forced) and on the VALU choice at H = 131, whose channel period
    idles a quarter or more of the tile kernel's grid at some waves per
    block (there the streaming kernel serves) and less at others."""
    from pathtile_amd import runtime

    monkeypatch.setenv("PATHTILE_ROWS_ALGO", algo)
    B, H, K = 1500, 131, 5
    x, w, dy = _inputs(B, H, L, K, seed=31 + wpb)
    xd, wd, dyd = _dev(x, w, dy)
    r = runtime.HipWarpRuntime(waves_per_block=wpb, dx_waves_per_block=wpb)
    assert np.array_equal(_fwd(r, xd, wd).cpu().numpy(), oracle.fwd_f32_refchain(x, w))
    assert np.array_equal(_dx(r, dyd, wd).cpu().numpy(), oracle.dx_f32_refchain(dy, w))


@pytest.mark.parametrize("algo", ["auto", "valu", "mfma"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_dk_atomic_and_deterministic(rt, shape, algo, monkeypatch):
    """Both DK algorithms (VALU lane-per-row and matrix-core batch GEMM);
    the library reads PATHTILE_DK_ALGO on every call."""
    if algo != "auto":
        monkeypatch.setenv("PATHTILE_DK_ALGO", algo)
    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=2000 + B + H + L + K)
    xd, dyd = _dev(x, dy)
    ref = oracle.dk_f64(dy, x, K)
    ga = _dk_atomic(rt, dyd, xd, K).cpu().numpy()
    gd1 = _dk_det(rt, dyd, xd, K).cpu().numpy()
    gd2 = _dk_det(rt, dyd, xd, K).cpu().numpy()
    assert np.isfinite(ga).all() and np.isfinite(gd1).all()
    assert oracle.normalized_max_abs(ga, ref) < DK_TOL
    assert oracle.normalized_max_abs(gd1, ref) < DK_TOL
    assert np.array_equal(gd1, gd2)  # run-to-run bitwise
    for j in range(K):
        lo, hi = oracle.valid_tap_range(L, K, j)
        if hi <= lo:
            assert np.all(ga[:, j] == 0.0) and np.all(gd1[:, j] == 0.0)


def _misaligned(t):
    """Same values, 4-byte but not 16-byte aligned storage."""
    flat = torch.zeros(t.numel() + 1, device="cuda:0")
    flat[1:] = t.reshape(-1).to("cuda:0")
    v = flat[1:].view(t.shape)
    assert v.data_ptr() % 16 != 0
    return v


STAGING_SHAPES = [
    (1001, 64, 48, 3),    # ragged last 4-sample step, K = 3 (coalesced atomics)
    (5, 32, 40, 24),      # fewer steps than interleaved ranges, L < bucket
    (2048, 128, 20, 9),   # L in the 32 bucket, odd K
    (4099, 16, 16, 48),   # K > L: zero-overlap taps
    (1001, 64, 37, 3),    # L % 4 != 0: dword staging whatever the alignment
    (777, 32, 45, 48),    # same, L three short of the bucket
    (300, 16, 29, 16),    # same, 32 bucket
    (500, 12, 30, 9),     # L % 4 == 2: whole chunks where the group is even
    (64, 96, 13, 5),      # 16 bucket, odd L
    (100, 16, 1, 3),      # L = 1: one column per row
    (70, 32, 2, 5),       # L = 2, K > L: taps without overlap
    (33, 16, 3, 48),      # L = 3
    (129, 64, 7, 7),
]
# (shape, threads) where H is a multiple of the channel group (one channel
# per wave for rows of 33-48 columns, two below): the cases the channel-group
# kernel serves.
STAGING_CASES = [(s, t) for s in STAGING_SHAPES for t in (64, 128, 256, 512)
                 if s[1] % ((1 if s[2] > 32 else 2) * (t // 64)) == 0]


@pytest.mark.parametrize("shape,threads", STAGING_CASES,
                         ids=lambda v: "B{}H{}L{}K{}".format(*v) if isinstance(v, tuple) else str(v))
def test_dk_channel_group_staging_widths(shape, threads):
    """Where H is a multiple of the channel group (one channel per wave for
    rows of 33-48 columns, two below; at most 8 waves) the channel-group
    kernel serves any L: 16-byte chunk staging for 16-byte aligned tensors
    whose group segments and samples are whole chunks, dword staging
    otherwise (odd L, or the same values in misaligned storage). These
    shapes take fewer workgroups than one resident round, so the range count
    (and with it the partition of the deterministic sums) comes from the
    shape alone and the deterministic results of the two stagings are
    bitwise equal; both agree with FP64 and repeat bit for bit with the
    workspace the API sizes. (Where one round caps the range count, the two
    staging kernels' occupancies can cap it differently:
    test_dk_capped_grid_repeats_per_alignment.)"""
    from pathtile_amd import runtime

    B, H, L, K = shape
    x, w, dy = _inputs(B, H, L, K, seed=3000 + B + L + K)
    xd, dyd = _dev(x, dy)
    xm, dym = _misaligned(x), _misaligned(dy)
    ref = oracle.dk_f64(dy, x, K)
    r = runtime.HipWarpRuntime(bwdk_block=threads)
    dets = []
    for a, b in ((dyd, xd), (dym, xm)):
        ga = _dk_atomic(r, a, b, K).cpu().numpy()
        g1 = _dk_det(r, a, b, K).cpu().numpy()
        g2 = _dk_det(r, a, b, K).cpu().numpy()
        assert oracle.normalized_max_abs(ga, ref) < DK_TOL
        assert oracle.normalized_max_abs(g1, ref) < DK_TOL
        assert np.array_equal(g1, g2)
        dets.append(g1)
        for j in range(K):
            lo, hi = oracle.valid_tap_range(L, K, j)
            if hi <= lo:
                assert np.all(ga[:, j] == 0.0) and np.all(g1[:, j] == 0.0)
    assert np.array_equal(dets[0], dets[1])
    r.close()


def test_dk_capped_grid_repeats_per_alignment():
    """B16384 H96 L48 K48: the range rule asks for 48 ranges of 48 channel
    groups (2304 workgroups), more than one resident round, so the launch
    caps the range count by the kernel's occupancy, which may differ between
    the 16-byte and the dword staging kernels. Each alignment must still
    repeat its own bits and stay within 1e-4 of FP64."""
    from pathtile_amd import runtime

    B, H, L, K = 16384, 96, 48, 48
    x, w, dy = _inputs(B, H, L, K, seed=3131)
    ref = oracle.dk_f64(dy, x, K)
    r = runtime.HipWarpRuntime(bwdk_block=128)
    for a, b in ((dy.to("cuda:0"), x.to("cuda:0")), (_misaligned(dy), _misaligned(x))):
        g1 = _dk_det(r, a, b, K).cpu().numpy()
        g2 = _dk_det(r, a, b, K).cpu().numpy()
        ga = _dk_atomic(r, a, b, K).cpu().numpy()
        assert np.array_equal(g1, g2)
        assert oracle.normalized_max_abs(g1, ref) < DK_TOL
        assert oracle.normalized_max_abs(ga, ref) < DK_TOL
        del a, b
        torch.cuda.empty_cache()
    r.close()


def test_golden_c1_fixture(rt):
    from pathlib import Path

    d = np.load(Path(__file__).resolve().parent / "golden" / "c1_b64_h16_l48_k48.npz")
    x, w, dy = (torch.from_numpy(d[k]) for k in ("x", "w", "dy"))
    xd, wd, dyd = _dev(x, w, dy)
    K = w.shape[1]
    assert oracle.normalized_max_abs(_fwd(rt, xd, wd).cpu().numpy(), d["y"]) < FWD_TOL
    assert oracle.normalized_max_abs(_dx(rt, dyd, wd).cpu().numpy(), d["dx"]) < FWD_TOL
    assert oracle.normalized_max_abs(_dk_atomic(rt, dyd, xd, K).cpu().numpy(), d["dk64"]) < DK_TOL
    assert oracle.normalized_max_abs(_dk_det(rt, dyd, xd, K).cpu().numpy(), d["dk64"]) < DK_TOL


def test_golden_edge_fixtures(rt):
    from pathlib import Path

    d = np.load(Path(__file__).resolve().parent / "golden" / "edge_cases.npz")
    names = sorted({k.split("/")[0] for k in d.files})
    for n in names:
        print(f"[fixture] {n}", flush=True)
        x, w, dy = (torch.from_numpy(d[f"{n}/{k}"]) for k in ("x", "w", "dy"))
        xd, wd, dyd = _dev(x, w, dy)
        K = w.shape[1]
        assert oracle.normalized_max_abs(_fwd(rt, xd, wd).cpu().numpy(), d[f"{n}/y64"]) < FWD_TOL
        assert oracle.normalized_max_abs(_dx(rt, dyd, wd).cpu().numpy(), d[f"{n}/dx64"]) < FWD_TOL
        assert oracle.normalized_max_abs(_dk_atomic(rt, dyd, xd, K).cpu().numpy(), d[f"{n}/dk64"]) < DK_TOL
        assert oracle.normalized_max_abs(_dk_det(rt, dyd, xd, K).cpu().numpy(), d[f"{n}/dk64"]) < DK_TOL


@pytest.mark.parametrize("algo", ["valu", "auto"])
@pytest.mark.parametrize("wpb,L,H", [(1, 48, 24), (2, 48, 24), (4, 48, 24), (8, 48, 24),
                                     (16, 32, 48), (16, 32, 24), (8, 37, 24), (16, 48, 48)])
def test_every_waves_per_block_gives_the_same_bits(wpb, L, H, algo, monkeypatch):
    """VALU: every waves_per_block reproduces the reference's fmaf chain
    (16 waves do not fit rows above 32: refused). Default: the matrix-core
    kernel (H % 8 == 0, K = 48) runs 8-channel workgroups
    whatever waves_per_block says (16 included, at every L), so every value
    gives the bits of waves_per_block = 1."""
    from pathtile_amd import runtime

    if algo != "auto":
        monkeypatch.setenv("PATHTILE_ROWS_ALGO", algo)
    B, K = 200, 48
    x, w, dy = _inputs(B, H, L, K, seed=7)
    xd, wd, dyd = _dev(x, w, dy)
    r = runtime.HipWarpRuntime(waves_per_block=wpb)
    if wpb == 16 and L > 32 and not _mfma_serves(B, H, L, K, algo):
        with pytest.raises(ValueError, match="unsupported launch configuration"):
            _fwd(r, xd, wd)
        return
    y = _fwd(r, xd, wd).cpu().numpy()
    dx = _dx(r, dyd, wd).cpu().numpy()
    if _mfma_serves(B, H, L, K, algo):
        r1 = runtime.HipWarpRuntime(waves_per_block=1)
        assert np.array_equal(y, _fwd(r1, xd, wd).cpu().numpy())
        assert np.array_equal(dx, _dx(r1, dyd, wd).cpu().numpy())
        assert oracle.normalized_max_abs(y, oracle.fwd_f64(x, w)) < FWD_TOL
        assert oracle.normalized_max_abs(dx, oracle.dx_f64(dy, w)) < FWD_TOL
    else:
        assert np.array_equal(y, oracle.fwd_f32_refchain(x, w))
        assert np.array_equal(dx, oracle.dx_f32_refchain(dy, w))


@pytest.mark.parametrize("threads", [64, 128, 192, 256, 320, 384, 512, 768])
def test_every_dk_block_size(threads):
    from pathtile_amd import runtime

    B, H, L, K = 1000, 12, 48, 48
    x, w, dy = _inputs(B, H, L, K, seed=8)
    xd, dyd = _dev(x, dy)
    ref = oracle.dk_f64(dy, x, K)
    r = runtime.HipWarpRuntime(bwdk_block=threads)
    assert oracle.normalized_max_abs(_dk_atomic(r, dyd, xd, K).cpu().numpy(), ref) < DK_TOL
    g1 = _dk_det(r, dyd, xd, K).cpu().numpy()
    assert oracle.normalized_max_abs(g1, ref) < DK_TOL
    assert np.array_equal(g1, _dk_det(r, dyd, xd, K).cpu().numpy())


def test_oversized_workgroup_is_rejected():
    """H = 4 leaves the VALU kernel, where 16 waves x a 64-row tile at L = 48
    need 213 KiB of LDS: refused before launch with the library's
    configuration error. At H = 8 the matrix-core kernel serves the same
    call (its workgroups are 8 waves whatever waves_per_block says)."""
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime(waves_per_block=16)
    x = torch.zeros(64, 4, 48, device="cuda:0")
    w = torch.zeros(4, 48, device="cuda:0")
    with pytest.raises(ValueError, match="unsupported launch configuration"):
        r.launch_fwd(x, w, torch.empty_like(x))
    x8, w8, _ = _inputs(64, 8, 48, 48, seed=12)
    y8 = _fwd(r, x8.cuda(), w8.cuda()).cpu().numpy()
    assert oracle.normalized_max_abs(y8, oracle.fwd_f64(x8, w8)) < FWD_TOL


def test_atomic_dk_accumulates_into_gk(rt):
    """The reference's contract: the atomic kernel adds into gk
    (kernels/warp_tiled_ampere.py:890-893)."""
    B, H, L, K = 256, 8, 48, 16
    x, w, dy = _inputs(B, H, L, K, seed=9)
    xd, dyd = _dev(x, dy)
    ref = oracle.dk_f64(dy, x, K)
    gk = torch.zeros(H, K, device="cuda:0")
    rt.launch_bwd_weight(dyd, xd, gk, K)
    rt.launch_bwd_weight(dyd, xd, gk, K)
    assert oracle.normalized_max_abs(gk.cpu().numpy(), 2 * ref) < DK_TOL
    rt.launch_bwd_weight(dyd, xd, gk, K, zero_first=True)
    assert oracle.normalized_max_abs(gk.cpu().numpy(), ref) < DK_TOL


def test_primary_shape_sampled_rows_and_full_dk(rt, monkeypatch):
    """B=16384 H=128 L=48 K=48: FWD/dX (matrix-core default) within 1e-5 of
    FP64 on 256 sampled batch rows (all channels), the VALU kernel bit-exact
    on the same rows, dK against FP64 over the full batch."""
    B, H, L, K = 16384, 128, 48, 48
    x, w, dy = _inputs(B, H, L, K, seed=42)
    xd, wd, dyd = _dev(x, w, dy)
    y = _fwd(rt, xd, wd)
    dx = _dx(rt, dyd, wd)
    idx = torch.from_numpy(np.random.default_rng(0).choice(B, 256, replace=False))
    ys, dxs = y[idx.cuda()].cpu().numpy(), dx[idx.cuda()].cpu().numpy()
    assert oracle.normalized_max_abs(ys, oracle.fwd_f64(x[idx], w)) < FWD_TOL
    assert oracle.normalized_max_abs(dxs, oracle.dx_f64(dy[idx], w)) < FWD_TOL
    monkeypatch.setenv("PATHTILE_ROWS_ALGO", "valu")
    yv, dxv = _fwd(rt, xd, wd), _dx(rt, dyd, wd)
    monkeypatch.delenv("PATHTILE_ROWS_ALGO")
    assert np.array_equal(yv[idx.cuda()].cpu().numpy(), oracle.fwd_f32_refchain(x[idx], w))
    assert np.array_equal(dxv[idx.cuda()].cpu().numpy(), oracle.dx_f32_refchain(dy[idx], w))
    del yv, dxv
    ref = oracle.dk_f64(dy, x, K)
    assert oracle.normalized_max_abs(_dk_atomic(rt, dyd, xd, K).cpu().numpy(), ref) < DK_TOL
    g1 = _dk_det(rt, dyd, xd, K).cpu().numpy()
    assert oracle.normalized_max_abs(g1, ref) < DK_TOL
    assert np.array_equal(g1, _dk_det(rt, dyd, xd, K).cpu().numpy())
    # size-independent: the adjoint identity <FWD(x), dY> = <x, DX(dY)> in FP64
    left = float((y.double() * dyd.double()).sum())
    right = float((xd.double() * dx.double()).sum())
    assert abs(left - right) <= 1e-6 * math.sqrt(float((y.double() ** 2).sum()) * float((dyd.double() ** 2).sum()))


def test_misaligned_and_noncontiguous_inputs(rt):
    """A storage offset that breaks 16-byte alignment takes the VALU kernel's
    dword path (the matrix-core kernel needs aligned rows); results stay
    bit-exact."""
    B, H, L, K = 64, 6, 48, 48
    x, w, dy = _inputs(B, H, L, K, seed=10)
    flat = torch.zeros(x.numel() + 1, device="cuda:0")
    flat[1:] = x.reshape(-1).cuda()
    xm = flat[1:].view(B, H, L)  # 4-byte aligned only
    assert xm.data_ptr() % 16 != 0
    y = _fwd(rt, xm, w.cuda()).cpu().numpy()
    assert np.array_equal(y, oracle.fwd_f32_refchain(x, w))


def test_autograd_depthconvampere_and_shared(rt):
    from pathtile_amd import runtime
    from pathtile_amd.kernels import warp_tiled as wt

    runtime.install_runtime(rt)
    B, H, L, K = 96, 10, 48, 48  # H % 8 != 0: the bit-exact VALU kernel
    x, w, dy = _inputs(B, H, L, K, seed=11)
    _, gx_ref, gk_ref = oracle.torch_grads(x.double(), w.double(), dy.double())
    for fn in (runtime.depthwise_conv_ampere, wt.depthwise_conv_shared):
        xd = x.cuda().requires_grad_(True)
        wd = w.cuda().requires_grad_(True)
        y = fn(xd, wd)
        assert np.array_equal(y.detach().cpu().numpy(), oracle.fwd_f32_refchain(x, w))
        gx, gk = torch.autograd.grad(y, (xd, wd), dy.cuda(), retain_graph=True)
        assert oracle.normalized_max_abs(gx.cpu().numpy(), gx_ref.numpy()) < FWD_TOL
        assert oracle.normalized_max_abs(gk.cpu().numpy(), gk_ref.numpy()) < DK_TOL
        # both backward passes take the two-pass dK: reproducible bits
        _, gk2 = torch.autograd.grad(y, (xd, wd), dy.cuda())
        assert torch.equal(gk, gk2)
    wt.reset_timing_collectors()
    xd = x.cuda().requires_grad_(True)
    y = wt.DepthwiseConvShared.apply(xd, w.cuda().requires_grad_(True))
    y.backward(dy.cuda())
    assert len(wt.FWD_TIMES) == len(wt.BWD_IN_TIMES) == len(wt.BWD_K_TIMES) == 1
    assert all(t > 0 for t in wt.FWD_TIMES + wt.BWD_IN_TIMES + wt.BWD_K_TIMES)


def test_api_errors_on_gpu_tensors():
    from pathtile_amd.kernels import warp_tiled as wt

    x = torch.zeros(2, 3, 8, device="cuda:0")
    k = torch.zeros(3, 4, device="cuda:0")
    with pytest.raises(TypeError, match="x must be float32"):
        wt.depthwise_conv_shared(x.double(), k)
    with pytest.raises(TypeError, match="kernel must be float32"):
        wt.depthwise_conv_shared(x, k.double())
    with pytest.raises(ValueError, match=r"x must be \[B,H,L\]"):
        wt.depthwise_conv_shared(x[0], k)
    with pytest.raises(ValueError, match=r"kernel must be \[H,K\]"):
        wt.depthwise_conv_shared(x, k[0])
    with pytest.raises(ValueError, match="Channel mismatch: x H=3, kernel H=2"):
        wt.depthwise_conv_shared(x, k[:2])
    with pytest.raises(ValueError, match="L<=192, K<=256"):
        wt.depthwise_conv_shared(torch.zeros(1, 3, 193, device="cuda:0"), k)


def test_empty_batch(rt):
    x = torch.zeros(0, 4, 16, device="cuda:0")
    w = torch.randn(4, 5, device="cuda:0")
    y = torch.empty_like(x)
    rt.launch_fwd(x, w, y)
    gk = torch.full((4, 5), 7.0, device="cuda:0")
    rt.launch_bwd_weight(x, x, gk, 5, zero_first=True)
    assert torch.all(gk == 0)
    gk.fill_(7.0)
    rt.launch_bwd_weight_deterministic(x, x, gk, 5)
    assert torch.all(gk == 0)


def test_maximum_size_sampled_rows_and_adjoint_identities(rt):
    """B*H*L just under 2^31 (the library's limit; 8.6 GB per tensor):
    FWD/dX within 1e-5 of FP64 on sampled batch rows, dK within 1e-4 of FP64
    on two full channels, and over the whole tensors the size-independent
    identities <FWD(x; w), dY> = <x, DX(dY; w)> = <dK(dY, x), w> in FP64."""
    B, H, L, K = 43690, 1024, 48, 48
    assert B * H * L < 2**31
    print(f"[case] max size B={B} H={H} L={L} K={K}", flush=True)
    g = torch.Generator(device="cuda").manual_seed(77)
    x = torch.randn(B, H, L, device="cuda", generator=g)
    dy = torch.randn(B, H, L, device="cuda", generator=g)
    w = torch.randn(H, K, device="cuda", generator=g) / K ** 0.5
    y = torch.empty_like(x)
    rt.launch_fwd(x, w, y)
    idx = torch.tensor([0, 1, 12345, 30001, B - 2, B - 1], device="cuda")
    xs, ys, dys = x[idx].cpu(), y[idx].cpu().numpy(), dy[idx].cpu()
    wc = w.cpu()
    assert oracle.normalized_max_abs(ys, oracle.fwd_f64(xs, wc)) < FWD_TOL
    left = float((y.double() * dy.double()).sum())
    ynorm = float(y.double().norm())
    del y
    dx = torch.empty_like(x)
    rt.launch_bwd_input(dy, w, dx)
    assert oracle.normalized_max_abs(dx[idx].cpu().numpy(), oracle.dx_f64(dys, wc)) < FWD_TOL
    right = float((x.double() * dx.double()).sum())
    del dx
    gk = torch.empty(H, K, device="cuda")
    rt.launch_bwd_weight_deterministic(dy, x, gk, K)
    dk_w = float((gk.double() * w.double()).sum())
    scale = ynorm * float(dy.double().norm())
    assert abs(left - right) <= 1e-6 * scale
    assert abs(left - dk_w) <= 1e-6 * scale
    for h in (3, H - 1):
        ref = oracle.dk_f64(dy[:, h:h + 1].cpu(), x[:, h:h + 1].cpu(), K)
        assert oracle.normalized_max_abs(gk[h:h + 1].cpu().numpy(), ref) < DK_TOL


def test_resource_report_lists_every_kernel(rt):
    """The reference's resource_report (kernels/warp_tiled_ampere.py:814-833):
    one row per kernel that can serve (L, K), with registers, LDS and an
    occupancy estimate; no kernel spills to scratch."""
    df = rt.resource_report(48, 48)
    assert list(df["kernel"]) == ["fwd", "fwd_matrix_cores", "fwd_matrix_cores_16",
                                  "bwd_input", "bwd_input_matrix_cores",
                                  "bwd_input_matrix_cores_16", "bwd_weight"]
    assert (df["scratch_bytes"] == 0).all()
    df = rt.resource_report(48, 4)
    assert list(df["kernel"]) == ["fwd", "fwd_stream", "fwd_matrix_cores", "fwd_matrix_cores_16",
                                  "bwd_input", "bwd_input_stream", "bwd_input_matrix_cores",
                                  "bwd_input_matrix_cores_16", "bwd_weight"]
    assert (df["scratch_bytes"] == 0).all()
    for L, K, n in ((16, 3, 7), (37, 48, 7), (8, 8, 7), (36, 9, 9)):
        df = rt.resource_report(L, K)
        assert len(df) == n
        assert (df["scratch_bytes"] == 0).all()


@pytest.mark.parametrize("env", [None, "mfma", "valu"])
def test_runtime_rows_algo_overrides_the_environment(env, monkeypatch):
    """HipWarpRuntime(rows_algo=...) picks the FWD/dX kernel per runtime,
    over PATHTILE_ROWS_ALGO: "valu" gives the reference's fmaf chain bit for
    bit where the default takes the matrix cores (C1), "mfma" stays within
    1e-5 of FP64 on a short chain the default leaves to the VALU kernel."""
    from pathtile_amd import runtime

    if env is None:
        monkeypatch.delenv("PATHTILE_ROWS_ALGO", raising=False)
    else:
        monkeypatch.setenv("PATHTILE_ROWS_ALGO", env)
    r_valu = runtime.HipWarpRuntime(rows_algo="valu")
    B, H, L, K = 64, 16, 48, 48
    # the default rule (the environment aside; pinned to the library's
    # dispatch in tests/test_abi_cpu.py)
    assert rows_rule.matrix_cores_serve(B, H, L, K)
    x, w, dy = _inputs(B, H, L, K, seed=31)
    xd, wd, dyd = _dev(x, w, dy)
    assert np.array_equal(_fwd(r_valu, xd, wd).cpu().numpy(), oracle.fwd_f32_refchain(x, w))
    assert np.array_equal(_dx(r_valu, dyd, wd).cpu().numpy(), oracle.dx_f32_refchain(dy, w))
    r_mfma = runtime.HipWarpRuntime(rows_algo="mfma")
    B, H, L, K = 257, 8, 48, 4
    assert not rows_rule.matrix_cores_serve(B, H, L, K)
    x, w, dy = _inputs(B, H, L, K, seed=32)
    xd, wd, dyd = _dev(x, w, dy)
    y = _fwd(r_mfma, xd, wd).cpu().numpy()
    dx = _dx(r_mfma, dyd, wd).cpu().numpy()
    assert oracle.normalized_max_abs(y, oracle.fwd_f64(x, w)) < FWD_TOL
    assert oracle.normalized_max_abs(dx, oracle.dx_f64(dy, w)) < FWD_TOL
    r_valu.close()
    r_mfma.close()
