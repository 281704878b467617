"""GPU parity at every BASELINE configuration's full size, on the reference's
own validation shapes, and on every tuner candidate (marked ``gpu``).

* S  = B32768 H256 L48 K4 (1.6 GB per tensor; the VALU rows kernel, the
  non-temporal channel-group dK) and E2 = B16384 H128 L48 K47 (the
  matrix-core FWD/dX, odd K) at their workload sizes: FWD/dX on sampled batch
  rows (all channels) bit-exact with the oracle's FP32 chain where the VALU
  kernel serves and within 1e-5 max-abs-scaled of FP64 everywhere; the
  atomic and the deterministic dK over the whole batch within 1e-4 of FP64,
  the deterministic one bitwise equal across two runs; and, over the whole
  tensors, the adjoint identities <FWD(x), dY> = <x, DX(dY)> = <dK, w>.
  (P runs at full size in test_gpu_parity.py, E1 at its full size there too.)
* The reference's validation shapes (kernels/warp_tiled_ampere.py:920-926,
  validate/validate_shared.py:236-249), with the reference's w ~ N(0, 1),
  through the autograd functions the reference tests: FWD, dX and dK within
  1e-5 / 1e-5 / 1e-4 of FP64 and within the reference's allclose bars
  (2e-3 / 2e-3, dK atol 1e-2 rtol 5e-4). K = 49 runs the long-row kernels.
* Every (shape, candidate) of the tuner's 30 seeded shapes through
  tune.sweep.validate_candidate at B = min(B, 128), as the reference's sweep
  validates before it times (benchmark/benchmark_pathtile_candidate_sweep.py:
  153-243).
* The deterministic dK launched on two streams at once: each stream keeps
  its own workspace, so both results equal the single-stream bits; on many
  short-lived streams the runtime keeps a bounded number of workspaces.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
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


def _valu_serves(B, H, L, K):
    """The VALU kernel serves a 16-byte aligned call wherever the library's
    dispatch does not pick the matrix cores (pt_rows_kernel_id)."""
    return not _runtime.rows_on_matrix_cores(B, H, L, K)


def _full_size_case(rt, B, H, L, K, seed, monkeypatch):
    print(f"[case] full size B={B} H={H} L={L} K={K} seed={seed}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    y = torch.empty_like(xd)
    dx = torch.empty_like(xd)
    rt.launch_fwd(xd, wd, y)
    rt.launch_bwd_input(dyd, wd, dx)
    idx = np.sort(np.random.default_rng(seed).choice(B, 256, replace=False))
    idx[0], idx[-1] = 0, B - 1          # first and last sample (ragged tail steps)
    it = torch.from_numpy(idx)
    ys, dxs = y[it.cuda()].cpu().numpy(), dx[it.cuda()].cpu().numpy()
    assert oracle.normalized_max_abs(ys, oracle.fwd_f64(x[it], w)) < FWD_TOL
    assert oracle.normalized_max_abs(dxs, oracle.dx_f64(dy[it], w)) < FWD_TOL
    y_chain, dx_chain = oracle.fwd_f32_refchain(x[it], w), oracle.dx_f32_refchain(dy[it], w)
    if _valu_serves(B, H, L, K):
        assert np.array_equal(ys, y_chain) and np.array_equal(dxs, dx_chain)
    else:
        monkeypatch.setenv("PATHTILE_ROWS_ALGO", "valu")
        yv, dxv = torch.empty_like(xd), torch.empty_like(xd)
        rt.launch_fwd(xd, wd, yv)
        rt.launch_bwd_input(dyd, wd, dxv)
        monkeypatch.delenv("PATHTILE_ROWS_ALGO")
        assert np.array_equal(yv[it.cuda()].cpu().numpy(), y_chain)
        assert np.array_equal(dxv[it.cuda()].cpu().numpy(), dx_chain)
        del yv, dxv
    ref = oracle.dk_f64(dy, x, K)
    ga = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight(dyd, xd, ga, K, zero_first=True)
    g1 = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_deterministic(dyd, xd, g1, K)
    g2 = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_deterministic(dyd, xd, g2, K)
    assert oracle.normalized_max_abs(ga.cpu().numpy(), ref) < DK_TOL
    assert oracle.normalized_max_abs(g1.cpu().numpy(), ref) < DK_TOL
    assert torch.equal(g1, g2)
    # size-independent identities over the whole tensors, in FP64
    left = float((y.double() * dyd.double()).sum())
    right = float((xd.double() * dx.double()).sum())
    dk_w = float((g1.double() * wd.double()).sum())
    scale = float(y.double().norm()) * float(dyd.double().norm())
    assert abs(left - right) <= 1e-6 * scale
    assert abs(left - dk_w) <= 1e-6 * scale


def test_short_config_full_size(rt, monkeypatch):
    """BASELINE S: B32768 H256 L48 K4 (the VALU rows kernel serves K = 4)."""
    _full_size_case(rt, 32768, 256, 48, 4, 77, monkeypatch)


def test_odd_k_config_full_size(rt, monkeypatch):
    """BASELINE E2: B16384 H128 L48 K47 (the matrix cores serve FWD/dX)."""
    _full_size_case(rt, 16384, 128, 48, 47, 78, monkeypatch)


def test_short_rows_above_the_mall_full_size(rt, monkeypatch):
    """The tuner's holdout_b32768_h256_l24_k32 at its full size (805 MB per
    tensor): rows of fewer than 33 columns on tensors above 256 MiB, where
    FWD/dX take non-temporal loads and 16-channel workgroups are not used,
    and dK ranges follow the 3 MiB stride rule."""
    _full_size_case(rt, 32768, 256, 24, 32, 80, monkeypatch)


def test_odd_row_length_above_the_mall_full_size(rt, monkeypatch):
    """L % 4 != 0 on tensors above 256 MiB (B16384 H128 L37 K48, 310 MB
    each): FWD/dX on the matrix-core kernel's element-wise form with
    non-temporal loads; dK on the channel-group kernel with two channels per
    wave and 16-byte chunk staging. The same values in 4-byte aligned
    storage take one channel per wave with dword staging (another range
    count, so other bits): within 1e-4 of FP64 and bitwise reproducible."""
    _full_size_case(rt, 16384, 128, 37, 48, 79, monkeypatch)
    B, H, L, K = 16384, 128, 37, 48
    x, w, dy = oracle.make_inputs(B, H, L, K, 79)
    xd, dyd = x.cuda(), dy.cuda()
    g_aligned = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_deterministic(dyd, xd, g_aligned, K)
    flat = torch.empty(2 * (xd.numel() + 1), device="cuda")
    xm = flat[1:xd.numel() + 1].view(B, H, L)
    dym = flat[xd.numel() + 2:].view(B, H, L)
    assert xm.data_ptr() % 16 != 0 and dym.data_ptr() % 16 != 0
    xm.copy_(xd)
    dym.copy_(dyd)
    del xd, dyd
    g_mis = [torch.full((H, K), float("nan"), device="cuda") for _ in range(2)]
    for g in g_mis:
        rt.launch_bwd_weight_deterministic(dym, xm, g, K)
    ga = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight(dym, xm, ga, K, zero_first=True)
    ref = oracle.dk_f64(dy, x, K)
    assert oracle.normalized_max_abs(g_aligned.cpu().numpy(), ref) < DK_TOL
    assert oracle.normalized_max_abs(g_mis[0].cpu().numpy(), ref) < DK_TOL
    assert oracle.normalized_max_abs(ga.cpu().numpy(), ref) < DK_TOL
    assert torch.equal(g_mis[0], g_mis[1])


def test_eight_channel_groups_above_the_mall(rt, monkeypatch):
    """H % 16 != 0 on tensors above 256 MiB: the matrix-core FWD/dX in
    8-channel workgroups with non-temporal loads, in both forms (L = 48 and
    L = 37, where rows are not whole float4s)."""
    _full_size_case(rt, 12288, 136, 48, 48, 81, monkeypatch)
    _full_size_case(rt, 14000, 136, 37, 40, 82, monkeypatch)


@pytest.mark.parametrize("shape", [(12000, 128, 44, 48), (13800, 128, 38, 13),
                                   (14000, 130, 37, 48)])
def test_dk_two_channels_per_wave_above_the_mall(shape):
    """Tensors just above 256 MiB with rows whose one-channel segments are
    not whole 64-byte units (L = 44, 38 at 128 threads): the channel-group dK
    runs two channels per wave; with H % 4 != 0 (H = 130, L = 37) it keeps
    one channel per wave and stages dwords. Atomic and deterministic within
    1e-4 of FP64, deterministic bitwise reproducible."""
    from pathtile_amd import runtime

    B, H, L, K = shape
    assert 4 * B * H * L >= 256 * 2**20
    print(f"[case] dK above the MALL B={B} H={H} L={L} K={K}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=B + L)
    xd, dyd = x.cuda(), dy.cuda()
    r = runtime.HipWarpRuntime(bwdk_block=128)
    ga = torch.full((H, K), float("nan"), device="cuda")
    r.launch_bwd_weight(dyd, xd, ga, K, zero_first=True)
    g1 = torch.full((H, K), float("nan"), device="cuda")
    g2 = torch.full((H, K), float("nan"), device="cuda")
    r.launch_bwd_weight_deterministic(dyd, xd, g1, K)
    r.launch_bwd_weight_deterministic(dyd, xd, g2, K)
    ref = oracle.dk_f64(dy, x, K)
    assert oracle.normalized_max_abs(ga.cpu().numpy(), ref) < DK_TOL
    assert oracle.normalized_max_abs(g1.cpu().numpy(), ref) < DK_TOL
    assert torch.equal(g1, g2)
    r.close()


REF_AMPERE_CASES = [(2, 4, 16, 8), (4, 8, 31, 16), (8, 16, 48, 24), (32, 64, 48, 48),
                    (128, 128, 48, 48)]        # kernels/warp_tiled_ampere.py:920-926
REF_SHARED_CASES = [(2, 4, 48, 47), (2, 4, 48, 48), (2, 4, 48, 49),
                    (8, 16, 48, 48)]           # validate/validate_shared.py:236-249


@pytest.mark.parametrize("api,shape",
                         [("ampere", s) for s in REF_AMPERE_CASES]
                         + [("shared", s) for s in REF_SHARED_CASES],
                         ids=lambda v: v if isinstance(v, str) else "B{}H{}L{}K{}".format(*v))
def test_reference_validation_cases(rt, api, shape):
    from pathtile_amd import runtime
    from pathtile_amd.kernels import warp_tiled as wt

    B, H, L, K = shape
    print(f"[case] reference {api} B={B} H={H} L={L} K={K}", flush=True)
    runtime.install_runtime(rt)
    g = torch.Generator().manual_seed(B * 1000 + K)
    x = torch.randn(B, H, L, generator=g)
    w = torch.randn(H, K, generator=g)          # the reference draws w ~ N(0, 1)
    dy = torch.randn(B, H, L, generator=g)
    fn = runtime.depthwise_conv_ampere if api == "ampere" else wt.depthwise_conv_shared
    xd = x.cuda().requires_grad_(True)
    wd = w.cuda().requires_grad_(True)
    y = fn(xd, wd)
    gx, gk = torch.autograd.grad(y, (xd, wd), dy.cuda())
    y, gx, gk = y.detach().cpu(), gx.cpu(), gk.cpu()
    y64, dx64, dk64 = oracle.fwd_f64(x, w), oracle.dx_f64(dy, w), oracle.dk_f64(dy, x, K)
    assert oracle.normalized_max_abs(y.numpy(), y64) < FWD_TOL
    assert oracle.normalized_max_abs(gx.numpy(), dx64) < FWD_TOL
    assert oracle.normalized_max_abs(gk.numpy(), dk64) < DK_TOL
    assert torch.allclose(y.double(), torch.from_numpy(y64), atol=2e-3, rtol=2e-3)
    assert torch.allclose(gx.double(), torch.from_numpy(dx64), atol=2e-3, rtol=2e-3)
    assert torch.allclose(gk.double(), torch.from_numpy(dk64), atol=1e-2, rtol=5e-4)


@pytest.mark.parametrize("group", ["train", "holdout"])
def test_every_tuner_candidate_validates_on_the_30_shapes(group):
    from pathtile_amd.tune import shapes, sweep

    train, holdout = shapes.draw_shapes()
    assert len(train) == 20 and len(holdout) == 10
    cases = train if group == "train" else holdout
    specs = [(sweep.FWD_DX_KIND, v) for v in sweep.FWD_DX_CANDIDATES]
    specs += [(sweep.DK_KIND, v) for v in sweep.DK_CANDIDATES]
    runtimes = {spec: sweep.make_runtime(*spec) for spec in specs}
    n = 0
    for case in cases:
        print(f"[case] tuner {case.config_id}", flush=True)
        seed = sweep.case_seed(0, case)
        for kind, value in specs:
            rows = sweep.validate_candidate(runtimes[(kind, value)], case, seed, kind, value)
            assert rows and all(r["allclose"] for r in rows), rows
            n += len(rows)
    assert n == len(cases) * (2 * len(sweep.FWD_DX_CANDIDATES) + len(sweep.DK_CANDIDATES))


def test_deterministic_dk_on_two_streams():
    """Two deterministic dK launches in flight at once on two streams (two
    shapes, two workspace sizes), three times over: each stream keeps its own
    workspace, so both results keep the single-stream bits."""
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime()
    cases = [(8192, 128, 48, 48), (6000, 64, 32, 16)]
    data, ref = [], []
    for i, (B, H, L, K) in enumerate(cases):
        print(f"[case] two streams B={B} H={H} L={L} K={K}", flush=True)
        x, w, dy = oracle.make_inputs(B, H, L, K, seed=90 + i)
        xd, dyd = x.cuda(), dy.cuda()
        g = torch.empty(H, K, device="cuda")
        r.launch_bwd_weight_deterministic(dyd, xd, g, K)
        torch.cuda.synchronize()
        assert oracle.normalized_max_abs(g.cpu().numpy(), oracle.dk_f64(dy, x, K)) < DK_TOL
        data.append((xd, dyd, K))
        ref.append(g)
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    outs = [torch.full_like(g, float("nan")) for g in ref]
    main = torch.cuda.current_stream()
    for s in streams:
        s.wait_stream(main)
    for _ in range(3):
        for s, (xd, dyd, K), o in zip(streams, data, outs):
            with torch.cuda.stream(s):
                r.launch_bwd_weight_deterministic(dyd, xd, o, K)
    torch.cuda.synchronize()
    for o, g in zip(outs, ref):
        assert torch.equal(o, g)
    keys = {k[1] for k in r._workspaces}
    assert {int(s.cuda_stream) for s in streams} <= keys
    r.close()


def test_deterministic_dk_workspaces_are_bounded():
    """A caller that launches on many short-lived streams keeps at most
    WORKSPACE_STREAMS workspaces alive (least recently used dropped), and
    every launch keeps the single-stream bits."""
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime()
    B, H, L, K = 4096, 64, 48, 24
    print(f"[case] many streams B={B} H={H} L={L} K={K}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=95)
    xd, dyd = x.cuda(), dy.cuda()
    g = torch.empty(H, K, device="cuda")
    r.launch_bwd_weight_deterministic(dyd, xd, g, K)
    torch.cuda.synchronize()
    main = torch.cuda.current_stream()
    for i in range(3 * runtime.WORKSPACE_STREAMS):
        s = torch.cuda.Stream()
        s.wait_stream(main)
        o = torch.full_like(g, float("nan"))
        with torch.cuda.stream(s):
            r.launch_bwd_weight_deterministic(dyd, xd, o, K)
        s.synchronize()
        assert torch.equal(o, g), i
        assert len(r._workspaces) <= runtime.WORKSPACE_STREAMS
    assert len(r._workspaces) == runtime.WORKSPACE_STREAMS
    r.close()
