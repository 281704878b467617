"""Long rows (L up to 192, K up to 256) on the GPU (marked ``gpu``): the long-row
FWD/dX/dK entry points against the FP64 oracle, and the
``kernels/shared_l192`` API (the reference's long-row module) end to end.

Bars: FWD/dX within 1e-5 and dK within 1e-4 max-abs-scaled of the FP64 sums
(the path's FP32 bars), dK bitwise reproducible. At the reference's own
benchmark shape (B16384 H128 L192 K192,
benchmark/benchmark_gmc_vs_shared_l192.py:14-17) the oracle is too slow for
the whole tensor: FWD/dX are checked on sampled samples (rows are
independent), dK through its FP64 adjoint identity over the whole tensors,
sum_hj dk[h,j] v[h,j] = sum_bht dy[b,h,t] (x conv v)[b,h,t].
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-5
DK_TOL = 1e-4


@pytest.fixture(scope="module")
def rt():
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime()
    runtime.install_runtime(r)
    yield r


SHAPES = [
    (16, 8, 192, 192),
    (33, 4, 100, 37),
    (8, 16, 192, 256),   # K > L
    (40, 8, 64, 3),
    (20, 4, 176, 256),   # K > L, ragged bucket
    (7, 12, 49, 49),     # just past the specialised path
    (64, 8, 130, 1),
    (5, 3, 1, 256),      # one-column rows
    (70, 2, 96, 48),
    (12, 5, 160, 96),    # 160-column bucket, full
    (9, 6, 80, 24),      # 96-column bucket, partial
]


@pytest.fixture(params=["auto", "split", "fp32"])
def long_algo(request, monkeypatch):
    """Algorithm of the long path: the default choice, the BF16 matrix
    cores on three-way split operands everywhere, or the FP32 matrix-core
    instructions everywhere."""
    if request.param == "auto":
        monkeypatch.delenv("PATHTILE_LONG_ALGO", raising=False)
    else:
        monkeypatch.setenv("PATHTILE_LONG_ALGO", request.param)
    return request.param


@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_long_fwd_dx_dk_against_fp64(rt, shape, long_algo):
    B, H, L, K = shape
    print(f"[case] long rows B={B} H={H} L={L} K={K} {long_algo}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=15000 + B + L + K)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    y = torch.full_like(xd, float("nan"))
    dx = torch.full_like(dyd, float("nan"))
    rt.launch_fwd_long(xd, wd, y)
    rt.launch_bwd_input_long(dyd, wd, dx)
    assert oracle.normalized_max_abs(y.cpu().numpy(), oracle.fwd_f64(x, w)) < FWD_TOL
    assert oracle.normalized_max_abs(dx.cpu().numpy(), oracle.dx_f64(dy, w)) < FWD_TOL
    g1 = torch.full((H, K), float("nan"), device="cuda")
    g2 = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_long(dyd, xd, g1, K)
    rt.launch_bwd_weight_long(dyd, xd, g2, K)
    ref = oracle.dk_f64(dy, x, K)
    assert oracle.normalized_max_abs(g1.cpu().numpy(), ref) < DK_TOL
    assert torch.equal(g1, g2)
    for j in range(K):
        lo, hi = oracle.valid_tap_range(L, K, j)
        if hi <= lo:
            assert torch.all(g1[:, j] == 0)


@pytest.mark.parametrize("shape", [(32, 4, 192, 192), (24, 3, 130, 77), (16, 2, 61, 256)],
                         ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_long_fwd_dx_wide_exponent_range(rt, shape, long_algo):
    """Inputs and taps with random exponents over 2^-40 .. 2^40 and full
    FP32 mantissas: every element within 1e-5 of the FP64 sum relative to
    that element's sum of |w| |x| (the FP32 bound of a K-term dot product,
    with a wide margin). A dropped split part (2^-8 of a product) or a
    mis-scaled one fails it by orders of magnitude."""
    B, H, L, K = shape
    print(f"[case] long rows wide exponents B={B} H={H} L={L} K={K} {long_algo}", flush=True)
    g = np.random.default_rng(19 + L)

    def wide(*shape):
        m = g.uniform(1.0, 2.0, size=shape) * g.choice([-1.0, 1.0], size=shape)
        return torch.from_numpy((m * np.exp2(g.integers(-40, 41, size=shape))).astype(np.float32))

    x, w = wide(B, H, L), wide(H, K)
    y = torch.empty(B, H, L, device="cuda")
    dx = torch.empty(B, H, L, device="cuda")
    rt.launch_fwd_long(x.cuda(), w.cuda(), y)
    rt.launch_bwd_input_long(x.cuda(), w.cuda(), dx)
    ax, aw = x.abs(), w.abs()
    for out, ref, bound in ((y, oracle.fwd_f64(x, w), oracle.fwd_f64(ax, aw)),
                            (dx, oracle.dx_f64(x, w), oracle.dx_f64(ax, aw))):
        err = np.abs(out.cpu().numpy().astype(np.float64) - ref)
        assert np.all(err <= 1e-5 * bound)


def _random_long_shapes(n, seed):
    g = np.random.default_rng(seed)
    return [(int(g.integers(1, 81)), int(g.integers(1, 13)), int(g.integers(1, 193)),
             int(g.integers(1, 257))) for _ in range(n)]


@pytest.mark.parametrize("shape", _random_long_shapes(16, 2026), ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_long_split_kernels_random_shapes(rt, shape, monkeypatch):
    """The split kernels forced on seeded random shapes over the whole long
    range (every row and tap bucket, ragged rows, K above and below L):
    FWD/dX within 1e-5 and dK within 1e-4 of FP64."""
    monkeypatch.setenv("PATHTILE_LONG_ALGO", "split")
    B, H, L, K = shape
    print(f"[case] long split random B={B} H={H} L={L} K={K}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=B * 7 + L * 3 + K)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    y = torch.full_like(xd, float("nan"))
    dx = torch.full_like(dyd, float("nan"))
    gk = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_fwd_long(xd, wd, y)
    rt.launch_bwd_input_long(dyd, wd, dx)
    rt.launch_bwd_weight_long(dyd, xd, gk, K)
    assert oracle.normalized_max_abs(y.cpu().numpy(), oracle.fwd_f64(x, w)) < FWD_TOL
    assert oracle.normalized_max_abs(dx.cpu().numpy(), oracle.dx_f64(dy, w)) < FWD_TOL
    ref = oracle.dk_f64(dy, x, K)
    assert oracle.normalized_max_abs(gk.cpu().numpy(), ref) < DK_TOL
    for j in range(K):
        lo, hi = oracle.valid_tap_range(L, K, j)
        if hi <= lo:
            assert torch.all(gk[:, j] == 0)


@pytest.mark.parametrize("shape", [(20, 6, 192, 192), (9, 4, 100, 37)], ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_long_rows_non_finite_input_stays_in_its_channel(rt, shape, long_algo):
    """An infinity or NaN in one channel's rows must not reach another
    channel: the odd channels hold them, the even channels' outputs (FWD,
    dX, dK) must equal a run without them and match FP64."""
    B, H, L, K = shape
    print(f"[case] long rows non-finite B={B} H={H} L={L} K={K} {long_algo}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=31 + L)
    xb, dyb = x.clone(), dy.clone()
    xb[:, 1::2, L // 2] = float("inf")
    xb[:, 1::2, 0] = float("nan")
    dyb[:, 1::2, L // 3] = float("-inf")
    y = torch.empty(B, H, L, device="cuda")
    dx = torch.empty(B, H, L, device="cuda")
    gk = torch.empty(H, K, device="cuda")
    rt.launch_fwd_long(xb.cuda(), w.cuda(), y)
    rt.launch_bwd_input_long(dyb.cuda(), w.cuda(), dx)
    rt.launch_bwd_weight_long(dyb.cuda(), xb.cuda(), gk, K)
    ev = slice(0, H, 2)
    xe, dye, we = x[:, ev].contiguous(), dy[:, ev].contiguous(), w[ev].contiguous()
    assert torch.isfinite(y[:, ev]).all() and torch.isfinite(dx[:, ev]).all() and torch.isfinite(gk[ev]).all()
    assert oracle.normalized_max_abs(y[:, ev].cpu().numpy(), oracle.fwd_f64(xe, we)) < FWD_TOL
    assert oracle.normalized_max_abs(dx[:, ev].cpu().numpy(), oracle.dx_f64(dye, we)) < FWD_TOL
    assert oracle.normalized_max_abs(gk[ev].cpu().numpy(), oracle.dk_f64(dye, xe, K)) < DK_TOL


def test_long_rows_on_short_shapes_match_the_specialised_path(rt):
    """The long kernels also serve L, K <= 48; they agree with the
    specialised kernels to the FP32 bars."""
    B, H, L, K = 300, 16, 48, 48
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=16)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    y1, y2 = torch.empty_like(xd), torch.empty_like(xd)
    rt.launch_fwd_long(xd, wd, y1)
    rt.launch_fwd(xd, wd, y2)
    assert float((y1 - y2).abs().max() / y2.abs().max()) < FWD_TOL
    g1, g2 = torch.empty(H, K, device="cuda"), torch.empty(H, K, device="cuda")
    rt.launch_bwd_weight_long(dyd, xd, g1, K)
    rt.launch_bwd_weight_deterministic(dyd, xd, g2, K)
    assert float((g1 - g2).abs().max() / g2.abs().max()) < DK_TOL


@pytest.mark.parametrize("module", ["shared_l192", "warp_tiled"])
def test_shared_l192_module_autograd(module):
    """The reference's long-row API (and the warp_tiled module's, which
    shares it): y, gx, gk against FP64, timing lists appended once per
    launch, short shapes routed to the specialised path."""
    import importlib

    sl = importlib.import_module(f"pathtile_amd.kernels.{module}")

    sl.reset_timing_collectors()
    for (B, H, L, K) in [(64, 8, 192, 192), (32, 4, 48, 48)]:
        x, w, dy = oracle.make_inputs(B, H, L, K, seed=17 + L)
        xd = x.cuda().requires_grad_(True)
        wd = w.cuda().requires_grad_(True)
        y = sl.depthwise_conv_shared(xd, wd)
        gx, gk = torch.autograd.grad(y, (xd, wd), dy.cuda())
        assert oracle.normalized_max_abs(y.detach().cpu().numpy(), oracle.fwd_f64(x, w)) < FWD_TOL
        assert oracle.normalized_max_abs(gx.cpu().numpy(), oracle.dx_f64(dy, w)) < FWD_TOL
        assert oracle.normalized_max_abs(gk.cpu().numpy(), oracle.dk_f64(dy, x, K)) < DK_TOL
    assert len(sl.FWD_TIMES) == len(sl.BWD_IN_TIMES) == len(sl.BWD_K_TIMES) == 2
    assert all(t > 0 for t in sl.FWD_TIMES + sl.BWD_IN_TIMES + sl.BWD_K_TIMES)


def test_shared_l192_module_errors():
    from pathtile_amd.kernels import shared_l192 as sl

    x = torch.zeros(2, 4, 300, device="cuda")
    with pytest.raises(ValueError, match="L<=192"):
        sl.depthwise_conv_shared(x, torch.zeros(4, 5, device="cuda"))
    with pytest.raises(TypeError, match="x must be float32"):
        sl.depthwise_conv_shared(x.double(), torch.zeros(4, 5, device="cuda"))
    with pytest.raises(ValueError, match="Channel mismatch"):
        sl.depthwise_conv_shared(x[:, :, :192], torch.zeros(3, 5, device="cuda"))


def test_long_rows_reference_benchmark_shape(rt):
    B, H, L, K = 16384, 128, 192, 192
    print(f"[case] long rows at the reference shape B={B} H={H} L={L} K={K}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=42)
    xd, wd, dyd = x.cuda(), w.cuda(), dy.cuda()
    y = torch.empty_like(xd)
    dx = torch.empty_like(dyd)
    rt.launch_fwd_long(xd, wd, y)
    rt.launch_bwd_input_long(dyd, wd, dx)
    idx = torch.from_numpy(np.random.default_rng(5).choice(B, 24, replace=False))
    assert oracle.normalized_max_abs(y[idx.cuda()].cpu().numpy(), oracle.fwd_f64(x[idx], w)) < FWD_TOL
    assert oracle.normalized_max_abs(dx[idx.cuda()].cpu().numpy(), oracle.dx_f64(dy[idx], w)) < FWD_TOL
    del y, dx
    gk = torch.empty(H, K, device="cuda")
    rt.launch_bwd_weight_long(dyd, xd, gk, K)
    v = torch.randn(H, K, generator=torch.Generator().manual_seed(8), dtype=torch.float64)
    lhs = float((gk.double().cpu() * v).sum())
    p = K // 2
    vd = v.cuda()
    rhs = 0.0
    for c0 in range(0, B, 2048):   # FP64 on the GPU, in sample chunks
        xs = torch.nn.functional.pad(xd[c0:c0 + 2048].double(), (p, K - 1 - p))
        conv = torch.zeros(xs.shape[0], H, L, dtype=torch.float64, device="cuda")
        for j in range(K):
            conv += vd[None, :, j:j + 1] * xs[:, :, j:j + L]
        rhs += float((dyd[c0:c0 + 2048].double() * conv).sum())
    assert abs(lhs - rhs) <= 1e-5 * float((gk.double().cpu().abs() * v.abs()).sum())


@pytest.mark.parametrize("shape", [(32, 160000, 192, 48), (32, 340000, 96, 48)],
                         ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_long_dk_step_spans_more_than_2gib(rt, shape, monkeypatch):
    """A 32-sample step of the split DK whose rows span more than 2 GiB
    (from sample 17 of a step on at these shapes, a row starts 2^31 bytes or
    more past sample 0's): with one buffer base per step those samples would
    read as zero. Both split kernels (in place from row bucket 128, staged
    below) against FP64 sums on the GPU, per channel block."""
    monkeypatch.setenv("PATHTILE_LONG_ALGO", "split")
    B, H, L, K = shape
    print(f"[case] long split DK past 2 GiB B={B} H={H} L={L} K={K}", flush=True)
    assert 16 * H * L * 4 < 2 ** 31 <= 31 * H * L * 4
    gen = torch.Generator(device="cuda").manual_seed(77)
    x = torch.randn(B, H, L, device="cuda", generator=gen)
    dy = torch.randn(B, H, L, device="cuda", generator=gen)
    gk = torch.full((H, K), float("nan"), device="cuda")
    rt.launch_bwd_weight_long(dy, x, gk, K)
    p = K // 2
    ref = torch.empty(H, K, dtype=torch.float64, device="cuda")
    for h0 in range(0, H, 16384):
        xs = torch.nn.functional.pad(x[:, h0:h0 + 16384].double(), (p, K - 1 - p))
        ds = dy[:, h0:h0 + 16384].double()
        for j in range(K):
            ref[h0:h0 + 16384, j] = (ds * xs[:, :, j:j + L]).sum(dim=(0, 2))
    err = (gk.double() - ref).abs().max() / ref.abs().max()
    assert float(err) < DK_TOL


def test_long_rows_misaligned_tensors_take_the_dword_path(rt):
    """L % 4 == 0 but a 4-byte aligned (not 16-byte) view: the dword-move
    kernel serves it, with the same results as the aligned call."""
    B, H, L, K = 24, 4, 96, 33
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=18)
    buf = torch.empty(B * H * L + 1, device="cuda")
    xm = buf[1:].view(B, H, L)
    xm.copy_(x.cuda())
    assert xm.data_ptr() % 16 != 0
    y = torch.empty(B * H * L + 1, device="cuda")[1:].view(B, H, L)
    rt.launch_fwd_long(xm, w.cuda(), y)
    y2 = torch.empty(B, H, L, device="cuda")
    rt.launch_fwd_long(x.cuda(), w.cuda(), y2)
    assert torch.equal(y, y2)
    assert oracle.normalized_max_abs(y.cpu().numpy(), oracle.fwd_f64(x, w)) < FWD_TOL


@pytest.mark.parametrize("shape", [(48, 4, 160, 48), (40, 3, 96, 48)], ids=lambda s: "B{}H{}L{}K{}".format(*s))
def test_long_dk_misaligned_tensors_match_aligned(rt, shape, monkeypatch):
    """Split DK on 4-byte aligned (not 16-byte) views: the in-place kernel
    (bucket 160) loads dwords whatever the alignment, the staged one (bucket
    96) takes its dword form; both give the aligned call's bits and stay
    within 1e-4 of FP64."""
    monkeypatch.setenv("PATHTILE_LONG_ALGO", "split")
    B, H, L, K = shape
    print(f"[case] long dK misaligned B={B} H={H} L={L} K={K}", flush=True)
    x, _, dy = oracle.make_inputs(B, H, L, K, seed=21 + L)

    def view(t):
        buf = torch.empty(t.numel() + 1, device="cuda")
        v = buf[1:].view(*t.shape)
        v.copy_(t.cuda())
        assert v.data_ptr() % 16 != 0
        return v

    g1 = torch.empty(H, K, device="cuda")
    g2 = torch.empty(H, K, device="cuda")
    rt.launch_bwd_weight_long(view(dy), view(x), g1, K)
    rt.launch_bwd_weight_long(dy.cuda(), x.cuda(), g2, K)
    assert torch.equal(g1, g2)
    assert oracle.normalized_max_abs(g1.cpu().numpy(), oracle.dk_f64(dy, x, K)) < DK_TOL
