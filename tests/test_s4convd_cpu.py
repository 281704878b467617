"""S4ConvD model around the path (kernels/warp_tiled_ampere.py:1116-1224), CPU
tier: the kernel parameterisation against closed forms, the skip-term fusion
identity against the oracle in FP64, the reference's parameter layout and
initial draws, the loss, and the backend switch."""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from pathtile_amd import s4convd
from pathtile_amd.kernels import warp_tiled_ampere as wta


@pytest.fixture
def backend():
    """Set TRAIN_CONV_BACKEND for one test and restore it afterwards."""
    old = wta.TRAIN_CONV_BACKEND

    def set_(value):
        wta.TRAIN_CONV_BACKEND = value

    yield set_
    wta.TRAIN_CONV_BACKEND = old


def _one_mode_kernel(log_dt, c_re, c_im, log_a_re, a_im, taps):
    m = s4convd.S4ConvKernel(1, 2)
    with torch.no_grad():
        m.log_dt.fill_(log_dt)
        m.C_re.fill_(c_re)
        m.C_im.fill_(c_im)
        m.log_A_re.fill_(log_a_re)
        m.A_im.fill_(a_im)
    return m.build_kernel(taps, torch.device("cpu"))[0].detach().double().numpy()


def test_build_kernel_real_mode_is_geometric():
    """One state with A real (A_im = 0), C real: k[t] = 2 C (e^{dt a} - 1)/a
    e^{dt a t} with a = -exp(log_A_re): k[0] in closed form and a constant
    ratio e^{dt a} between taps."""
    log_dt, c, log_a = math.log(0.05), 0.7, math.log(1.3)
    k = _one_mode_kernel(log_dt, c, 0.0, log_a, 0.0, 48)
    dt, a = math.exp(log_dt), -math.exp(log_a)
    assert k[0] == pytest.approx(2 * c * (math.exp(dt * a) - 1) / a, rel=1e-6)
    np.testing.assert_allclose(k[1:] / k[:-1], math.exp(dt * a), rtol=2e-6)


def test_build_kernel_oscillating_mode_recurrence():
    """A = a + i w: k[t] = 2 Re(C_eff z^t), z = e^{dt A}, satisfies
    k[t+2] = 2 Re(z) k[t+1] - |z|^2 k[t] (pins the exponent dt * A * t), and
    k[0] = 2 Re(C (z - 1) / A) (the zero-order-hold factor)."""
    log_dt, cr, ci, log_a, w = math.log(0.09), 0.4, -1.1, math.log(0.6), 2.5
    k = _one_mode_kernel(log_dt, cr, ci, log_a, w, 40)
    dt = math.exp(log_dt)
    A = complex(-math.exp(log_a), w)
    z = complex(math.e ** (dt * A.real) * math.cos(dt * A.imag),
                math.e ** (dt * A.real) * math.sin(dt * A.imag))
    C = complex(cr, ci)
    assert k[0] == pytest.approx(2 * (C * (z - 1) / A).real, rel=1e-5)
    lhs = k[2:]
    rhs = 2 * z.real * k[1:-1] - abs(z) ** 2 * k[:-2]
    np.testing.assert_allclose(lhs, rhs, atol=2e-6 * np.abs(k).max())


def test_build_kernel_sums_modes_and_small_dt_limit():
    """Modes add linearly; for small dt the zero-order-hold factor is
    C_eff = C dt (1 + dt A / 2 + (dt A)^2 / 6 + O(dt^3)), so
    k[0] = 2 Re sum_n C_eff[n] follows from the series (dt = 1e-3; FP32
    cancellation in exp(dt A) - 1 leaves about 1e-4 relative)."""
    torch.manual_seed(3)
    m = s4convd.S4ConvKernel(3, 8)
    k = m.build_kernel(16, torch.device("cpu")).detach().double()
    parts = torch.zeros_like(k)
    for n in range(4):
        mn = s4convd.S4ConvKernel(3, 2)
        with torch.no_grad():
            mn.log_dt.copy_(m.log_dt)
            for name in ("C_re", "C_im", "log_A_re", "A_im"):
                getattr(mn, name).copy_(getattr(m, name)[:, n:n + 1])
        parts += mn.build_kernel(16, torch.device("cpu")).detach().double()
    torch.testing.assert_close(k, parts, rtol=1e-5, atol=1e-5 * float(k.abs().max()))
    dt = 1e-3
    with torch.no_grad():
        m.log_dt.fill_(math.log(dt))
    k0 = m.build_kernel(1, torch.device("cpu"))[:, 0].detach().double().numpy()
    A = -np.exp(m.log_A_re.detach().double().numpy()) + 1j * m.A_im.detach().double().numpy()
    C = m.C_re.detach().double().numpy() + 1j * m.C_im.detach().double().numpy()
    series = C * dt * (1 + dt * A / 2 + (dt * A) ** 2 / 6)
    expect = 2 * series.sum(axis=1).real
    np.testing.assert_allclose(k0, expect, rtol=1e-3, atol=1e-3 * np.abs(expect).max())


@pytest.mark.parametrize("B,H,L,K", [(3, 5, 48, 48), (4, 3, 17, 17), (2, 4, 20, 7), (2, 2, 9, 48)])
def test_skip_term_is_the_centre_tap(B, H, L, K):
    """conv(x, k) + skip * x = conv(x, k') with k' = k + skip on tap K // 2,
    in FP64 through the oracle; for the backward, dX(dy; k') = dX(dy; k) +
    skip * dy and dL/dskip = sum dy * x = dK[:, K // 2]. Dyadic k and skip
    make k' exact in FP32, so the identities hold to FP64 rounding."""
    g = np.random.default_rng(B * 100 + K)
    x = g.standard_normal((B, H, L)).astype(np.float32)
    dy = g.standard_normal((B, H, L)).astype(np.float32)
    k = (g.integers(-64, 64, (H, K)) / 64.0).astype(np.float32)
    skip = (g.integers(-64, 64, H) / 64.0).astype(np.float32)
    p = K // 2
    k2 = k.copy()
    k2[:, p] += skip
    scale = np.abs(oracle.fwd_f64(x, k)).max() + 1.0
    np.testing.assert_allclose(oracle.fwd_f64(x, k2),
                               oracle.fwd_f64(x, k) + skip[None, :, None] * x.astype(np.float64),
                               rtol=0, atol=1e-12 * scale)
    np.testing.assert_allclose(oracle.dx_f64(dy, k2),
                               oracle.dx_f64(dy, k) + skip[None, :, None] * dy.astype(np.float64),
                               rtol=0, atol=1e-12 * scale)
    dk = oracle.dk_f64(dy, x, K)
    dskip = (dy.astype(np.float64) * x.astype(np.float64)).sum(axis=(0, 2))
    np.testing.assert_allclose(dk[:, p], dskip, rtol=1e-12, atol=1e-12)


def test_pytorch_backend_is_the_reference_composition(backend):
    """The "pytorch" backend computes conv(x, k) and then adds x * skip
    (:1160-1165, :1187-1188); it equals conv(x, k') to FP32 rounding."""
    backend("pytorch")
    torch.manual_seed(0)
    m = s4convd.S4ConvKernel(6, 16)
    x = torch.randn(5, 6, 40)
    skip = torch.randn(6)
    with torch.no_grad():
        y = m(x, skip)
        k = m.build_kernel(40, x.device)
        y_sep = wta.reference_depthwise_conv(x, k) + x * skip[:, None]
        k2 = k.clone()
        k2[:, 20] += skip
        y_fused = wta.reference_depthwise_conv(x, k2)
    assert torch.equal(y, y_sep)
    torch.testing.assert_close(y, y_fused, rtol=1e-5, atol=1e-5 * float(y.abs().max()))


REFERENCE_BLOCK_PARAMS = [
    ("skip", (8,)),
    ("kernel_layer.log_dt", (8,)),
    ("kernel_layer.C_re", (8, 6)),
    ("kernel_layer.C_im", (8, 6)),
    ("kernel_layer.log_A_re", (8, 6)),
    ("kernel_layer.A_im", (8, 6)),
    ("output_linear.0.weight", (16, 8, 1)),
    ("output_linear.0.bias", (16,)),
]


def test_parameter_layout_matches_the_reference():
    """Names, shapes and order of the reference's parameters
    (:1122-1135, :1172-1182, :1193-1208), so its state_dicts load."""
    m = s4convd.Model(state_dim=12, hidden_dim=8, input_dim=3, output_dim=2, num_blocks=2)
    got = [(n, tuple(p.shape)) for n, p in m.named_parameters()]
    expect = [("encoder.weight", (8, 3)), ("encoder.bias", (8,))]
    for b in range(2):
        expect += [(f"blocks.{b}.{n}", s) for n, s in REFERENCE_BLOCK_PARAMS]
    expect += [("decoder.weight", (2, 8)), ("decoder.bias", (2,))]
    assert got == expect


def test_initial_draws_follow_the_reference_order():
    """Under one seed the kernel parameters are the reference's draws, in
    its order: rand(H) scaled into [log 1e-3, log 1e-1) for log_dt, then
    randn for C_re, C_im, log_A_re, and ones for A_im (:1126-1134)."""
    H, half = 7, 5
    torch.manual_seed(11)
    m = s4convd.S4ConvKernel(H, 2 * half)
    torch.manual_seed(11)
    u = torch.rand(H)
    c_re, c_im, a_re = torch.randn(H, half), torch.randn(H, half), torch.randn(H, half)
    lo, hi = math.log(0.001), math.log(0.1)
    assert torch.equal(m.log_dt.detach(), u * (hi - lo) + lo)
    assert torch.equal(m.C_re.detach(), c_re)
    assert torch.equal(m.C_im.detach(), c_im)
    assert torch.equal(m.log_A_re.detach(), a_re)
    assert torch.equal(m.A_im.detach(), torch.ones(H, half))


def test_rmsle_closed_form():
    a = torch.tensor([0.0, 1.0, 2.5, 0.3])
    b = torch.tensor([0.5, 1.0, 0.2, 2.0])
    got = s4convd.rmsle(torch.expm1(a), torch.expm1(b))
    assert float(got) == pytest.approx(math.sqrt(float(((a - b) ** 2).mean()) + 1e-12), rel=1e-6)
    # negative parts are clamped to 0 before the log
    assert float(s4convd.rmsle(torch.tensor([-3.0]), torch.tensor([0.0]))) == pytest.approx(1e-6)


def test_model_trains_on_the_pytorch_backend(backend):
    backend("pytorch")
    torch.manual_seed(1)
    m = s4convd.Model(state_dim=8, hidden_dim=16, input_dim=4, output_dim=1, num_blocks=2)
    x = torch.randn(6, 24, 4)
    target = torch.rand(6, 1)
    out = m(x)
    assert out.shape == (6, 1)
    loss = s4convd.rmsle(out, target)
    loss.backward()
    for n, p in m.named_parameters():
        assert p.grad is not None and torch.isfinite(p.grad).all(), n


def test_backend_switch_and_errors(backend):
    m = s4convd.S4ConvKernel(4, 8)
    backend("bogus")
    with pytest.raises(RuntimeError, match="Unknown training backend: bogus"):
        m(torch.zeros(1, 4, 8))
    backend("pytorch")
    with pytest.raises(ValueError, match="Expected H=4, got 3"):
        m(torch.zeros(1, 3, 8))
    with pytest.raises(ValueError, match="L<=48"):
        m(torch.zeros(1, 4, 49))
    assert "TRAIN_CONV_BACKEND" in wta.__all__ and "S4ConvBlock" in wta.__all__
