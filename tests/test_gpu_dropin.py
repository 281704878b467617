"""The drop-in module's harness helpers on the GPU (marked ``gpu``), called
through ``pathtile_amd.kernels.warp_tiled_ampere`` as a reference harness
calls them (kernels/warp_tiled_ampere.py:909-987 validate_correctness,
:1021-1113 benchmark_kernels, :1666-1679 print_device_report; the runtime's
device_id / device :662-663).

Bars: the reference's allclose bars against PyTorch's FP32 convolution (FWD
and dX atol = rtol = 2e-3; dK atol 1e-2, rtol 5e-4), and on the same cases
this build's bars against the CPU oracle in FP64 (FWD/dX 1e-5, dK 1e-4
max-abs-scaled)."""

from __future__ import annotations

import pytest
import torch

import oracle
from pathtile_amd.kernels import warp_tiled_ampere as wta

pytestmark = pytest.mark.gpu


@pytest.fixture()
def installed():
    from pathtile_amd import runtime

    saved = runtime._RUNTIME
    rt = wta.HipWarpRuntime()
    wta.install_runtime(rt)
    yield rt
    runtime._RUNTIME = saved
    rt.close()


def test_validate_correctness_default_cases(installed, tmp_path):
    print("[case] validate_correctness default cases", flush=True)
    df = wta.validate_correctness(tmp_path, seed=3)
    assert (tmp_path / "correctness.csv").exists()
    assert len(df) == len(wta.DEFAULT_VALIDATION_CASES)
    for ph in ("fwd", "bwd_input", "bwd_weight"):
        assert df[f"{ph}_allclose"].all()
    assert df["within_fp64_bars"].all(), df.filter(like="fp64").to_string()


@pytest.mark.parametrize("case", wta.DEFAULT_VALIDATION_CASES, ids=lambda c: "B{}H{}L{}K{}".format(*c))
def test_dropin_autograd_against_the_oracle(installed, case):
    """depthwise_conv_ampere through the drop-in module, on the reference's
    validation cases with its w ~ N(0, 1), against the CPU oracle in FP64."""
    B, H, L, K = case
    print(f"[case] drop-in oracle B={B} H={H} L={L} K={K}", flush=True)
    g = torch.Generator().manual_seed(100 + B + H + L + K)
    x = torch.randn(B, H, L, generator=g)
    w = torch.randn(H, K, generator=g)
    gy = torch.randn(B, H, L, generator=g)
    xd = x.cuda().requires_grad_(True)
    wd = w.cuda().requires_grad_(True)
    y = wta.depthwise_conv_ampere(xd, wd)
    gx, gk = torch.autograd.grad(y, (xd, wd), gy.cuda())
    assert oracle.normalized_max_abs(y.detach().cpu().numpy(), oracle.fwd_f64(x, w)) < 1e-5
    assert oracle.normalized_max_abs(gx.cpu().numpy(), oracle.dx_f64(gy, w)) < 1e-5
    assert oracle.normalized_max_abs(gk.cpu().numpy(), oracle.dk_f64(gy, x, K)) < 1e-4


def test_benchmark_kernels_and_device_report(installed, tmp_path, capsys):
    rt = installed
    assert rt.device_id == torch.cuda.current_device()
    assert rt.device == torch.device("cuda", rt.device_id)
    assert rt.profile.key == "mi355x"
    raw, summary = wta.benchmark_kernels(rt, tmp_path, B=512, H=64, L=48, K=48,
                                         warmup=2, runs=5, seed=1)
    assert (tmp_path / "benchmark_raw.csv").exists()
    assert (tmp_path / "benchmark_summary.csv").exists()
    assert len(raw) == 15
    assert list(summary["phase"]) == ["fwd", "bwd_input", "bwd_weight"]
    assert (summary["runs"] == 5).all()
    assert (summary["mean_ms"] > 0).all()
    nbytes = wta.minimum_algorithmic_bytes(512, 64, 48, 48)
    assert (summary["algorithmic_bytes"] == nbytes).all()
    expect = 100 * nbytes / (summary["mean_ms"] / 1e3) / 1e9 / 8000.0
    assert ((summary["pct_of_peak_algorithmic"] - expect).abs() < 1e-6).all()
    assert set(summary["device_name"]) == {torch.cuda.get_device_name(rt.device_id)}
    wta.print_device_report(rt)
    out = capsys.readouterr().out
    assert "KERNEL MICROBENCHMARK" in out and "CU count:" in out and "mi355x" in out
