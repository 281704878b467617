"""The reference's ``kernels/warp_tiled_ampere.py`` names: the runtime and
autograd surface S4ConvD and the PathTile tuner call, backed by the MI355X
kernels (definitions in ``pathtile_amd.runtime``), the S4ConvD model
(definitions in ``pathtile_amd.s4convd``), and the module's own harness
helpers, defined here: ``validate_correctness`` (:909-987),
``benchmark_kernels`` (:1021-1113) and ``print_device_report`` (:1666-1679).

``TRAIN_CONV_BACKEND`` is the reference's backend switch (:1119): ``"warp"``
(the HIP path) or ``"pytorch"``; the S4ConvD modules read it from this module
on every forward call, so assigning it here switches them."""

from __future__ import annotations

from pathlib import Path

import torch
import torch.nn.functional as F

from ..runtime import *  # noqa: F401,F403
from ..runtime import __all__ as _runtime_all
from ..s4convd import *  # noqa: F401,F403
from ..s4convd import __all__ as _s4_all

TRAIN_CONV_BACKEND = "warp"

# The reference's allclose bars (:950-958) and this build's bars against FP64
# (max |error| / max |FP64 value|).
ALLCLOSE_BARS = {"fwd": (2e-3, 2e-3), "bwd_input": (2e-3, 2e-3), "bwd_weight": (1e-2, 5e-4)}
FP64_BARS = {"fwd": 1e-5, "bwd_input": 1e-5, "bwd_weight": 1e-4}
DEFAULT_VALIDATION_CASES = [
    (2, 4, 16, 8),
    (4, 8, 31, 16),
    (8, 16, 48, 24),
    (32, 64, 48, 48),
    (128, 128, 48, 48),
]


def _fp64_conv_and_grads(x, k, gy):
    """PyTorch's convolution (the reference's reference_depthwise_conv) and
    its two gradients in FP64 on the same device."""
    xd = x.detach().double().requires_grad_(True)
    kd = k.detach().double().requires_grad_(True)
    y = F.conv1d(xd, kd.unsqueeze(1), padding=kd.shape[1] // 2, groups=xd.shape[1])
    y = y[..., : xd.shape[-1]]
    gx, gk = torch.autograd.grad(y, (xd, kd), gy.double())
    return y.detach(), gx, gk


def validate_correctness(
    output_dir: Path,
    cases: list[tuple[int, int, int, int]] | None = None,
    seed: int = 0,
):
    """FWD, dX and dK of ``depthwise_conv_ampere`` (the installed runtime)
    against PyTorch's FP32 convolution on the GPU, case by case, with the
    reference's error columns and allclose bars (kernels/warp_tiled_ampere.py:
    909-987): writes ``correctness.csv`` to `output_dir` and raises
    AssertionError if a case misses an allclose bar. Added columns give the
    errors against FP64 (``*_fp64_normalized``) and whether every path is
    within this build's bars (FWD/dX 1e-5, dK 1e-4; ``within_fp64_bars``)."""
    import numpy as np
    import pandas as pd

    torch.manual_seed(seed)
    np.random.seed(seed)
    KERNEL_EVENTS.enabled = False
    KERNEL_EVENTS.clear()
    if cases is None:
        cases = list(DEFAULT_VALIDATION_CASES)

    rows = []
    print("\n" + "=" * 88)
    print("CORRECTNESS AGAINST PYTORCH FP32")
    print("=" * 88)
    for B, H, L, K in cases:
        x = torch.randn(B, H, L, device="cuda", dtype=torch.float32, requires_grad=True)
        k = torch.randn(H, K, device="cuda", dtype=torch.float32, requires_grad=True)
        gy = torch.randn(B, H, L, device="cuda", dtype=torch.float32)
        x_ref = x.detach().clone().requires_grad_(True)
        k_ref = k.detach().clone().requires_grad_(True)

        y = depthwise_conv_ampere(x, k)
        y_ref = reference_depthwise_conv(x_ref, k_ref)
        gx, gk = torch.autograd.grad(y, (x, k), gy)
        gx_ref, gk_ref = torch.autograd.grad(y_ref, (x_ref, k_ref), gy)
        y64, gx64, gk64 = _fp64_conv_and_grads(x, k, gy)
        torch.cuda.synchronize()

        got = {"fwd": (y, y_ref, y64), "bwd_input": (gx, gx_ref, gx64),
               "bwd_weight": (gk, gk_ref, gk64)}
        row = {"B": B, "H": H, "L": L, "K": K}
        for ph, (a, ref, ref64) in got.items():
            row[f"{ph}_max_abs"] = max_abs_diff(a, ref)
        for ph, (a, ref, ref64) in got.items():
            row[f"{ph}_normalized_max_abs"] = normalized_max_abs(a, ref)
        for ph, (a, ref, ref64) in got.items():
            atol, rtol = ALLCLOSE_BARS[ph]
            row[f"{ph}_allclose"] = bool(torch.allclose(a, ref, atol=atol, rtol=rtol))
        for ph, (a, ref, ref64) in got.items():
            row[f"{ph}_fp64_normalized"] = normalized_max_abs(a.double(), ref64)
        row["within_fp64_bars"] = all(row[f"{ph}_fp64_normalized"] < FP64_BARS[ph] for ph in got)
        rows.append(row)
        ok = row["fwd_allclose"] and row["bwd_input_allclose"] and row["bwd_weight_allclose"]
        print(f"B={B:4d} H={H:3d} L={L:2d} K={K:2d} | "
              f"fwd={row['fwd_max_abs']:.3e} dx={row['bwd_input_max_abs']:.3e} "
              f"dk={row['bwd_weight_max_abs']:.3e} | ok={ok} | "
              f"fp64 bars={row['within_fp64_bars']}")
        del x, k, gy, x_ref, k_ref, y, y_ref, gx, gk, gx_ref, gk_ref, y64, gx64, gk64

    result = pd.DataFrame(rows)
    output_dir = Path(output_dir)
    output_dir.mkdir(parents=True, exist_ok=True)
    result.to_csv(output_dir / "correctness.csv", index=False)
    if not bool(result[["fwd_allclose", "bwd_input_allclose", "bwd_weight_allclose"]]
                .to_numpy().all()):
        raise AssertionError("At least one correctness case failed")
    return result


def benchmark_kernels(
    runtime: HipWarpRuntime,
    output_dir: Path,
    B: int = DEFAULT_B,
    H: int = DEFAULT_H,
    L: int = DEFAULT_L,
    K: int = DEFAULT_K,
    warmup: int = 5,
    runs: int = 100,
    seed: int = 0,
):
    """The reference's microbenchmark (kernels/warp_tiled_ampere.py:
    1021-1113): `warmup` untimed FWD / dX / zero + dK rounds, then `runs`
    launches per path with an event pair around each launch (dK re-zeroed
    outside its events); per-phase summary with algorithmic bandwidth and
    its share of the device's peak; writes ``benchmark_raw.csv`` and
    ``benchmark_summary.csv``. Returns (raw, summary)."""
    torch.manual_seed(seed)
    x = torch.randn(B, H, L, device="cuda", dtype=torch.float32)
    k = torch.randn(H, K, device="cuda", dtype=torch.float32)
    gy = torch.randn_like(x)
    y = torch.empty_like(x)
    gx = torch.empty_like(x)
    gk = torch.zeros_like(k)

    KERNEL_EVENTS.enabled = False
    for _ in range(warmup):
        runtime.launch_fwd(x, k, y)
        runtime.launch_bwd_input(gy, k, gx)
        gk.zero_()
        runtime.launch_bwd_weight(gy, x, gk, K)
    torch.cuda.synchronize()

    device_name = torch.cuda.get_device_name(runtime.device_id)
    collector = KernelEventCollector()
    collector.enabled = True
    common = {
        "technique": runtime.technique,
        "gpu_profile": runtime.profile.key,
        "device_name": device_name,
        "warps_per_block": runtime.warps_per_block,
        "bwdk_btile": runtime.bwdk_btile,
        "bwdk_block": runtime.bwdk_block,
    }
    for run_id in range(1, runs + 1):
        collector.set_context(**common, run_id_requested=run_id)
        runtime.launch_fwd(x, k, y, collector)
    for run_id in range(1, runs + 1):
        collector.set_context(**common, run_id_requested=run_id)
        runtime.launch_bwd_input(gy, k, gx, collector)
    for run_id in range(1, runs + 1):
        gk.zero_()
        collector.set_context(**common, run_id_requested=run_id)
        runtime.launch_bwd_weight(gy, x, gk, K, collector)

    raw = collector.resolve(synchronize=True)
    summary = summarize_kernel_times(raw)
    nbytes = minimum_algorithmic_bytes(B, H, L, K)
    summary["algorithmic_bytes"] = nbytes
    summary["algorithmic_bandwidth_gbps"] = summary["mean_ms"].map(
        lambda v: algorithmic_bandwidth_gbps(nbytes, v))
    summary["pct_of_peak_algorithmic"] = (
        100.0 * summary["algorithmic_bandwidth_gbps"] / runtime.profile.peak_bandwidth_gbps)
    for key, value in common.items():
        summary[key] = value

    print("\n" + "=" * 88)
    print(f"{runtime.profile.display_name} KERNEL MICROBENCHMARK")
    print("=" * 88)
    print(f"B={B}, H={H}, L={L}, K={K}, warmup={warmup}, runs={runs}")
    print(summary.to_string(index=False))
    print(f"\nSum of phase means:   {float(summary['mean_ms'].sum()):.4f} ms")
    print(f"Sum of phase medians: {float(summary['median_ms'].sum()):.4f} ms")
    print("Note: algorithmic bandwidth uses unique minimum bytes; rocprofv3 "
          "FETCH_SIZE / WRITE_SIZE give the HBM traffic.")

    output_dir = Path(output_dir)
    output_dir.mkdir(parents=True, exist_ok=True)
    raw.to_csv(output_dir / "benchmark_raw.csv", index=False)
    summary.to_csv(output_dir / "benchmark_summary.csv", index=False)
    del x, k, gy, y, gx, gk
    torch.cuda.empty_cache()
    return raw, summary


def print_device_report(runtime: HipWarpRuntime) -> None:
    """The reference's device summary (:1666-1679). On ROCm torch reports
    the gfx target's major.minor (9.5 for gfx950) as the compute capability
    and compute units as its multiprocessor count."""
    device_id = torch.cuda.current_device()
    props = torch.cuda.get_device_properties(device_id)
    capability = torch.cuda.get_device_capability(device_id)
    print("\n" + "=" * 88)
    print("GPU")
    print("=" * 88)
    print(f"Name:               {torch.cuda.get_device_name(device_id)}")
    print(f"Compute capability: {capability[0]}.{capability[1]}")
    print(f"Architecture:       {getattr(props, 'gcnArchName', 'unknown')}")
    print(f"CU count:           {props.multi_processor_count}")
    print(f"Total memory:       {props.total_memory / 1024**3:.2f} GiB")
    print(f"Selected profile:   {runtime.profile.key}")
    print(f"Peak BW reference:  {runtime.profile.peak_bandwidth_gbps:.1f} GB/s")


__all__ = list(_runtime_all) + list(_s4_all) + [
    "TRAIN_CONV_BACKEND", "validate_correctness", "benchmark_kernels", "print_device_report",
]
