"""The Python drop-in surface on CPU: names, constants, error types and
messages in the reference's order (kernels/warp_tiled.py:787-1031,
kernels/warp_tiled_ampere.py:625-903), and host-side helpers."""

from __future__ import annotations

import pytest
import torch

from pathtile_amd import runtime as rt
from pathtile_amd.kernels import warp_tiled as wt
from pathtile_amd.kernels import warp_tiled_ampere as wta


def test_reference_names_exist():
    for name in wt.__all__:
        assert hasattr(wt, name), name
    assert wt.__all__ == [
        "DepthwiseConvShared", "depthwise_conv_shared", "THREADS_PER_BLOCK", "TTILE",
        "HTILE", "shared_memory_bytes", "FWD_TIMES", "BWD_IN_TIMES", "BWD_K_TIMES",
        "reset_timing_collectors",
    ]
    for name in ("DepthConvAmpere", "depthwise_conv_ampere", "reference_depthwise_conv",
                 "AmpereWarpRuntime", "install_runtime", "get_runtime",
                 "KernelEventCollector", "KERNEL_EVENTS", "MAX_L", "MAX_K",
                 "DEFAULT_B", "DEFAULT_H", "DEFAULT_L", "DEFAULT_K",
                 "DEFAULT_WARPS_PER_BLOCK", "DEFAULT_BWDK_BTILE", "DEFAULT_BWDK_KPACK",
                 "DEFAULT_BWDK_BLOCK", "minimum_algorithmic_bytes", "normalized_max_abs",
                 "configure_torch", "validate_correctness", "benchmark_kernels",
                 "print_device_report", "estimate_ampere_occupancy",
                 "estimate_gpu_occupancy", "summarize_kernel_times"):
        assert hasattr(wta, name), name
        assert name in wta.__all__, name
    # the reference's alias (kernels/warp_tiled_ampere.py:260)
    assert wta.estimate_ampere_occupancy is wta.estimate_gpu_occupancy
    # the harness helpers take the reference's parameters, in its order
    import inspect

    assert list(inspect.signature(wta.validate_correctness).parameters) == [
        "output_dir", "cases", "seed"]
    assert list(inspect.signature(wta.benchmark_kernels).parameters) == [
        "runtime", "output_dir", "B", "H", "L", "K", "warmup", "runs", "seed"]
    assert list(inspect.signature(wta.print_device_report).parameters) == ["runtime"]
    # the runtime records its device (None without a GPU)
    r = wta.HipWarpRuntime()
    assert hasattr(r, "device_id") and hasattr(r, "device")
    if not torch.cuda.is_available():
        assert r.device_id is None and r.device is None


def test_legacy_constants():
    assert (wt.TTILE, wt.HTILE, wt.THREADS_PER_BLOCK, wt.BWD_K_B_TILE) == (32, 16, 512, 64)
    assert wt.shared_memory_bytes(48) == 16 * (32 + 47) * 4 == 5056
    assert wt.bwd_kernel_shared_memory_bytes(48) == 2 * 64 * 48 * 4 == 24576
    assert (rt.MAX_L, rt.MAX_K, rt.DEFAULT_BWDK_BTILE) == (48, 48, 64)


def test_forward_error_order_matches_reference():
    cpu = torch.zeros(2, 3, 8)
    k = torch.zeros(3, 4)
    with pytest.raises(ValueError, match="x and kernel must be CUDA tensors"):
        wt.DepthwiseConvShared.apply(cpu, k)
    with pytest.raises(ValueError, match="x and kernel must be CUDA tensors"):
        wt.depthwise_conv_shared(cpu.double(), k)


def test_runtime_config_validation():
    from pathtile_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    for bad in (0, 3, 32):
        with pytest.raises(ValueError, match="waves_per_block must be one of"):
            rt.HipWarpRuntime(waves_per_block=bad)
    with pytest.raises(ValueError, match="fixes BWDK_BTILE=64"):
        rt.HipWarpRuntime(bwdk_btile=32)
    for bad in (32, 96, 1024, 0):
        with pytest.raises(ValueError, match="bwdk_block must be a multiple of 64"):
            rt.HipWarpRuntime(bwdk_block=bad)
    with pytest.raises(ValueError, match="rows_algo must be one of"):
        rt.HipWarpRuntime(rows_algo="tile")
    for name in ("auto", "valu", "mfma"):
        assert rt.HipWarpRuntime(rows_algo=name).rows_algo == name
    r = rt.HipWarpRuntime(waves_per_block=8, bwdk_block=512, dx_waves_per_block=2)
    assert (r.fwd_block, r.dx_waves_per_block, r.bwdk_block) == (512, 2, 512)
    assert r.rows_algo == "auto"
    r.close()
    r.close()  # idempotent
    with pytest.raises(RuntimeError):
        r.launch_fwd(torch.zeros(1, 1, 1), torch.zeros(1, 1), torch.zeros(1, 1, 1))


def test_runtime_shape_checks_on_cpu_tensors():
    with pytest.raises(ValueError, match="x and k must be CUDA tensors"):
        rt.HipWarpRuntime._check_shapes(torch.zeros(1, 2, 3), torch.zeros(2, 3))


def test_get_runtime_requires_install():
    saved = rt._RUNTIME
    try:
        rt._RUNTIME = None
        with pytest.raises(RuntimeError, match="has not been installed"):
            rt.get_runtime()
    finally:
        rt._RUNTIME = saved


def test_algorithmic_bytes_and_flops():
    assert rt.minimum_algorithmic_bytes(16384, 128, 48, 48) == 805_330_944
    assert rt.minimum_algorithmic_bytes(32768, 256, 48, 4) == 3_221_229_568
    assert rt.minimum_algorithmic_bytes(1000, 96, 37, 48) == 28_434_432
    assert rt.minimum_algorithmic_bytes(16384, 128, 48, 47) == 805_330_432
    assert rt.useful_flops(16384, 128, 48, 48) == 7_247_757_312
    assert rt.algorithmic_bandwidth_gbps(805_330_944, 0.1) == pytest.approx(8053.30944)


def test_occupancy_estimate():
    est = rt.estimate_gpu_occupancy(256, 85, 4 * 5120)
    # 88 VGPRs -> 5 waves/SIMD -> 20 waves/CU -> 5 blocks of 4 waves
    assert est["allocated_regs_per_lane"] == 88
    assert est["resident_blocks_per_cu_est"] == 5
    assert est["active_waves_per_cu_est"] == 20
    est = rt.estimate_gpu_occupancy(1024, 64, 16 * 5120)
    # 64 VGPRs -> 8 waves/SIMD; 80 KiB LDS -> 2 blocks of 16 waves either way
    assert est["resident_blocks_per_cu_est"] == 2
    est = rt.estimate_gpu_occupancy(1024, 64, 100 * 1024)
    assert est["resident_blocks_per_cu_est"] == 1
    assert est["limiting_resources_est"] == "lds"
    with pytest.raises(ValueError):
        rt.estimate_gpu_occupancy(2048, 32, 0)


def test_event_collector_disabled_passthrough():
    c = rt.KernelEventCollector()
    calls = []
    c.launch("fwd", lambda: calls.append(1))
    assert calls == [1]
    assert c.rows(synchronize=False) == []


def test_reference_depthwise_conv_is_torch_math():
    import oracle

    x, w, _ = oracle.make_inputs(2, 3, 10, 4, seed=1)
    a = rt.reference_depthwise_conv(x.double(), w.double())
    b = oracle.pytorch_depthwise_same(x.double(), w.double())
    assert torch.equal(a, b)
