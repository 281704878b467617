"""Drop-in for the reference's ``kernels/shared_l192.py`` API (long rows),
on MI355X.

The reference module is the shared-memory family's long-row variant, with
the same public surface as ``kernels/warp_tiled.py`` (``__all__`` at
kernels/shared_l192.py:1020-1031) and benchmarked at B16384 H128 L192 K192
(benchmark/benchmark_gmc_vs_shared_l192.py:14-17). Here the same names run
the hand-written gfx950 kernels of ``libpathtile_hip.so``:

* rows and taps up to 48: the specialised path (the FWD/dX kernels chosen
  per shape, the deterministic two-pass dK);
* anything up to L = 192, K = 256: the long-row matrix-core kernels
  (``pt_dwconv1d_{fwd,dx,dk}_long_f32``), at FP32 accuracy (by default the
  BF16 matrix cores on FP32 operands split three ways, six exact part
  products summed in FP32; ``PATHTILE_LONG_ALGO=fp32`` selects the FP32
  instructions), dK deterministic and written into ``gk`` as the
  reference's dK kernel writes it (one thread per tap,
  kernels/shared_l192.py:966-1001).

Every launch is host-synchronous and its kernel time (ms, HIP events) is
appended to ``FWD_TIMES`` / ``BWD_IN_TIMES`` / ``BWD_K_TIMES`` (:741-780).

Differences from the reference, by design:

* Importing this module needs no GPU (the reference raises at import
  without CUDA, :15-18); CPU tensors raise
  ``ValueError("x and kernel must be CUDA tensors")`` at the first call.
* L is limited to 192 and K to 256 (``ValueError``); the reference's kernel
  has no stated bound.
* ``CudaContextGuard`` is a no-op and ``TorchCudaInterop.as_gpuarray``
  validates and returns the tensor (no PyCUDA), as in the ``warp_tiled``
  mirror. The launch constants and shared-memory helpers keep the
  reference's values (BWD_K_B_TILE = 32 here, :118) as documented constants.
"""

from __future__ import annotations

import torch

from .warp_tiled import CudaContextGuard, TorchCudaInterop, make_shared_function  # noqa: F401

# Legacy launch constants (kernels/shared_l192.py:109-118)
TTILE = 32
HTILE = 16
THREADS_PER_BLOCK = TTILE * HTILE  # 512
BWD_K_B_TILE = 32


def bwd_kernel_shared_memory_bytes(L: int) -> int:
    """Reference backward-weight shared memory, 2 * 32 * L * 4 (:690-705)."""
    return 2 * BWD_K_B_TILE * L * 4


def shared_memory_bytes(K: int) -> int:
    """Reference forward/backward-input shared memory,
    HTILE * (TTILE + K - 1) * 4 (:708-729)."""
    return HTILE * (TTILE + K - 1) * 4


FWD_TIMES: list[float] = []
BWD_IN_TIMES: list[float] = []
BWD_K_TIMES: list[float] = []


def reset_timing_collectors():
    FWD_TIMES.clear()
    BWD_IN_TIMES.clear()
    BWD_K_TIMES.clear()


DepthwiseConvShared = make_shared_function(FWD_TIMES, BWD_IN_TIMES, BWD_K_TIMES, __name__)


def depthwise_conv_shared(x: torch.Tensor, kernel: torch.Tensor) -> torch.Tensor:
    return DepthwiseConvShared.apply(x, kernel)


__all__ = [
    "DepthwiseConvShared",
    "depthwise_conv_shared",
    "THREADS_PER_BLOCK",
    "TTILE",
    "HTILE",
    "shared_memory_bytes",
    "FWD_TIMES",
    "BWD_IN_TIMES",
    "BWD_K_TIMES",
    "reset_timing_collectors",
]
