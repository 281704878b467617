"""Drop-in for the reference's long-row module ``kernels/shared_l192.py``
(public surface as ``kernels/warp_tiled.py``, ``__all__`` at :1020-1031;
benchmarked at B16384 H128 L192 K192, benchmark/benchmark_gmc_vs_shared_l192.py:14-17).

Rows and taps up to 48 take the specialised kernels; anything up to L = 192,
K = 256 takes ``pt_dwconv1d_{fwd,dx,dk}_long_f32`` at FP32 accuracy, dK
deterministic and written into ``gk`` (no zero-init, as the reference's
one-thread-per-tap kernel writes it, :966-1001). Every launch is
host-synchronous and appends its kernel time (ms) to ``FWD_TIMES`` /
``BWD_IN_TIMES`` / ``BWD_K_TIMES`` (:741-780).

Differences by design: importing needs no GPU (the reference raises at
import without CUDA, :15-18; CPU tensors raise at the first call instead);
L > 192 or K > 256 raise ``ValueError``; ``CudaContextGuard`` and
``TorchCudaInterop`` are the no-PyCUDA shims of the ``warp_tiled`` mirror;
the launch constants keep the reference's values (:109-118).
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
