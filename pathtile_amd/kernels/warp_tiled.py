"""Drop-in for the reference's ``kernels/warp_tiled.py`` API, on MI355X.

Same public names, argument meaning, exception types/messages and timing
side effects as the reference module (``__all__`` at
kernels/warp_tiled.py:1020-1031); underneath, the three paths run the
hand-written gfx950 kernels of ``libpathtile_hip.so``:

* ``DepthwiseConvShared.forward``  -> the FWD kernel chosen per shape (the
  long-row kernel above L or K = 48);
* ``DepthwiseConvShared.backward`` -> dX kernel, then the deterministic
  two-pass dK, which writes ``gk`` directly like the reference's shared
  kernel does (``gk = torch.empty_like(kernel)``, kernels/warp_tiled.py:902).

Every launch is host-synchronous and its kernel time (ms, HIP events) is
appended to ``FWD_TIMES`` / ``BWD_IN_TIMES`` / ``BWD_K_TIMES``, as the
reference's ``_time_kernel`` does (:747-780).

Differences from the reference, by design:

* Importing this module does not need a GPU; the reference raises at import
  without CUDA (:15-18). Here the first call with CPU tensors raises
  ``ValueError("x and kernel must be CUDA tensors")``.
* Rows and taps up to 48 run the specialised kernels; longer rows (L up to
  192, K up to 256) run the long-row matrix-core kernels, and beyond that
  the call raises ``ValueError``. The reference's shared kernels have no
  stated bound (their dK's shared memory, 2 * 64 * L * 4 bytes, caps L near
  96 in practice).
* ``CudaContextGuard`` is a no-op context manager (HIP has no context stack to
  push) and ``TorchCudaInterop.as_gpuarray`` validates like the reference and
  returns the tensor itself (there is no PyCUDA GPUArray).
* The legacy launch constants (TTILE, HTILE, THREADS_PER_BLOCK,
  BWD_K_B_TILE) and the two shared-memory size helpers keep the reference's
  values as documented constants; the HIP kernels use their own geometry.

The S4ConvD-facing ``warp_tiled_ampere`` names (``DepthConvAmpere``,
``depthwise_conv_ampere``, the runtime class, ...) are re-exported here too.
"""

from __future__ import annotations

import torch

from .. import runtime as _rt
from ..runtime import (  # noqa: F401  (re-exported S4ConvD / tuner surface)
    AmpereWarpRuntime,
    DEFAULT_BWDK_BLOCK,
    DEFAULT_BWDK_BTILE,
    DEFAULT_BWDK_KPACK,
    DEFAULT_WARPS_PER_BLOCK,
    DEFAULT_WAVES_PER_BLOCK,
    DepthConvAmpere,
    HipWarpRuntime,
    KERNEL_EVENTS,
    KernelEventCollector,
    MAX_K,
    MAX_L,
    configure_torch,
    depthwise_conv_ampere,
    get_runtime,
    install_runtime,
    minimum_algorithmic_bytes,
    normalized_max_abs,
    reference_depthwise_conv,
)

# =============================================================================
# Legacy launch constants (kernels/warp_tiled.py:109-118)
# =============================================================================
TTILE = 32
HTILE = 16
THREADS_PER_BLOCK = TTILE * HTILE  # 512
BWD_K_B_TILE = 64


class CudaContextGuard:
    """No-op: the HIP runtime keeps one current device per thread and torch
    already selects it (reference: PyCUDA primary-context push, :30-38)."""

    def __enter__(self):
        return self

    def __exit__(self, exc_type, exc_val, exc_tb):
        return False


class TorchCudaInterop:
    """Validation of the reference's zero-copy view (:44-87). The HIP path
    passes raw device pointers, so the "array" is the tensor itself."""

    @staticmethod
    def as_gpuarray(tensor: torch.Tensor) -> torch.Tensor:
        if not tensor.is_cuda:
            raise ValueError("Tensor must be on CUDA")
        if tensor.dtype != torch.float32:
            raise TypeError(f"Expected torch.float32, got {tensor.dtype}")
        if not tensor.is_contiguous():
            raise ValueError("Tensor must be contiguous")
        return tensor


def bwd_kernel_shared_memory_bytes(L: int) -> int:
    """Reference backward-weight shared memory, 2 * 64 * L * 4 (:690-705)."""
    return 2 * BWD_K_B_TILE * L * 4


def shared_memory_bytes(K: int) -> int:
    """Reference forward/backward-input shared memory,
    HTILE * (TTILE + K - 1) * 4 (:708-729)."""
    return HTILE * (TTILE + K - 1) * 4


# =============================================================================
# Timing collectors (:736-745)
# =============================================================================
FWD_TIMES: list[float] = []
BWD_IN_TIMES: list[float] = []
BWD_K_TIMES: list[float] = []


def reset_timing_collectors():
    FWD_TIMES.clear()
    BWD_IN_TIMES.clear()
    BWD_K_TIMES.clear()


def _time_kernel(launch) -> float:
    """Synchronise, bracket one launch with events on the current stream,
    wait for it and return the elapsed ms (the reference's _time_kernel,
    :747-780)."""
    torch.cuda.synchronize()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record()
    launch()
    end.record()
    end.synchronize()
    return float(start.elapsed_time(end))


def _runtime() -> HipWarpRuntime:
    return _rt.get_or_create_runtime()


# =============================================================================
# Autograd (:787-1017)
# =============================================================================
def _is_short(L: int, K: int) -> bool:
    return L <= MAX_L and K <= MAX_K


def make_shared_function(fwd_times: list, bwd_in_times: list, bwd_k_times: list,
                         module: str = __name__):
    """The reference's ``DepthwiseConvShared`` (:787-1005) appending its
    kernel times to the given lists. Checks and messages in the reference's
    order (:796-830). Rows and taps up to 48 run the specialised kernels;
    longer ones (L up to 192, K up to 256) the long-row matrix-core kernels.
    Backward: dX, then a deterministic dK written into a fresh ``gk``
    (``gk = torch.empty_like(kernel)``, :902)."""

    class DepthwiseConvShared(torch.autograd.Function):

        @staticmethod
        def forward(ctx, x: torch.Tensor, kernel: torch.Tensor) -> torch.Tensor:
            if not x.is_cuda or not kernel.is_cuda:
                raise ValueError("x and kernel must be CUDA tensors")
            if x.dtype != torch.float32:
                raise TypeError("x must be float32")
            if kernel.dtype != torch.float32:
                raise TypeError("kernel must be float32")
            if x.ndim != 3:
                raise ValueError(f"x must be [B,H,L], got {tuple(x.shape)}")
            if kernel.ndim != 2:
                raise ValueError(f"kernel must be [H,K], got {tuple(kernel.shape)}")

            x = x.contiguous()
            kernel = kernel.contiguous()

            B, H, L = x.shape
            Hk, K = kernel.shape
            if H != Hk:
                raise ValueError(f"Channel mismatch: x H={H}, kernel H={Hk}")
            if L > _rt.LONG_MAX_L or K > _rt.LONG_MAX_K:
                raise ValueError(
                    f"Long-row kernels require L<={_rt.LONG_MAX_L}, K<={_rt.LONG_MAX_K}")

            ctx.save_for_backward(x, kernel)
            ctx.params = (B, H, L, K)

            y = torch.empty_like(x)
            rt = _runtime()
            fwd = rt.launch_fwd if _is_short(L, K) else rt.launch_fwd_long
            fwd_times.append(_time_kernel(lambda: fwd(x, kernel, y)))
            return y

        @staticmethod
        def backward(ctx, grad_y: torch.Tensor):
            x, kernel = ctx.saved_tensors
            B, H, L, K = ctx.params
            grad_y = grad_y.contiguous()
            gx = torch.empty_like(x)
            gk = torch.empty_like(kernel)
            rt = _runtime()
            if _is_short(L, K):
                dx, dk = rt.launch_bwd_input, rt.launch_bwd_weight_deterministic
            else:
                dx, dk = rt.launch_bwd_input_long, rt.launch_bwd_weight_long
            bwd_in_times.append(_time_kernel(lambda: dx(grad_y, kernel, gx)))
            bwd_k_times.append(_time_kernel(lambda: dk(grad_y, x, gk, K)))
            return gx, gk

    DepthwiseConvShared.__qualname__ = "DepthwiseConvShared"
    DepthwiseConvShared.__module__ = module
    return DepthwiseConvShared


DepthwiseConvShared = make_shared_function(FWD_TIMES, BWD_IN_TIMES, BWD_K_TIMES)


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
