"""S4ConvD, the model that calls the depthwise Conv1D path, with the block's
skip term fused into the convolution.

Follows the reference's S4 model (``kernels/warp_tiled_ampere.py:1116-1224``):
``S4ConvKernel`` builds the H x L convolution kernel from a diagonal
state-space parameterisation (:1122-1169), ``S4ConvBlock`` applies it with a
per-channel skip term, a GELU, dropout and a GLU output projection
(:1172-1190), ``Model`` stacks the blocks between a linear encoder and
decoder (:1193-1215), and ``rmsle`` is the training loss (:1218-1224).
Parameter names, shapes, registration order and initial distributions are
the reference's, so its checkpoints load unchanged.

The fused skip term. The block computes ``y = conv(x, k) + x * skip[h]``
(:1187-1188). The skip term reads ``x[b,h,t]``, which is what tap
``p = K // 2`` of the convolution reads (``y[t]`` gets ``w[p] * x[t+p-p]``).
So ``conv(x, k) + skip * x = conv(x, k')`` with ``k' = k`` plus ``skip`` on
column p, and the HIP path runs the block's FWD and dX with ``k'``: the skip
term costs no pass over ``y``. In backward, ``dL/dk = dK`` (``k' - k`` does
not depend on k) and ``dL/dskip = dK[:, p]``.

Backend switch: ``pathtile_amd.kernels.warp_tiled_ampere.TRAIN_CONV_BACKEND``
(the reference's module global, :1119), read on every forward call:
``"warp"`` runs the HIP path with the fused skip term, ``"pytorch"`` runs the
reference's composition (``reference_depthwise_conv`` + a separate skip add).
"""

from __future__ import annotations

import math
from typing import Any

import torch
from torch import nn

from .runtime import MAX_L, get_runtime, reference_depthwise_conv


def _backend() -> str:
    from .kernels import warp_tiled_ampere

    return warp_tiled_ampere.TRAIN_CONV_BACKEND


class DepthConvSkipAmpere(torch.autograd.Function):
    """``conv(x, k) + x * skip[:, None]`` on the HIP path, the skip term
    folded into tap ``K // 2``; backward returns ``(gx, gk, gskip)`` with
    the two-pass deterministic dK."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, k: torch.Tensor, skip: torch.Tensor) -> torch.Tensor:
        runtime = get_runtime()
        x_c = x.contiguous()
        k_c = k.contiguous()
        B, H, L, K = runtime._check_shapes(x_c, k_c)
        if tuple(skip.shape) != (H,):
            raise ValueError(f"skip must have shape {(H,)}")
        if skip.dtype != torch.float32 or skip.device != k_c.device:
            raise ValueError("skip must be a float32 tensor on the kernel's device")
        p = K // 2
        k_eff = k_c.clone()
        k_eff[:, p] += skip
        y = torch.empty_like(x_c)
        runtime.launch_fwd(x_c, k_eff, y)
        ctx.save_for_backward(x_c, k_eff)
        ctx.params = (B, H, L, K)
        return y

    @staticmethod
    def backward(ctx: Any, gy: torch.Tensor):
        runtime = get_runtime()
        x_c, k_eff = ctx.saved_tensors
        B, H, L, K = ctx.params
        gy_c = gy.contiguous()
        gx = gk = gskip = None
        if ctx.needs_input_grad[0]:
            gx = torch.empty_like(x_c)
            runtime.launch_bwd_input(gy_c, k_eff, gx)
        if ctx.needs_input_grad[1] or ctx.needs_input_grad[2]:
            dk = torch.empty_like(k_eff)
            runtime.launch_bwd_weight_deterministic(gy_c, x_c, dk, K)
            if ctx.needs_input_grad[1]:
                gk = dk
            if ctx.needs_input_grad[2]:
                gskip = dk[:, K // 2].contiguous()
        return gx, gk, gskip


def depthwise_conv_skip_ampere(x: torch.Tensor, k: torch.Tensor, skip: torch.Tensor) -> torch.Tensor:
    return DepthConvSkipAmpere.apply(x, k, skip)


class S4ConvKernel(nn.Module):
    """Diagonal SSM convolution kernel (:1122-1169). For channel h and tap t:
    ``k[h, t] = 2 Re( sum_n C_eff[h, n] * exp(dt[h] A[h, n] t) )`` with
    ``A = -exp(log_A_re) + i A_im``, ``C = C_re + i C_im`` and
    ``C_eff = C (exp(dt A) - 1) / A`` (zero-order-hold discretisation)."""

    def __init__(self, hidden_dim: int, state_dim: int) -> None:
        super().__init__()
        self.H = hidden_dim
        self.N = state_dim
        half = state_dim // 2
        lo, hi = math.log(0.001), math.log(0.1)
        self.log_dt = nn.Parameter(torch.rand(hidden_dim) * (hi - lo) + lo)
        self.C_re = nn.Parameter(torch.randn(hidden_dim, half))
        self.C_im = nn.Parameter(torch.randn(hidden_dim, half))
        self.log_A_re = nn.Parameter(torch.randn(hidden_dim, half))
        self.A_im = nn.Parameter(torch.ones(hidden_dim, half))

    def build_kernel(self, taps: int, device: torch.device) -> torch.Tensor:
        dt = self.log_dt.exp()
        A = torch.complex(-self.log_A_re.exp(), self.A_im)
        C = torch.complex(self.C_re, self.C_im)
        dtA = A * dt[:, None]
        C_eff = C * (dtA.exp() - 1.0) / A
        t = torch.arange(taps, device=device, dtype=torch.float32)
        powers = torch.exp(dtA[:, :, None] * t)  # [H, N/2, taps]
        # elementwise product and sum over n (no batched matmul)
        return (2.0 * (C_eff[:, :, None] * powers).sum(dim=1).real).contiguous()

    def forward(self, x: torch.Tensor, skip: torch.Tensor | None = None) -> torch.Tensor:
        """``conv(x, k)`` with ``k = build_kernel(L)``; with ``skip`` the block's
        skip term is added (fused into the convolution on the "warp" backend)."""
        _, H, L = x.shape
        if H != self.H:
            raise ValueError(f"Expected H={self.H}, got {H}")
        if L > MAX_L:
            raise ValueError(f"Warp-tiled paper kernel supports L<={MAX_L}")
        k = self.build_kernel(L, x.device)
        backend = _backend()
        if backend == "warp":
            if skip is None:
                from .runtime import depthwise_conv_ampere

                return depthwise_conv_ampere(x.contiguous(), k)
            return depthwise_conv_skip_ampere(x.contiguous(), k, skip)
        if backend == "pytorch":
            y = reference_depthwise_conv(x.contiguous(), k)
            return y if skip is None else y + x * skip.unsqueeze(-1)
        raise RuntimeError(f"Unknown training backend: {backend}")


class S4ConvBlock(nn.Module):
    """Depthwise S4 convolution + skip, GELU, dropout, GLU projection and a
    residual connection (:1172-1190); input and output are ``[B, L, H]``."""

    def __init__(self, hidden_dim: int, state_dim: int, dropout: float) -> None:
        super().__init__()
        self.skip = nn.Parameter(torch.randn(hidden_dim))
        self.kernel_layer = S4ConvKernel(hidden_dim, state_dim)
        self.activation = nn.GELU()
        self.dropout = nn.Dropout(dropout)
        self.output_linear = nn.Sequential(
            nn.Conv1d(hidden_dim, 2 * hidden_dim, kernel_size=1),
            nn.GLU(dim=1),
        )

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x_hl = x.transpose(1, 2).contiguous()
        y = self.kernel_layer(x_hl, self.skip)
        y = self.output_linear(self.activation(self.dropout(y)))
        return y.transpose(1, 2) + x


class Model(nn.Module):
    """Encoder, ``num_blocks`` S4ConvD blocks, decoder; ``x`` is
    ``[B, L, input_dim]`` and the output is the last step's ``[B, output_dim]``
    (:1193-1215)."""

    def __init__(
        self,
        state_dim: int = 64,
        hidden_dim: int = 128,
        input_dim: int = 4,
        output_dim: int = 1,
        num_blocks: int = 4,
        dropout: float = 0.01,
    ) -> None:
        super().__init__()
        self.encoder = nn.Linear(input_dim, hidden_dim)
        self.blocks = nn.ModuleList(
            [S4ConvBlock(hidden_dim, state_dim, dropout) for _ in range(num_blocks)]
        )
        self.decoder = nn.Linear(hidden_dim, output_dim)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        x = self.encoder(x)
        for block in self.blocks:
            x = block(x)
        return self.decoder(x)[:, -1, :]


def rmsle(prediction: torch.Tensor, target: torch.Tensor) -> torch.Tensor:
    """Root mean squared log error on non-negative parts (:1218-1224)."""
    p = prediction.reshape(-1).clamp(min=0.0)
    t = target.reshape(-1).clamp(min=0.0)
    return torch.sqrt((p.log1p() - t.log1p()).square().mean() + 1e-12)


__all__ = [
    "DepthConvSkipAmpere", "depthwise_conv_skip_ampere",
    "S4ConvKernel", "S4ConvBlock", "Model", "rmsle",
]
