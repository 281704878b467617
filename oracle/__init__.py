"""CPU oracle for the depthwise Conv1D hot path (FWD, dX, dK; the FP32
reference chains for L, K <= 48, the FP64 sums for L, K <= 256).

TEST INFRASTRUCTURE ONLY. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this package, and only as the
checker. ``pathtile_amd`` never imports it and never falls back to it.

Three restatements of the reference semantics, each pinned by the tests in
``tests/test_oracle.py``:

* ``fwd_f32_refchain`` / ``dx_f32_refchain`` (C): the reference kernels' exact
  per-output FP32 ``fmaf`` chain (kernels/warp_tiled_ampere.py:404-433 and
  :472-501), so an implementation of that chain matches bit for bit.
* ``fwd_f64`` / ``dx_f64`` / ``dk_f64`` (C): FP64 accumulation of the exact
  float products; ``dk_f64`` follows benchmark/check_dk_fp64_comparison.py:29-39.
* ``pytorch_depthwise_same`` (torch, CPU): the reference's PyTorch boundary
  (benchmark/benchmark_shape_sweep_ampere.py:220-239) and
  ``reference_depthwise_conv`` (kernels/warp_tiled_ampere.py:901-903).
* ``brute_*`` (pure Python, tiny shapes): the defining double sums.

The C library is ``oracle/liboracle.so``, built by ``oracle/Makefile``
(``make -C oracle``); it is built on first use when missing.
"""

from __future__ import annotations

import ctypes
import math
import os
import subprocess
import threading
from pathlib import Path

import numpy as np

_HERE = Path(__file__).resolve().parent
_LIB_PATH = _HERE / "liboracle.so"
_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None

MAX_L = 48          # the FP32 reference chains (the reference kernels' range)
MAX_K = 48
MAX_LONG = 256      # the FP64 sums (same formulas, long rows)


def build(force: bool = False) -> Path:
    """Compile ``liboracle.so`` with the committed Makefile."""
    if force or not _LIB_PATH.exists():
        cmd = ["make", "-C", str(_HERE)]
        if force:
            cmd.append("-B")
        subprocess.run(cmd, check=True, capture_output=True, text=True)
    return _LIB_PATH


def _lib() -> ctypes.CDLL:
    global _LIB
    with _LOCK:
        if _LIB is None:
            build()
            lib = ctypes.CDLL(str(_LIB_PATH))
            fp = ctypes.POINTER(ctypes.c_float)
            dp = ctypes.POINTER(ctypes.c_double)
            i = ctypes.c_int
            for name, out in (
                ("oracle_fwd_f32_refchain", fp),
                ("oracle_dx_f32_refchain", fp),
                ("oracle_fwd_f64", dp),
                ("oracle_dx_f64", dp),
                ("oracle_dk_f64", dp),
            ):
                fn = getattr(lib, name)
                fn.argtypes = [fp, fp, out, i, i, i, i]
                fn.restype = ctypes.c_int
            _LIB = lib
        return _LIB


def _f32(a) -> np.ndarray:
    if hasattr(a, "detach"):  # torch tensor
        a = a.detach().cpu().numpy()
    a = np.ascontiguousarray(a, dtype=np.float32)
    return a


def _shape(x: np.ndarray, w: np.ndarray, limit: int = MAX_L) -> tuple[int, int, int, int]:
    if x.ndim != 3 or w.ndim != 2:
        raise ValueError("expected x[B,H,L] and w[H,K]")
    B, H, L = x.shape
    Hw, K = w.shape
    if H != Hw:
        raise ValueError("channel mismatch")
    if L < 1 or K < 1 or L > limit or K > limit:
        raise ValueError(f"oracle supports 1 <= L, K <= {limit}")
    return int(B), int(H), int(L), int(K)


def _call(name: str, a: np.ndarray, b: np.ndarray, out: np.ndarray, dims) -> None:
    fp = ctypes.POINTER(ctypes.c_float)
    outp = ctypes.POINTER(ctypes.c_double if out.dtype == np.float64 else ctypes.c_float)
    rc = getattr(_lib(), name)(
        a.ctypes.data_as(fp), b.ctypes.data_as(fp), out.ctypes.data_as(outp), *dims
    )
    if rc != 0:
        raise ValueError(f"{name} rejected shape {dims} (status {rc})")


def fwd_f32_refchain(x, w) -> np.ndarray:
    """y in the reference's FP32 fmaf order (kernels/warp_tiled_ampere.py:404-433)."""
    x, w = _f32(x), _f32(w)
    dims = _shape(x, w)
    y = np.empty_like(x)
    _call("oracle_fwd_f32_refchain", x, w, y, dims)
    return y


def dx_f32_refchain(dy, w) -> np.ndarray:
    """dX in the reference's FP32 fmaf order (kernels/warp_tiled_ampere.py:472-501)."""
    dy, w = _f32(dy), _f32(w)
    dims = _shape(dy, w)
    dx = np.empty_like(dy)
    _call("oracle_dx_f32_refchain", dy, w, dx, dims)
    return dx


def fwd_f64(x, w) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    dims = _shape(x, w, MAX_LONG)
    y = np.empty(x.shape, dtype=np.float64)
    _call("oracle_fwd_f64", x, w, y, dims)
    return y


def dx_f64(dy, w) -> np.ndarray:
    dy, w = _f32(dy), _f32(w)
    dims = _shape(dy, w, MAX_LONG)
    dx = np.empty(dy.shape, dtype=np.float64)
    _call("oracle_dx_f64", dy, w, dx, dims)
    return dx


def dk_f64(dy, x, K: int) -> np.ndarray:
    """dK[h,j] = sum_{b,t} dy[b,h,t] x[b,h,t+j-p] in FP64
    (benchmark/check_dk_fp64_comparison.py:29-39)."""
    dy, x = _f32(dy), _f32(x)
    if dy.shape != x.shape:
        raise ValueError("dy and x must have the same [B,H,L] shape")
    B, H, L = map(int, x.shape)
    if L < 1 or K < 1 or L > MAX_LONG or K > MAX_LONG:
        raise ValueError(f"oracle supports 1 <= L, K <= {MAX_LONG}")
    dk = np.empty((H, K), dtype=np.float64)
    _call("oracle_dk_f64", dy, x, dk, (B, H, L, K))
    return dk


# ---------------------------------------------------------------------------
# Pure-Python restatement of the defining sums (tiny shapes only).
# ---------------------------------------------------------------------------
def brute_fwd(x, w) -> np.ndarray:
    x, w = _f32(x), _f32(w)
    B, H, L, K = _shape(x, w)
    p = K // 2
    y = np.zeros((B, H, L), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            for t in range(L):
                acc = 0.0
                for j in range(K):
                    s = t + j - p
                    if 0 <= s < L:
                        acc += float(x[b, h, s]) * float(w[h, j])
                y[b, h, t] = acc
    return y


def brute_dx(dy, w) -> np.ndarray:
    dy, w = _f32(dy), _f32(w)
    B, H, L, K = _shape(dy, w)
    p = K // 2
    dx = np.zeros((B, H, L), dtype=np.float64)
    for b in range(B):
        for h in range(H):
            for s in range(L):
                acc = 0.0
                for j in range(K):
                    t = s - j + p
                    if 0 <= t < L:
                        acc += float(dy[b, h, t]) * float(w[h, j])
                dx[b, h, s] = acc
    return dx


def brute_dk(dy, x, K: int) -> np.ndarray:
    dy, x = _f32(dy), _f32(x)
    B, H, L = x.shape
    p = K // 2
    dk = np.zeros((H, K), dtype=np.float64)
    for h in range(H):
        for j in range(K):
            acc = 0.0
            for b in range(B):
                for t in range(L):
                    s = t + j - p
                    if 0 <= s < L:
                        acc += float(dy[b, h, t]) * float(x[b, h, s])
            dk[h, j] = acc
    return dk


def fsum_dk_coefficient(dy, x, K: int, h: int, j: int) -> float:
    """One dK coefficient with math.fsum over the exact valid range
    (benchmark/diagnose_dk_correctness.py:21,193)."""
    dy, x = _f32(dy), _f32(x)
    B, H, L = x.shape
    p = K // 2
    lo, hi = max(0, p - j), min(L, L + p - j)
    terms = []
    for b in range(B):
        for t in range(lo, hi):
            terms.append(float(dy[b, h, t]) * float(x[b, h, t + j - p]))
    return math.fsum(terms)


def valid_tap_range(L: int, K: int, j: int) -> tuple[int, int]:
    """[lo, hi) of output positions t that tap j meets
    (benchmark/diagnose_dk_correctness.py:21)."""
    p = K // 2
    return max(0, p - j), min(L, L + p - j)


def useful_fma_per_row(L: int, K: int) -> int:
    """FMAs of one row that touch a real element:
    sum_j max(0, min(L, L - s_j) - max(0, -s_j)), s_j = j - p
    (scripts/prototype_pathtile_shape_queries.py:62-68)."""
    p = K // 2
    total = 0
    for j in range(K):
        s = j - p
        total += max(0, min(L, L - s) - max(0, -s))
    return total


# ---------------------------------------------------------------------------
# torch restatements of the reference's PyTorch boundary (CPU here).
# ---------------------------------------------------------------------------
def pytorch_depthwise_same(x, k):
    """benchmark/benchmark_shape_sweep_ampere.py:220-239: explicit asymmetric
    pad (K//2, K-1-K//2) then grouped conv1d."""
    import torch.nn.functional as F

    K = int(k.shape[1])
    left = K // 2
    right = K - 1 - left
    x_pad = F.pad(x, (left, right))
    return F.conv1d(x_pad, k.unsqueeze(1), bias=None, stride=1, padding=0,
                    groups=int(x.shape[1]))


def reference_depthwise_conv(x, k):
    """kernels/warp_tiled_ampere.py:901-903: symmetric padding K//2, cropped
    to the first L outputs."""
    import torch.nn.functional as F

    y = F.conv1d(x, k.unsqueeze(1), padding=k.shape[1] // 2, groups=x.shape[1])
    return y[..., : x.shape[-1]].contiguous()


def torch_grads(x, k, dy, fn=None):
    """(y, dX, dK) through torch autograd of ``fn`` (default
    pytorch_depthwise_same) on whatever device/dtype the inputs have."""
    import torch

    fn = fn or pytorch_depthwise_same
    xr = x.detach().clone().requires_grad_(True)
    kr = k.detach().clone().requires_grad_(True)
    y = fn(xr, kr)
    gx, gk = torch.autograd.grad(y, (xr, kr), dy)
    return y.detach(), gx.detach(), gk.detach()


def normalized_max_abs(a, b, eps: float = 1e-12) -> float:
    """max|a-b| / max|b| (kernels/warp_tiled_ampere.py:182-184)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    if a.size == 0:
        return 0.0
    scale = max(float(np.abs(b).max()), eps)
    return float(np.abs(a - b).max()) / scale


def make_inputs(B: int, H: int, L: int, K: int, seed: int):
    """Seeded CPU inputs in the order x, w, dY: x, dY ~ N(0,1), w ~ N(0,1/K)
    (benchmark/check_dk_fp64_comparison.py:25-27 draws from one CPU
    torch.Generator in order)."""
    import torch

    g = torch.Generator().manual_seed(int(seed))
    x = torch.randn(B, H, L, generator=g, dtype=torch.float32)
    w = torch.randn(H, K, generator=g, dtype=torch.float32) / math.sqrt(K)
    dy = torch.randn(B, H, L, generator=g, dtype=torch.float32)
    return x, w, dy


__all__ = [
    "build",
    "fwd_f32_refchain",
    "dx_f32_refchain",
    "fwd_f64",
    "dx_f64",
    "dk_f64",
    "brute_fwd",
    "brute_dx",
    "brute_dk",
    "fsum_dk_coefficient",
    "valid_tap_range",
    "useful_fma_per_row",
    "pytorch_depthwise_same",
    "reference_depthwise_conv",
    "torch_grads",
    "normalized_max_abs",
    "make_inputs",
]
