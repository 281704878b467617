"""Host runtime of the MI355X depthwise Conv1D path.

Mirrors the runtime surface of the reference's ``kernels/warp_tiled_ampere.py``
(constants :62-74, helpers :174-272, ``KernelEventCollector`` :278-330,
``AmpereWarpRuntime`` :625-846, ``install_runtime``/``get_runtime`` :852-860,
``DepthConvAmpere`` :863-898, ``reference_depthwise_conv`` :901-903,
``summarize_kernel_times`` :990-1018, ``configure_torch`` :1658-1663), backed
by the hipcc-built C ABI in ``libpathtile_hip.so`` instead of PyCUDA.

Differences from the reference, by design:

* "Warps" are 64-lane wavefronts. ``waves_per_block`` (FWD/dX) takes
  1, 2, 4, 8 or 16; ``bwdk_block`` (dK threads per workgroup) is a multiple
  of 64 in [64, 768].
* Launches go on torch's current stream of the tensors' device (the
  reference used the legacy default stream); there is no context push.
* Nothing falls back to PyTorch: a missing or failing native library raises.
"""

from __future__ import annotations

import ctypes
import math
import threading
from collections import OrderedDict
from dataclasses import dataclass
from typing import Any, Callable

import torch

from . import _lib

# =============================================================================
# Workload constants (kernels/warp_tiled_ampere.py:62-74)
# =============================================================================
WAVE_SIZE = 64
WARP_SIZE = WAVE_SIZE  # the reference's name; 64 lanes on CDNA
MAX_L = 48
MAX_K = 48
LONG_MAX_L = 192   # long-row kernels (pt_dwconv1d_*_long_f32)
LONG_MAX_K = 256

DEFAULT_B = 16_384
DEFAULT_H = 128
DEFAULT_L = 48
DEFAULT_K = 48

# Launch defaults: the frozen PathTile policy for MI355X when the tuner has
# installed one (pathtile_amd/tune/frozen_policy.json), else these values.
FROZEN_POLICY_PATH = __import__("pathlib").Path(__file__).resolve().parent / "tune" / "frozen_policy.json"


def _frozen_policy() -> dict:
    try:
        import json

        return dict(json.loads(FROZEN_POLICY_PATH.read_text()).get("selected", {}))
    except (OSError, ValueError):
        return {}


_POLICY = _frozen_policy()
DEFAULT_WAVES_PER_BLOCK = int(_POLICY.get("fwd_waves_per_block", 4))
DEFAULT_DX_WAVES_PER_BLOCK = int(_POLICY.get("dx_waves_per_block", 4))
DEFAULT_WARPS_PER_BLOCK = DEFAULT_WAVES_PER_BLOCK
DEFAULT_BWDK_BTILE = 64  # samples per wave chunk (one per lane)
# The reference packs 4 taps per thread (:64-66); here each lane packs the
# whole tap window of its channel (both rows are register resident), and the
# default matrix-core dK contracts over the batch instead.
DEFAULT_BWDK_KPACK = 4
DEFAULT_BWDK_BLOCK = int(_POLICY.get("dk_threads_per_block", 128))

ALLOWED_WAVES = (1, 2, 4, 8, 16)
MAX_BWDK_BLOCK = 768
# Deterministic-dK workspaces a runtime keeps, one per (device, stream).
WORKSPACE_STREAMS = 4


# =============================================================================
# GPU profile (the reference keys profiles by CUDA compute capability, :76-171)
# =============================================================================
@dataclass(frozen=True)
class GPUProfile:
    key: str
    display_name: str
    gfx_arch: str
    peak_bandwidth_gbps: float
    compute_units: int
    simds_per_cu: int
    max_waves_per_simd: int
    vgprs_per_simd_lane: int
    lds_per_cu: int
    max_threads_per_block: int

    @property
    def limits(self) -> dict[str, int]:
        return {
            "max_waves_per_cu": self.simds_per_cu * self.max_waves_per_simd,
            "vgprs_per_simd_lane": self.vgprs_per_simd_lane,
            "lds_per_cu": self.lds_per_cu,
            "max_threads_per_block": self.max_threads_per_block,
        }


GPU_PROFILES = {
    "gfx950": GPUProfile(
        key="mi355x",
        display_name="AMD Instinct MI355X",
        gfx_arch="gfx950",
        peak_bandwidth_gbps=8000.0,
        compute_units=256,
        simds_per_cu=4,
        max_waves_per_simd=8,
        vgprs_per_simd_lane=512,
        lds_per_cu=160 * 1024,
        max_threads_per_block=1024,
    ),
}
MI355X = GPU_PROFILES["gfx950"]


def detect_gpu_profile(device_id: int) -> GPUProfile:
    props = torch.cuda.get_device_properties(device_id)
    arch = str(getattr(props, "gcnArchName", "")).split(":")[0]
    if arch not in GPU_PROFILES:
        raise RuntimeError(
            f"This build targets gfx950 (MI355X); detected {arch or 'unknown'}"
        )
    return GPU_PROFILES[arch]


# =============================================================================
# Small helpers (kernels/warp_tiled_ampere.py:174-272)
# =============================================================================
def ceil_div(a: int, b: int) -> int:
    return (a + b - 1) // b


def round_up(value: int, quantum: int) -> int:
    return ceil_div(value, quantum) * quantum


def max_abs_diff(a: torch.Tensor, b: torch.Tensor) -> float:
    return float((a - b).abs().max().item())


def normalized_max_abs(a: torch.Tensor, b: torch.Tensor, eps: float = 1e-12) -> float:
    scale = max(float(b.abs().max().item()), eps)
    return max_abs_diff(a, b) / scale


def estimate_gpu_occupancy(
    threads_per_block: int,
    regs_per_thread: int,
    lds_per_block: int,
    profile: GPUProfile = MI355X,
) -> dict[str, Any]:
    """Analytical waves-per-CU estimate for CDNA (the reference's
    estimate_gpu_occupancy, :187-256, redone for 64-lane waves): VGPRs are
    allocated in granules of 8 per lane from a 512-entry file per SIMD lane,
    LDS in 512-byte granules from 160 KiB per CU, at most 8 waves per SIMD.
    rocprofv3 counters remain authoritative for achieved occupancy."""
    if threads_per_block <= 0 or threads_per_block > profile.max_threads_per_block:
        raise ValueError("threads_per_block must be in [1, 1024]")
    waves_per_block = ceil_div(threads_per_block, WAVE_SIZE)
    regs = max(8, round_up(max(regs_per_thread, 1), 8))
    waves_per_simd_regs = min(profile.max_waves_per_simd, profile.vgprs_per_simd_lane // regs)
    by_regs = (waves_per_simd_regs * profile.simds_per_cu) // waves_per_block
    lds = round_up(lds_per_block, 512) if lds_per_block else 0
    by_lds = profile.lds_per_cu // lds if lds else 1 << 30
    by_waves = (profile.simds_per_cu * profile.max_waves_per_simd) // waves_per_block
    constraints = {"registers": by_regs, "lds": by_lds, "waves": by_waves}
    blocks = max(0, min(constraints.values()))
    waves = blocks * waves_per_block
    limiting = [k for k, v in constraints.items() if v == blocks]
    return {
        "threads_per_block": threads_per_block,
        "waves_per_block": waves_per_block,
        "regs_per_thread": regs_per_thread,
        "allocated_regs_per_lane": regs,
        "lds_bytes_per_block": lds_per_block,
        "resident_blocks_per_cu_est": blocks,
        "active_waves_per_cu_est": waves,
        "occupancy_est": waves / (profile.simds_per_cu * profile.max_waves_per_simd),
        "limiting_resources_est": ",".join(limiting),
        "gpu_profile": profile.key,
    }


# The reference's backward-compatible name (kernels/warp_tiled_ampere.py:260).
estimate_ampere_occupancy = estimate_gpu_occupancy


def minimum_algorithmic_bytes(B: int, H: int, L: int, K: int) -> int:
    """Unique input/output bytes, not profiler-measured DRAM traffic
    (kernels/warp_tiled_ampere.py:263-266)."""
    return (2 * B * H * L + H * K) * 4


def algorithmic_bandwidth_gbps(num_bytes: int, time_ms: float) -> float:
    if time_ms <= 0:
        return float("nan")
    return num_bytes / (time_ms / 1000.0) / 1e9


def useful_flops(B: int, H: int, L: int, K: int) -> int:
    """2 * FMAs that touch a real element
    (scripts/prototype_pathtile_shape_queries.py:62-68)."""
    p = K // 2
    per_row = sum(max(0, min(L, L - (j - p)) - max(0, -(j - p))) for j in range(K))
    return 2 * B * H * per_row


# =============================================================================
# Event collection without per-kernel synchronisation (:278-330)
# =============================================================================
class KernelEventCollector:
    """Records a start/end event pair around each launch on torch's current
    stream (the stream the kernels run on) and resolves them lazily."""

    def __init__(self) -> None:
        self.enabled = False
        self._context: dict[str, Any] = {}
        self._events: list[tuple[str, Any, Any, dict[str, Any]]] = []

    def set_context(self, **context: Any) -> None:
        self._context = dict(context)

    def clear(self) -> None:
        self._events.clear()
        self._context.clear()

    def launch(
        self,
        phase: str,
        launch_fn: Callable[[], None],
        metadata: dict[str, Any] | None = None,
    ) -> None:
        if not self.enabled:
            launch_fn()
            return
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record()
        launch_fn()
        end.record()
        row = dict(self._context)
        if metadata:
            row.update(metadata)
        self._events.append((phase, start, end, row))

    def rows(self, synchronize: bool = True) -> list[dict[str, Any]]:
        if synchronize:
            torch.cuda.synchronize()
        out: list[dict[str, Any]] = []
        counts: dict[str, int] = {}
        for phase, start, end, meta in self._events:
            counts[phase] = counts.get(phase, 0) + 1
            out.append({**meta, "phase": phase, "run_id": counts[phase],
                        "runtime_ms": float(start.elapsed_time(end))})
        return out

    def resolve(self, synchronize: bool = True):
        import pandas as pd

        return pd.DataFrame(self.rows(synchronize))


KERNEL_EVENTS = KernelEventCollector()


def summarize_kernel_times(raw):
    """Per-phase mean/median/std/p05/p95 (kernels/warp_tiled_ampere.py:990-1018)."""
    import numpy as np
    import pandas as pd

    columns = ["phase", "runs", "mean_ms", "median_ms", "std_ms", "p05_ms", "p95_ms"]
    if raw.empty:
        return pd.DataFrame(columns=columns)
    rows = []
    for phase, group in raw.groupby("phase", sort=False):
        v = group["runtime_ms"].to_numpy(dtype=float)
        rows.append({
            "phase": phase,
            "runs": len(v),
            "mean_ms": float(np.mean(v)),
            "median_ms": float(np.median(v)),
            "std_ms": float(np.std(v, ddof=1)) if len(v) > 1 else 0.0,
            "p05_ms": float(np.quantile(v, 0.05)),
            "p95_ms": float(np.quantile(v, 0.95)),
        })
    return pd.DataFrame(rows, columns=columns)


# =============================================================================
# Runtime
# =============================================================================
def _ptr(t: torch.Tensor) -> ctypes.c_void_p:
    return ctypes.c_void_p(t.data_ptr())


def _stream_handle(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


# FWD/dX kernel choice of HipWarpRuntime(rows_algo=...): the C ABI's
# PT_ROWS_AUTO, PT_ROWS_VALU and PT_ROWS_MATRIX.
ROWS_ALGOS = {"auto": _lib.PT_ROWS_AUTO, "valu": _lib.PT_ROWS_VALU, "mfma": _lib.PT_ROWS_MATRIX}

# PT_KERNEL_* ids of the FWD / dX kernels -> (kernel template, matrix cores?)
ROWS_KERNELS = {
    _lib.PT_KERNEL_FWD: ("dwconv_rows_kernel<FWD>", False),
    _lib.PT_KERNEL_DX: ("dwconv_rows_kernel<DX>", False),
    _lib.PT_KERNEL_FWD_STREAM: ("dwconv_stream_kernel<FWD>", False),
    _lib.PT_KERNEL_DX_STREAM: ("dwconv_stream_kernel<DX>", False),
    _lib.PT_KERNEL_FWD_CG: ("dwconv_rows_cg_kernel<FWD>", True),
    _lib.PT_KERNEL_DX_CG: ("dwconv_rows_cg_kernel<DX>", True),
    _lib.PT_KERNEL_FWD_CG16: ("dwconv_rows_cg_kernel<FWD, 16 channels>", True),
    _lib.PT_KERNEL_DX_CG16: ("dwconv_rows_cg_kernel<DX, 16 channels>", True),
}


def rows_kernel_id(B: int, H: int, L: int, K: int, dx: bool = False,
                   waves_per_block: int = 4, algo: str = "auto",
                   aligned16: bool = True) -> int:
    """PT_KERNEL_* id of the kernel a FWD (dx=False) or dX launch of this
    shape would run on the current device (-1: nothing, B or H = 0); the
    library's dispatch itself answers (pt_rows_kernel_id), so no restated
    rule can drift from it. Raises ValueError where the launch would."""
    out = ctypes.c_int(-1)
    st = _lib.load().pt_rows_kernel_id(int(B), int(H), int(L), int(K), int(waves_per_block),
                                       ROWS_ALGOS[algo], int(bool(aligned16)), int(bool(dx)),
                                       ctypes.byref(out))
    _lib.check(st, "pt_rows_kernel_id")
    return int(out.value)


def rows_kernel_name(B: int, H: int, L: int, K: int, dx: bool = False,
                     waves_per_block: int = 4, algo: str = "auto",
                     aligned16: bool = True) -> str:
    """Name of the kernel rows_kernel_id reports ("none" for empty calls)."""
    kid = rows_kernel_id(B, H, L, K, dx, waves_per_block, algo, aligned16)
    return ROWS_KERNELS[kid][0] if kid >= 0 else "none"


def rows_on_matrix_cores(B: int, H: int, L: int, K: int, dx: bool = False,
                         waves_per_block: int = 4, aligned16: bool = True) -> bool:
    """True where the library serves this FWD/dX call on the matrix cores."""
    kid = rows_kernel_id(B, H, L, K, dx, waves_per_block, "auto", aligned16)
    return kid >= 0 and ROWS_KERNELS[kid][1]


class HipWarpRuntime:
    """Owns the launch configuration of the three paths and launches them
    through the C ABI (the reference's AmpereWarpRuntime, :625-846).

    waves_per_block     FWD wavefronts per workgroup (1, 2, 4, 8, 16)
    dx_waves_per_block  dX wavefronts per workgroup (default: waves_per_block)
    bwdk_block          dK threads per workgroup (multiple of 64, <= 768)
    bwdk_btile          samples per dK wave chunk; fixed at 64 (one per lane)
    fast_math           accepted for signature compatibility; the kernels are
                        FMA-only, so it changes nothing
    rows_algo           FWD/dX kernel: "auto" (PATHTILE_ROWS_ALGO, then the
                        library's rule), "valu" (the VALU kernels: the
                        reference's fmaf chain bit for bit) or "mfma" (the
                        matrix cores wherever the layout allows); an explicit
                        choice takes precedence over PATHTILE_ROWS_ALGO
    """

    def __init__(
        self,
        waves_per_block: int = DEFAULT_WAVES_PER_BLOCK,
        bwdk_btile: int = DEFAULT_BWDK_BTILE,
        bwdk_block: int = DEFAULT_BWDK_BLOCK,
        fast_math: bool = False,
        *,
        dx_waves_per_block: int | None = None,
        rows_algo: str = "auto",
    ) -> None:
        if rows_algo not in ROWS_ALGOS:
            raise ValueError(f"rows_algo must be one of {', '.join(ROWS_ALGOS)}")
        if dx_waves_per_block is None:
            dx_waves_per_block = (DEFAULT_DX_WAVES_PER_BLOCK
                                  if waves_per_block == DEFAULT_WAVES_PER_BLOCK
                                  else waves_per_block)
        dxw = dx_waves_per_block
        for value in (waves_per_block, dxw):
            if value not in ALLOWED_WAVES:
                raise ValueError("waves_per_block must be one of 1,2,4,8,16")
        if bwdk_btile != 64:
            raise ValueError("This paper-confirmed version fixes BWDK_BTILE=64")
        if not (WAVE_SIZE <= bwdk_block <= MAX_BWDK_BLOCK) or bwdk_block % WAVE_SIZE:
            raise ValueError(
                "bwdk_block must be a multiple of 64 in the inclusive range [64, 768]"
            )
        self.waves_per_block = int(waves_per_block)
        self.dx_waves_per_block = int(dxw)
        self.warps_per_block = self.waves_per_block  # reference attribute name
        self.fwd_block = self.waves_per_block * WAVE_SIZE
        self.bwdk_btile = int(bwdk_btile)
        self.bwdk_block = int(bwdk_block)
        self.fast_math = bool(fast_math)
        self.rows_algo = rows_algo
        self._rows_algo_id = ROWS_ALGOS[rows_algo]
        self.technique = "WaveRow-mi355x"
        # The device current at construction, as the reference records it
        # (:662-664); launches still follow each call's tensors. The profile
        # is detected from it (gfx950 only) where a GPU is present.
        if torch.cuda.is_available():
            self.device_id: int | None = torch.cuda.current_device()
            self.device: torch.device | None = torch.device("cuda", self.device_id)
            self.profile = detect_gpu_profile(self.device_id)
        else:
            self.device_id = None
            self.device = None
            self.profile = MI355X
        self._lib = _lib.load()
        self._closed = False
        self._ws_lock = threading.Lock()
        # (device index, stream handle) -> (stream, workspace), least
        # recently used first
        self._workspaces: OrderedDict[tuple[int, int], tuple[Any, torch.Tensor]] = OrderedDict()

    # ------------------------------------------------------------------ checks
    @staticmethod
    def _check_shapes(x: torch.Tensor, k: torch.Tensor) -> tuple[int, int, int, int]:
        """Same checks and messages as kernels/warp_tiled_ampere.py:704-717."""
        if not x.is_cuda or not k.is_cuda:
            raise ValueError("x and k must be CUDA tensors")
        if x.dtype != torch.float32 or k.dtype != torch.float32:
            raise ValueError("Only FP32 is supported")
        if x.ndim != 3 or k.ndim != 2:
            raise ValueError("Expected x[B,H,L] and k[H,K]")
        B, H, L = map(int, x.shape)
        Hk, K = map(int, k.shape)
        if H != Hk:
            raise ValueError("x and k channel dimensions do not match")
        if L > MAX_L or K > MAX_K:
            raise ValueError(f"Specialized kernels require L<={MAX_L}, K<={MAX_K}")
        return B, H, L, K

    @staticmethod
    def _require_contiguous(*tensors: torch.Tensor) -> None:
        for t in tensors:
            if not t.is_contiguous():
                raise ValueError("Tensors passed to the runtime must be contiguous")

    def _check_open(self) -> None:
        if self._closed:
            raise RuntimeError("runtime has been closed")

    # ---------------------------------------------------------------- launches
    def launch_fwd(
        self,
        x: torch.Tensor,
        k: torch.Tensor,
        y: torch.Tensor,
        collector: KernelEventCollector | None = None,
    ) -> None:
        self._check_open()
        B, H, L, K = self._check_shapes(x, k)
        if y.shape != x.shape or y.dtype != torch.float32 or y.device != x.device:
            raise ValueError("y must be a float32 tensor shaped like x on x's device")
        self._require_contiguous(x, k, y)

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.pt_dwconv1d_fwd_f32_algo(
                    _ptr(x), _ptr(k), _ptr(y), B, H, L, K,
                    self.waves_per_block, self._rows_algo_id, _stream_handle(x.device))
            _lib.check(st, "pt_dwconv1d_fwd_f32_algo")

        (collector or KERNEL_EVENTS).launch("fwd", launch, {"B": B, "H": H, "L": L, "K": K})

    def launch_bwd_input(
        self,
        gy: torch.Tensor,
        k: torch.Tensor,
        gx: torch.Tensor,
        collector: KernelEventCollector | None = None,
    ) -> None:
        self._check_open()
        B, H, L, K = self._check_shapes(gy, k)
        if gx.shape != gy.shape or gx.dtype != torch.float32 or gx.device != gy.device:
            raise ValueError("gx must be a float32 tensor shaped like gy on gy's device")
        self._require_contiguous(gy, k, gx)

        def launch() -> None:
            with torch.cuda.device(gy.device):
                st = self._lib.pt_dwconv1d_dx_f32_algo(
                    _ptr(gy), _ptr(k), _ptr(gx), B, H, L, K,
                    self.dx_waves_per_block, self._rows_algo_id, _stream_handle(gy.device))
            _lib.check(st, "pt_dwconv1d_dx_f32_algo")

        (collector or KERNEL_EVENTS).launch("bwd_input", launch, {"B": B, "H": H, "L": L, "K": K})

    def _check_bwd_weight(self, gy, x, gk, K) -> tuple[int, int, int]:
        """Same checks and messages as kernels/warp_tiled_ampere.py:772-793."""
        if not gy.is_cuda or not x.is_cuda or not gk.is_cuda:
            raise ValueError("gy, x, and gk must be CUDA tensors")
        if gy.dtype != torch.float32 or x.dtype != torch.float32 or gk.dtype != torch.float32:
            raise ValueError("Only FP32 is supported")
        if gy.shape != x.shape:
            raise ValueError("gy and x must have the same [B,H,L] shape")
        if x.ndim != 3:
            raise ValueError("Expected x[B,H,L] and k[H,K]")
        B, H, L = map(int, x.shape)
        if tuple(gk.shape) != (H, K):
            raise ValueError(f"gk must have shape {(H, K)}")
        if L > MAX_L or K > MAX_K:
            raise ValueError(f"Specialized kernels require L<={MAX_L}, K<={MAX_K}")
        self._require_contiguous(gy, x, gk)
        return B, H, L

    def launch_bwd_weight(
        self,
        gy: torch.Tensor,
        x: torch.Tensor,
        gk: torch.Tensor,
        K: int,
        collector: KernelEventCollector | None = None,
        zero_first: bool = False,
    ) -> None:
        """Atomic dK: accumulates into gk, which the caller zeroes (as in the
        reference, :890-893) unless zero_first=True, which clears gk inside the
        same launch sequence (so "dK including zero-init" is one timed call)."""
        self._check_open()
        K = int(K)
        B, H, L = self._check_bwd_weight(gy, x, gk, K)

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.pt_dwconv1d_dk_atomic_f32(
                    _ptr(gy), _ptr(x), _ptr(gk), B, H, L, K, self.bwdk_block,
                    1 if zero_first else 0, _stream_handle(x.device))
            _lib.check(st, "pt_dwconv1d_dk_atomic_f32")

        phase = "bwd_weight_zero" if zero_first else "bwd_weight"
        (collector or KERNEL_EVENTS).launch(phase, launch, {"B": B, "H": H, "L": L, "K": K})

    def dk_workspace_bytes(self, B: int, H: int, L: int, K: int) -> int:
        out = ctypes.c_size_t(0)
        st = self._lib.pt_dwconv1d_dk_det_workspace_bytes(B, H, L, K, self.bwdk_block,
                                                          ctypes.byref(out))
        _lib.check(st, "pt_dwconv1d_dk_det_workspace_bytes")
        return int(out.value)

    def _get_workspace(self, nbytes: int, device: torch.device) -> torch.Tensor:
        """Reusable byte workspace for the deterministic dK
        (kernels/warp_tiled_noatomic_optimized.py:1448-1471), one per
        (device, stream): the launch goes to torch's current stream of the
        device, and each stream keeps its own buffer, so launches on two
        streams never share partials. The buffer is allocated from torch's
        caching allocator while that stream is current, so when it is
        replaced by a larger one, or dropped, its memory returns to that
        stream's pool and is reused only by work ordered after the launches
        that read it. At most WORKSPACE_STREAMS (device, stream) buffers are
        kept, the least recently used dropped first, so callers that make
        short-lived streams do not pile up workspaces; an entry holds its
        stream, so no live entry's handle can be recycled by a new stream."""
        stream = torch.cuda.current_stream(device)
        key = (device.index if device.index is not None else torch.cuda.current_device(),
               int(stream.cuda_stream))
        with self._ws_lock:
            entry = self._workspaces.get(key)
            if entry is None or entry[1].numel() < nbytes:
                with torch.cuda.stream(stream):
                    ws = torch.empty(max(nbytes, 256), dtype=torch.uint8, device=device)
                self._workspaces[key] = (stream, ws)
            self._workspaces.move_to_end(key)
            while len(self._workspaces) > WORKSPACE_STREAMS:
                self._workspaces.popitem(last=False)
            return self._workspaces[key][1]

    def launch_bwd_weight_deterministic(
        self,
        gy: torch.Tensor,
        x: torch.Tensor,
        gk: torch.Tensor,
        K: int,
        collector: KernelEventCollector | None = None,
    ) -> None:
        """Two-pass dK: per-batch-tile partials, then a fixed-order reduction
        that overwrites gk (no zero-init). Bitwise reproducible for a fixed
        shape, bwdk_block and input alignment (16-byte aligned or not) on a
        given device: the range count that partitions the sums may be capped
        by the device's CU count and the kernel's occupancy
        (kernels/warp_tiled_noatomic_optimized.py:1473)."""
        self._check_open()
        K = int(K)
        B, H, L = self._check_bwd_weight(gy, x, gk, K)
        nbytes = self.dk_workspace_bytes(B, H, L, K)
        ws = self._get_workspace(nbytes, x.device)

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.pt_dwconv1d_dk_det_f32(
                    _ptr(gy), _ptr(x), _ptr(gk), _ptr(ws), ws.numel(),
                    B, H, L, K, self.bwdk_block, _stream_handle(x.device))
            _lib.check(st, "pt_dwconv1d_dk_det_f32")

        (collector or KERNEL_EVENTS).launch("bwd_weight_det", launch, {"B": B, "H": H, "L": L, "K": K})

    # ------------------------------------------------------------- BF16 I/O
    # No counterpart in the reference (FP32 only): bfloat16 activations and
    # gradients, FP32 taps and dK, FP32 accumulation on the matrix cores.
    @staticmethod
    def _check_bf16(t: torch.Tensor, k: torch.Tensor, name: str) -> tuple[int, int, int, int]:
        if not t.is_cuda or not k.is_cuda:
            raise ValueError(f"{name} and k must be CUDA tensors")
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} must be bfloat16")
        if k.dtype != torch.float32:
            raise ValueError("k must be float32")
        if t.ndim != 3 or k.ndim != 2:
            raise ValueError(f"Expected {name}[B,H,L] and k[H,K]")
        B, H, L = map(int, t.shape)
        Hk, K = map(int, k.shape)
        if H != Hk:
            raise ValueError(f"Channel mismatch: {name} H={H}, k H={Hk}")
        if L > MAX_L or K > MAX_K:
            raise ValueError(f"Specialized kernels require L<={MAX_L}, K<={MAX_K}")
        return B, H, L, K

    def launch_fwd_bf16(self, x: torch.Tensor, k: torch.Tensor, y: torch.Tensor,
                        collector: KernelEventCollector | None = None) -> None:
        self._check_open()
        B, H, L, K = self._check_bf16(x, k, "x")
        if y.dtype != torch.bfloat16 or y.shape != x.shape:
            raise ValueError("y must be a bfloat16 tensor shaped like x")
        self._require_contiguous(x, k, y)

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.pt_dwconv1d_fwd_bf16(_ptr(x), _ptr(k), _ptr(y), B, H, L, K,
                                                    _stream_handle(x.device))
            _lib.check(st, "pt_dwconv1d_fwd_bf16")

        (collector or KERNEL_EVENTS).launch("fwd_bf16", launch, {"B": B, "H": H, "L": L, "K": K})

    def launch_bwd_input_bf16(self, gy: torch.Tensor, k: torch.Tensor, gx: torch.Tensor,
                              collector: KernelEventCollector | None = None) -> None:
        self._check_open()
        B, H, L, K = self._check_bf16(gy, k, "gy")
        if gx.dtype != torch.bfloat16 or gx.shape != gy.shape:
            raise ValueError("gx must be a bfloat16 tensor shaped like gy")
        self._require_contiguous(gy, k, gx)

        def launch() -> None:
            with torch.cuda.device(gy.device):
                st = self._lib.pt_dwconv1d_dx_bf16(_ptr(gy), _ptr(k), _ptr(gx), B, H, L, K,
                                                   _stream_handle(gy.device))
            _lib.check(st, "pt_dwconv1d_dx_bf16")

        (collector or KERNEL_EVENTS).launch("bwd_input_bf16", launch, {"B": B, "H": H, "L": L, "K": K})

    def _check_bf16_dk(self, gy, x, gk, K) -> tuple[int, int, int]:
        if not gy.is_cuda or not x.is_cuda or not gk.is_cuda:
            raise ValueError("gy, x, and gk must be CUDA tensors")
        if gy.dtype != torch.bfloat16 or x.dtype != torch.bfloat16 or gk.dtype != torch.float32:
            raise ValueError("gy and x must be bfloat16, gk float32")
        if gy.shape != x.shape or x.ndim != 3:
            raise ValueError("gy and x must have the same [B,H,L] shape")
        B, H, L = map(int, x.shape)
        if tuple(gk.shape) != (H, K):
            raise ValueError(f"gk must have shape {(H, K)}")
        if L > MAX_L or K > MAX_K:
            raise ValueError(f"Specialized kernels require L<={MAX_L}, K<={MAX_K}")
        self._require_contiguous(gy, x, gk)
        return B, H, L

    def launch_bwd_weight_bf16(self, gy: torch.Tensor, x: torch.Tensor, gk: torch.Tensor, K: int,
                               collector: KernelEventCollector | None = None,
                               zero_first: bool = False) -> None:
        """Atomic BF16 dK: accumulates into the FP32 gk (zero_first clears it)."""
        self._check_open()
        K = int(K)
        B, H, L = self._check_bf16_dk(gy, x, gk, K)

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.pt_dwconv1d_dk_atomic_bf16(
                    _ptr(gy), _ptr(x), _ptr(gk), B, H, L, K, self.bwdk_block,
                    1 if zero_first else 0, _stream_handle(x.device))
            _lib.check(st, "pt_dwconv1d_dk_atomic_bf16")

        (collector or KERNEL_EVENTS).launch("bwd_weight_bf16", launch, {"B": B, "H": H, "L": L, "K": K})

    def launch_bwd_weight_deterministic_bf16(self, gy: torch.Tensor, x: torch.Tensor,
                                             gk: torch.Tensor, K: int,
                                             collector: KernelEventCollector | None = None) -> None:
        """Two-pass BF16 dK: overwrites the FP32 gk, bitwise reproducible."""
        self._check_open()
        K = int(K)
        B, H, L = self._check_bf16_dk(gy, x, gk, K)
        out = ctypes.c_size_t(0)
        st = self._lib.pt_dwconv1d_dk_det_bf16_workspace_bytes(B, H, L, K, self.bwdk_block,
                                                               ctypes.byref(out))
        _lib.check(st, "pt_dwconv1d_dk_det_bf16_workspace_bytes")
        ws = self._get_workspace(int(out.value), x.device)

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.pt_dwconv1d_dk_det_bf16(
                    _ptr(gy), _ptr(x), _ptr(gk), _ptr(ws), ws.numel(),
                    B, H, L, K, self.bwdk_block, _stream_handle(x.device))
            _lib.check(st, "pt_dwconv1d_dk_det_bf16")

        (collector or KERNEL_EVENTS).launch("bwd_weight_det_bf16", launch, {"B": B, "H": H, "L": L, "K": K})

    def launch_bwd_weight_channels_last(self, x: torch.Tensor, gy: torch.Tensor,
                                        dw: torch.Tensor, gz: int = 1,
                                        collector: KernelEventCollector | None = None,
                                        zero_first: bool = False) -> None:
        """Channels-last FP32 dK through the Flash-DWC bridge ABI
        (``flash_dk_fp32``, benchmark/flashdwc_fp32_bridge.cu:6-34): x and gy
        are [B, 1, L, H], dw is [1, K, H] and is accumulated into
        (zero_first clears it). ``gz`` is the bridge's batch split, checked as
        the bridge checks it (B % gz == 0, (B / gz) % 16 == 0)."""
        self._check_open()
        if not x.is_cuda or not gy.is_cuda or not dw.is_cuda:
            raise ValueError("x, gy, and dw must be CUDA tensors")
        if x.dtype != torch.float32 or gy.dtype != torch.float32 or dw.dtype != torch.float32:
            raise ValueError("x, gy, and dw must be float32")
        if x.ndim != 4 or x.shape[1] != 1 or gy.shape != x.shape:
            raise ValueError("x and gy must have the same [B,1,L,H] shape")
        if dw.ndim != 3 or dw.shape[0] != 1 or dw.shape[2] != x.shape[3]:
            raise ValueError("dw must have shape [1,K,H]")
        self._require_contiguous(x, gy, dw)
        B, _, L, H = map(int, x.shape)
        K = int(dw.shape[1])
        if zero_first:
            dw.zero_()

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.flash_dk_fp32(_ptr(x), _ptr(gy), _ptr(dw), B, H, L, K, int(gz),
                                             _stream_handle(x.device))
            _lib.check(st, "flash_dk_fp32")

        (collector or KERNEL_EVENTS).launch("bwd_weight_cl", launch, {"B": B, "H": H, "L": L, "K": K})

    # ------------------------------------------------------------- long rows
    @staticmethod
    def _check_long(x: torch.Tensor, k: torch.Tensor, what: str = "k") -> tuple[int, int, int, int]:
        if not x.is_cuda or not k.is_cuda:
            raise ValueError(f"x and {what} must be CUDA tensors")
        if x.dtype != torch.float32 or k.dtype != torch.float32:
            raise ValueError("Only FP32 is supported")
        if x.ndim != 3 or k.ndim != 2:
            raise ValueError("Expected x[B,H,L] and k[H,K]")
        B, H, L = map(int, x.shape)
        Hk, K = map(int, k.shape)
        if H != Hk:
            raise ValueError("x and k channel dimensions do not match")
        if L > LONG_MAX_L or K > LONG_MAX_K:
            raise ValueError(f"Long-row kernels require L<={LONG_MAX_L}, K<={LONG_MAX_K}")
        return B, H, L, K

    def launch_fwd_long(self, x: torch.Tensor, k: torch.Tensor, y: torch.Tensor,
                        collector: KernelEventCollector | None = None) -> None:
        """FWD for rows up to 192 with up to 256 taps (matrix cores, FP32
        accuracy; see pt_dwconv1d_fwd_long_f32)."""
        self._check_open()
        B, H, L, K = self._check_long(x, k)
        if y.shape != x.shape or y.dtype != torch.float32 or y.device != x.device:
            raise ValueError("y must be a float32 tensor shaped like x on x's device")
        self._require_contiguous(x, k, y)

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.pt_dwconv1d_fwd_long_f32(_ptr(x), _ptr(k), _ptr(y), B, H, L, K,
                                                        _stream_handle(x.device))
            _lib.check(st, "pt_dwconv1d_fwd_long_f32")

        (collector or KERNEL_EVENTS).launch("fwd_long", launch, {"B": B, "H": H, "L": L, "K": K})

    def launch_bwd_input_long(self, gy: torch.Tensor, k: torch.Tensor, gx: torch.Tensor,
                              collector: KernelEventCollector | None = None) -> None:
        """dX for rows up to 192 with up to 256 taps (matrix cores, FP32
        accuracy; see pt_dwconv1d_dx_long_f32)."""
        self._check_open()
        B, H, L, K = self._check_long(gy, k)
        if gx.shape != gy.shape or gx.dtype != torch.float32 or gx.device != gy.device:
            raise ValueError("gx must be a float32 tensor shaped like gy on gy's device")
        self._require_contiguous(gy, k, gx)

        def launch() -> None:
            with torch.cuda.device(gy.device):
                st = self._lib.pt_dwconv1d_dx_long_f32(_ptr(gy), _ptr(k), _ptr(gx), B, H, L, K,
                                                       _stream_handle(gy.device))
            _lib.check(st, "pt_dwconv1d_dx_long_f32")

        (collector or KERNEL_EVENTS).launch("bwd_input_long", launch, {"B": B, "H": H, "L": L, "K": K})

    def launch_bwd_weight_long(self, gy: torch.Tensor, x: torch.Tensor, gk: torch.Tensor, K: int,
                               collector: KernelEventCollector | None = None) -> None:
        """Deterministic dK for rows up to 192 with up to 256 taps: overwrites
        gk, bitwise reproducible (fixed-order partials and reduction)."""
        self._check_open()
        K = int(K)
        if not gy.is_cuda or not x.is_cuda or not gk.is_cuda:
            raise ValueError("gy, x, and gk must be CUDA tensors")
        if gy.dtype != torch.float32 or x.dtype != torch.float32 or gk.dtype != torch.float32:
            raise ValueError("Only FP32 is supported")
        if gy.shape != x.shape or x.ndim != 3:
            raise ValueError("gy and x must have the same [B,H,L] shape")
        B, H, L = map(int, x.shape)
        if tuple(gk.shape) != (H, K):
            raise ValueError(f"gk must have shape {(H, K)}")
        if L > LONG_MAX_L or K > LONG_MAX_K:
            raise ValueError(f"Long-row kernels require L<={LONG_MAX_L}, K<={LONG_MAX_K}")
        self._require_contiguous(gy, x, gk)
        out = ctypes.c_size_t(0)
        st = self._lib.pt_dwconv1d_dk_long_workspace_bytes(B, H, L, K, ctypes.byref(out))
        _lib.check(st, "pt_dwconv1d_dk_long_workspace_bytes")
        ws = self._get_workspace(int(out.value), x.device)

        def launch() -> None:
            with torch.cuda.device(x.device):
                st = self._lib.pt_dwconv1d_dk_long_f32(
                    _ptr(gy), _ptr(x), _ptr(gk), _ptr(ws), ws.numel(), B, H, L, K,
                    _stream_handle(x.device))
            _lib.check(st, "pt_dwconv1d_dk_long_f32")

        (collector or KERNEL_EVENTS).launch("bwd_weight_long", launch, {"B": B, "H": H, "L": L, "K": K})

    # ------------------------------------------------------------- reporting
    def rows_kernel(self, B: int, H: int, L: int, K: int, dx: bool = False,
                    aligned16: bool = True) -> str:
        """Name of the kernel this runtime's FWD (or dX) launch would run
        for the shape (the library's own dispatch, queried through
        pt_rows_kernel_id on the current device)."""
        wpb = self.dx_waves_per_block if dx else self.waves_per_block
        return rows_kernel_name(B, H, L, K, dx=dx, waves_per_block=wpb,
                                algo=self.rows_algo, aligned16=aligned16)

    def kernel_attributes(self, kernel_id: int, L: int, K: int) -> dict[str, int]:
        regs, lds, scratch, maxt = (ctypes.c_int(0) for _ in range(4))
        st = self._lib.pt_kernel_attributes(kernel_id, L, K, ctypes.byref(regs),
                                            ctypes.byref(lds), ctypes.byref(scratch),
                                            ctypes.byref(maxt))
        _lib.check(st, "pt_kernel_attributes")
        return {"regs": regs.value, "static_lds": lds.value,
                "scratch_bytes": scratch.value, "max_threads": maxt.value}

    def dynamic_lds_bytes(self, kernel_id: int, L: int, K: int, config: int) -> int:
        out = ctypes.c_int(0)
        st = self._lib.pt_dynamic_lds_bytes(kernel_id, L, K, config, ctypes.byref(out))
        _lib.check(st, "pt_dynamic_lds_bytes")
        return int(out.value)

    def resource_report(self, L: int = DEFAULT_L, K: int = DEFAULT_K):
        """Registers, LDS, scratch and estimated occupancy of the kernels that
        serve (L, K) (the reference's resource_report, :814-833). FWD and dX
        list every kernel that can serve them: the VALU tile kernel and, for
        K <= 9 on rows of L % 4 == 0, the VALU streaming kernel, both at this
        runtime's waves per block; the channel-group matrix-core kernel (8
        waves; long FMA chains on 16-byte aligned tensors with H % 8 == 0)
        and, for 33 <= L <= 48, its 16-channel variant (16 waves,
        H % 16 == 0)."""
        import pandas as pd

        rows = []
        cg_block = 8 * WAVE_SIZE
        cg16_block = 16 * WAVE_SIZE
        stream = K <= 9 and L % 4 == 0
        cg16 = 33 <= L <= 48
        fwd_wpb, dx_wpb = self.waves_per_block, self.dx_waves_per_block
        kernels = [("fwd", _lib.PT_KERNEL_FWD, self.fwd_block, fwd_wpb)]
        if stream:
            kernels.append(("fwd_stream", _lib.PT_KERNEL_FWD_STREAM, self.fwd_block, fwd_wpb))
        kernels.append(("fwd_matrix_cores", _lib.PT_KERNEL_FWD_CG, cg_block, fwd_wpb))
        if cg16:
            kernels.append(("fwd_matrix_cores_16", _lib.PT_KERNEL_FWD_CG16, cg16_block, fwd_wpb))
        kernels.append(("bwd_input", _lib.PT_KERNEL_DX, dx_wpb * WAVE_SIZE, dx_wpb))
        if stream:
            kernels.append(("bwd_input_stream", _lib.PT_KERNEL_DX_STREAM, dx_wpb * WAVE_SIZE, dx_wpb))
        kernels.append(("bwd_input_matrix_cores", _lib.PT_KERNEL_DX_CG, cg_block, dx_wpb))
        if cg16:
            kernels.append(("bwd_input_matrix_cores_16", _lib.PT_KERNEL_DX_CG16, cg16_block, dx_wpb))
        kernels.append(("bwd_weight", _lib.PT_KERNEL_DK, self.bwdk_block, self.bwdk_block))
        for name, kid, block, cfg in kernels:
            a = self.kernel_attributes(kid, L, K)
            lds = a["static_lds"] + self.dynamic_lds_bytes(kid, L, K, cfg)
            row = {"kernel": name, "L": L, "K": K}
            row.update(estimate_gpu_occupancy(block, a["regs"], lds, self.profile))
            row["scratch_bytes"] = a["scratch_bytes"]
            rows.append(row)
        return pd.DataFrame(rows)

    def close(self) -> None:
        if self._closed:
            return
        if torch.cuda.is_available():
            torch.cuda.synchronize()
        self._workspaces.clear()
        self._closed = True


# The reference's class name; waves, not 32-lane warps (see module docstring).
AmpereWarpRuntime = HipWarpRuntime

_RUNTIME: HipWarpRuntime | None = None


def install_runtime(runtime: HipWarpRuntime) -> None:
    global _RUNTIME
    _RUNTIME = runtime


def get_runtime() -> HipWarpRuntime:
    if _RUNTIME is None:
        raise RuntimeError("CUDA runtime has not been installed")
    return _RUNTIME


def get_or_create_runtime() -> HipWarpRuntime:
    """The installed runtime, or a default one installed on first use."""
    global _RUNTIME
    if _RUNTIME is None:
        _RUNTIME = HipWarpRuntime()
    return _RUNTIME


# =============================================================================
# autograd drop-in (kernels/warp_tiled_ampere.py:863-898)
# =============================================================================
class DepthConvAmpere(torch.autograd.Function):
    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
        runtime = get_runtime()
        x_c = x.contiguous()
        k_c = k.contiguous()
        B, H, L, K = runtime._check_shapes(x_c, k_c)
        y = torch.empty_like(x_c)
        runtime.launch_fwd(x_c, k_c, y)
        ctx.save_for_backward(x_c, k_c)
        ctx.params = (B, H, L, K)
        return y

    @staticmethod
    def backward(ctx: Any, gy: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        runtime = get_runtime()
        x_c, k_c = ctx.saved_tensors
        B, H, L, K = ctx.params
        gy_c = gy.contiguous()
        if tuple(gy_c.shape) != (B, H, L):
            raise ValueError("Unexpected gradient shape")
        gx = torch.empty_like(x_c)
        runtime.launch_bwd_input(gy_c, k_c, gx)
        # The reference zero-fills gk and adds into it with atomics
        # (:890-893). The two-pass dK overwrites gk instead: no memset, a
        # fixed summation order (reproducible gradients), and on MI355X the
        # same time as zero-fill + atomics.
        gk = torch.empty_like(k_c)
        runtime.launch_bwd_weight_deterministic(gy_c, x_c, gk, K)
        return gx, gk


def depthwise_conv_ampere(x: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    return DepthConvAmpere.apply(x, k)


class DepthConvBf16(torch.autograd.Function):
    """BF16-I/O counterpart of DepthConvAmpere (no reference counterpart):
    x, y and the activation gradients are bfloat16, k and its gradient FP32
    (the two-pass deterministic dK)."""

    @staticmethod
    def forward(ctx: Any, x: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
        runtime = get_runtime()
        x_c = x.contiguous()
        k_c = k.contiguous()
        B, H, L, K = runtime._check_bf16(x_c, k_c, "x")
        y = torch.empty_like(x_c)
        runtime.launch_fwd_bf16(x_c, k_c, y)
        ctx.save_for_backward(x_c, k_c)
        ctx.params = (B, H, L, K)
        return y

    @staticmethod
    def backward(ctx: Any, gy: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        runtime = get_runtime()
        x_c, k_c = ctx.saved_tensors
        B, H, L, K = ctx.params
        gy_c = gy.to(torch.bfloat16).contiguous()
        gx = gk = None
        if ctx.needs_input_grad[0]:
            gx = torch.empty_like(x_c)
            runtime.launch_bwd_input_bf16(gy_c, k_c, gx)
        if ctx.needs_input_grad[1]:
            gk = torch.empty_like(k_c)
            runtime.launch_bwd_weight_deterministic_bf16(gy_c, x_c, gk, K)
        return gx, gk


def depthwise_conv_bf16(x: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """y = conv(x, k) for bfloat16 x and FP32 k (L % 4 == 0, H % 8 == 0)."""
    return DepthConvBf16.apply(x, k)


def reference_depthwise_conv(x: torch.Tensor, k: torch.Tensor) -> torch.Tensor:
    """PyTorch form of the same op (kernels/warp_tiled_ampere.py:901-903); the
    S4ConvD "pytorch" backend, not a fallback of the HIP path."""
    import torch.nn.functional as F

    y = F.conv1d(x, k.unsqueeze(1), padding=k.shape[1] // 2, groups=x.shape[1])
    return y[..., : x.shape[-1]].contiguous()


def configure_torch() -> None:
    """kernels/warp_tiled_ampere.py:1658-1663."""
    if not torch.cuda.is_available():
        raise RuntimeError("CUDA is not available")
    torch.backends.cudnn.allow_tf32 = False
    torch.backends.cuda.matmul.allow_tf32 = False
    torch.backends.cudnn.benchmark = True


__all__ = [
    "WAVE_SIZE", "WARP_SIZE", "MAX_L", "MAX_K", "LONG_MAX_L", "LONG_MAX_K",
    "DEFAULT_B", "DEFAULT_H", "DEFAULT_L", "DEFAULT_K",
    "DEFAULT_WAVES_PER_BLOCK", "DEFAULT_DX_WAVES_PER_BLOCK", "DEFAULT_WARPS_PER_BLOCK",
    "DEFAULT_BWDK_BTILE", "DEFAULT_BWDK_KPACK", "DEFAULT_BWDK_BLOCK",
    "GPUProfile", "GPU_PROFILES", "MI355X", "detect_gpu_profile",
    "ceil_div", "round_up", "max_abs_diff", "normalized_max_abs",
    "estimate_gpu_occupancy", "estimate_ampere_occupancy", "minimum_algorithmic_bytes",
    "algorithmic_bandwidth_gbps", "useful_flops",
    "KernelEventCollector", "KERNEL_EVENTS", "summarize_kernel_times",
    "HipWarpRuntime", "AmpereWarpRuntime",
    "install_runtime", "get_runtime", "get_or_create_runtime",
    "DepthConvAmpere", "depthwise_conv_ampere", "reference_depthwise_conv",
    "DepthConvBf16", "depthwise_conv_bf16",
    "configure_torch",
]
