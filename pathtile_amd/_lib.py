"""ctypes binding of ``libpathtile_hip.so`` (C ABI in ``include/pathtile_hip.h``).

torch is imported first on purpose: its bundled HIP runtime registers the
soname ``libamdhip64.so.7``, and the dynamic loader then resolves this
library's dependency to that same runtime, so both share one HIP context and
torch's streams are valid handles here. There is no CPU fallback: if the
library is missing or fails to load, every entry point raises.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch  # noqa: F401  (must precede the CDLL load, see module docstring)

LIB_PATH = Path(__file__).resolve().parent / "libpathtile_hip.so"

PT_OK = 0
PT_ERR_NULL = -1
PT_ERR_SHAPE = -2
PT_ERR_CONFIG = -3
PT_ERR_WORKSPACE = -4
PT_ERR_HIP = -5
PT_ERR_ALIGN = -6
PT_ERR_SCRATCH = -7
PT_DK_SCRATCH_BYTES = 8 << 20

# FWD / DX kernel choice of the *_algo entry points
PT_ROWS_AUTO = 0
PT_ROWS_VALU = 1
PT_ROWS_MATRIX = 2

PT_KERNEL_FWD = 0
PT_KERNEL_DX = 1
PT_KERNEL_DK = 2
PT_KERNEL_DK_REDUCE = 3
PT_KERNEL_DK_CG = 4
PT_KERNEL_FWD_CG = 5
PT_KERNEL_DX_CG = 6
PT_KERNEL_FWD_STREAM = 7
PT_KERNEL_DX_STREAM = 8
PT_KERNEL_FWD_CG16 = 9
PT_KERNEL_DX_CG16 = 10

# Every symbol include/pathtile_hip.h declares, with (restype, argtypes).
_vp = ctypes.c_void_p
_i = ctypes.c_int
_ip = ctypes.POINTER(ctypes.c_int)
_szp = ctypes.POINTER(ctypes.c_size_t)
SIGNATURES = {
    "pt_abi_version": (_i, []),
    "pt_status_string": (ctypes.c_char_p, [_i]),
    "pt_dwconv1d_fwd_f32": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_dx_f32": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_fwd_f32_algo": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_dx_f32_algo": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "pt_rows_kernel_id": (_i, [_i, _i, _i, _i, _i, _i, _i, _i, _ip]),
    "pt_dwconv1d_dk_atomic_f32": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_dk_det_workspace_bytes": (_i, [_i, _i, _i, _i, _i, _szp]),
    "pt_dwconv1d_dk_det_f32": (
        _i, [_vp, _vp, _vp, _vp, ctypes.c_size_t, _i, _i, _i, _i, _i, _vp]
    ),
    "pt_dwconv1d_dk_det_f32_noalloc": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_fwd_bf16": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_dx_bf16": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_dk_atomic_bf16": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_dk_det_bf16_workspace_bytes": (_i, [_i, _i, _i, _i, _i, _szp]),
    "pt_dwconv1d_dk_det_bf16": (
        _i, [_vp, _vp, _vp, _vp, ctypes.c_size_t, _i, _i, _i, _i, _i, _vp]
    ),
    "flash_dk_fp32": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_fwd_long_f32": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_dx_long_f32": (_i, [_vp, _vp, _vp, _i, _i, _i, _i, _vp]),
    "pt_dwconv1d_dk_long_workspace_bytes": (_i, [_i, _i, _i, _i, _szp]),
    "pt_dwconv1d_dk_long_f32": (
        _i, [_vp, _vp, _vp, _vp, ctypes.c_size_t, _i, _i, _i, _i, _vp]
    ),
    "pt_kernel_attributes": (_i, [_i, _i, _i, _ip, _ip, _ip, _ip]),
    "pt_dynamic_lds_bytes": (_i, [_i, _i, _i, _i, _ip]),
}

_LOCK = threading.Lock()
_LIB: ctypes.CDLL | None = None


class PathTileLibraryError(RuntimeError):
    """The native library is missing, stale or returned an error."""


def load() -> ctypes.CDLL:
    """Load (once) and return the native library; raise if unavailable."""
    global _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not LIB_PATH.exists():
            raise PathTileLibraryError(
                f"{LIB_PATH} is missing: build it with "
                "`python -m pathtile_amd.build` (hipcc, gfx950)"
            )
        try:
            lib = ctypes.CDLL(str(LIB_PATH))
        except OSError as exc:
            raise PathTileLibraryError(f"cannot load {LIB_PATH}: {exc}") from exc
        for name, (res, args) in SIGNATURES.items():
            try:
                fn = getattr(lib, name)
            except AttributeError as exc:
                raise PathTileLibraryError(f"{LIB_PATH} lacks {name}") from exc
            fn.restype = res
            fn.argtypes = args
        if lib.pt_abi_version() != 1:
            raise PathTileLibraryError("ABI version mismatch; rebuild the library")
        _LIB = lib
        return lib


def status_string(status: int) -> str:
    return load().pt_status_string(int(status)).decode()


def check(status: int, what: str) -> None:
    """Map a negative status to the Python exception the reference raises for
    the same condition (kernels/warp_tiled_ampere.py:704-717)."""
    if status == PT_OK:
        return
    msg = f"{what}: {status_string(status)} (status {status})"
    if status in (PT_ERR_SHAPE, PT_ERR_CONFIG, PT_ERR_NULL, PT_ERR_ALIGN,
                  PT_ERR_WORKSPACE, PT_ERR_SCRATCH):
        raise ValueError(msg)
    raise PathTileLibraryError(msg)
