"""Build ``libpathtile_hip.so`` (gfx950) in-tree with hipcc.

Usage: ``python -m pathtile_amd.build`` (or ``__graft_entry__.build()``).

The library is a plain C-ABI shared object (``include/pathtile_hip.h``); it
links against libamdhip64 by its soname, so inside a process that already
imported torch it binds to torch's HIP runtime and shares its streams.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
import time
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
# One translation unit per dispatch table (compiled in parallel) + host side.
SOURCES = [
    "dwconv1d_abi.hip",
    "inst_fwd_v.hip",
    "inst_fwd_vp.hip",
    "inst_fwd_s.hip",
    "inst_dx_v.hip",
    "inst_dx_vp.hip",
    "inst_dx_s.hip",
    "inst_stream.hip",
    "inst_dk_v.hip",
    "inst_dk_s.hip",
    "inst_dk_mfma.hip",
    "inst_dk_cg1.hip",
    "inst_rows_mfma.hip",
    "inst_rows_mfma_u.hip",
    "inst_bf16.hip",
    "inst_dk_cl.hip",
    "inst_long.hip",
    "inst_long_vec.hip",
    "inst_long_s3.hip",
    "inst_long_s3_vec.hip",
]
INCLUDE = ROOT / "include"
BUILD_DIR = PKG / "_build"
LIB = PKG / "libpathtile_hip.so"
ARCH = os.environ.get("PATHTILE_OFFLOAD_ARCH", "gfx950")

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    # Packed FP32 (v_pk_fma_f32 and friends) stays off on this pool.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # float atomicAdd lowers to the hardware global_atomic_add_f32.
    "-munsafe-fp-atomics",
    "-Wall",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found (set HIPCC or install ROCm)")


def _compile(src: str) -> Path:
    obj = BUILD_DIR / (Path(src).stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, f"-I{INCLUDE}", "-c", "-o", str(obj), str(CSRC / src)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError("hipcc failed:\n" + " ".join(cmd) + "\n" + proc.stdout + proc.stderr)
    return obj


def build(verbose: bool = False, output: Path | None = None, jobs: int | None = None) -> Path:
    """Compile the HIP sources (one hipcc per translation unit, in parallel)
    and link ``pathtile_amd/libpathtile_hip.so``."""
    from concurrent.futures import ThreadPoolExecutor

    out = Path(output) if output else LIB
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    t0 = time.time()
    jobs = jobs or min(len(SOURCES), max(1, os.cpu_count() or 1), 16)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(_compile, SOURCES))
    tmp = out.with_name(out.name + f".tmp{os.getpid()}")
    cmd = [hipcc(), "-shared", "-fPIC", f"--offload-arch={ARCH}", "-o", str(tmp),
           *map(str, objs)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        try:
            tmp.unlink()
        except FileNotFoundError:
            pass
        raise RuntimeError("link failed:\n" + " ".join(cmd) + "\n" + proc.stdout + proc.stderr)
    os.replace(tmp, out)
    if verbose:
        print(f"[pathtile_amd.build] {out} in {time.time() - t0:.1f}s ({jobs} jobs)", flush=True)
    return out


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
