"""Placement probe: FWD / dX time against where the output lies relative to
the input.

A streaming kernel's time can depend on the distance between the tensor it
reads and the tensor it writes, through how the two address streams meet
in the memory channels. This probe allocates one buffer, puts x at its
start and the output `offset` MiB after the end of x, and times the FWD and
dX launches for each offset and each front count of the VALU tile kernel
(PATHTILE_ROWS_FRONTS) or, with ``--algo mfma``, the matrix-core kernel.
Outputs of every front count are compared bit for bit at the first offset.

    python -m pathtile_amd.placement --shape 32768,256,48,4 \\
        --offsets 0,0.5,32,64,256 --fronts 1,2 [--runs 30] [--algo valu]

Prints one JSON line per offset: {"offset_mib": d, "fwd_f1": us, ...}.
"""

from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m pathtile_amd.placement",
                                description=__doc__.split("\n")[0])
    p.add_argument("--shape", default="32768,256,48,4", help="B,H,L,K")
    p.add_argument("--offsets", default="0,0.0625,0.5,2,8,32,64,128,192,256,512",
                   help="MiB between the end of x and the start of the output")
    p.add_argument("--fronts", default="1,2", help="front counts of the VALU tile kernel")
    p.add_argument("--algo", choices=("valu", "mfma"), default="valu")
    p.add_argument("--waves-per-block", type=int, default=4)
    p.add_argument("--runs", type=int, default=30)
    p.add_argument("--warmup", type=int, default=8)
    a = p.parse_args(argv)

    import torch

    from . import _lib

    if not torch.cuda.is_available():
        print("the placement probe needs a ROCm GPU", file=sys.stderr)
        return 1
    lib = _lib.load()
    B, H, L, K = (int(v) for v in a.shape.split(","))
    offsets = [float(v) for v in a.offsets.split(",")]
    fronts = [int(v) for v in a.fronts.split(",")]
    if min(offsets) < 0:
        raise SystemExit("offsets must be >= 0")
    n = B * H * L
    mib = 1 << 18  # floats per MiB
    big = torch.empty(2 * n + int(max(offsets) * mib) + 4096, device="cuda")
    x = big[:n]
    x.normal_()
    w = torch.randn(H, K, device="cuda") / K ** 0.5
    stream = torch.cuda.current_stream()
    sh = ctypes.c_void_p(stream.cuda_stream)
    algo = _lib.PT_ROWS_VALU if a.algo == "valu" else _lib.PT_ROWS_MATRIX

    def time_us(fn) -> float:
        for _ in range(a.warmup):
            fn()
        e0 = torch.cuda.Event(enable_timing=True)
        e1 = torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        for _ in range(a.runs):
            fn()
        e1.record(stream)
        e1.synchronize()
        return e0.elapsed_time(e1) / a.runs * 1e3

    ref = {}
    prev = os.environ.get("PATHTILE_ROWS_FRONTS")
    try:
        for d in offsets:
            off = n + int(d * mib)
            y = big[off:off + n]
            xp, wp, yp = (ctypes.c_void_p(t.data_ptr()) for t in (x, w, y))
            row = {"offset_mib": d}
            for f in fronts:
                os.environ["PATHTILE_ROWS_FRONTS"] = str(f)
                for tag, fn in (("fwd", lib.pt_dwconv1d_fwd_f32_algo),
                                ("dx", lib.pt_dwconv1d_dx_f32_algo)):
                    def launch(fn=fn):
                        _lib.check(fn(xp, wp, yp, B, H, L, K, a.waves_per_block, algo, sh), tag)
                    row[f"{tag}_f{f}"] = round(time_us(launch), 1)
                    if d == offsets[0]:
                        torch.cuda.synchronize()
                        if tag in ref:
                            if not torch.equal(ref[tag], y):
                                raise SystemExit(f"{tag}: front count {f} changed the output bits")
                        else:
                            ref[tag] = y.clone()
            print(json.dumps(row), flush=True)
    finally:
        if prev is None:
            os.environ.pop("PATHTILE_ROWS_FRONTS", None)
        else:
            os.environ["PATHTILE_ROWS_FRONTS"] = prev
    return 0


if __name__ == "__main__":
    raise SystemExit(main())
