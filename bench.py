"""Benchmark of the MI355X depthwise Conv1D hot path (one JSON line).

Metric: "FWD+dX+dK ms & HBM GB/s (% peak), B16384 H128 L48
K48 fp32, 1 GPU". A step is one pass of the hot path over one batch: FWD, dX
and dK. Inputs are synthetic, drawn on a CPU torch.Generator in the order x,
w, dY (x, dY ~ N(0,1), w ~ N(0,1/K)) and copied to HBM before timing.

    python bench.py [--gpus 1] [--steps 20] [--warmup 5] [--no-cpu-baseline]

``value`` = FWD + dX + dK (atomic, zero-init outside the dK timing as in the
reference's protocol, README.md:136-140) in ms, each path timed with the
reference's protocol (artifact/REPRODUCIBILITY.md:81-93): 3 trials, each of
50 warm-up launches and 100 timed launches per path, path order reversed on
even trials (benchmark/benchmark_pathtile_candidate_sweep.py:488-501), mean
of the trial means; the between-trial standard deviation is reported beside
it. The timed launches run back to back between two HIP events on the launch
stream; ``paths_rotated`` repeats FWD, dX and dK over rotated buffer sets, so
that no launch finds its inputs in the MALL (the cold control), and the
roofline takes the slower of the two. ``ms_per_step`` is the wall time of the
contract's ``--steps`` interleaved FWD/dX/zero+dK steps (after 0.3 s of steps
and ``--warmup`` steps) between two device synchronisations, with an event
pair beside it (``ms_per_step_gpu``). Every configuration prints its
per-path ms and % of peak on stderr. After timing, the outputs of the timed launches are
checked against PyTorch FP64 on the GPU: FWD/dX on sampled batch rows (all
channels), dK over the whole batch. The same protocol and checks run for the
BASELINE's other configurations (S, E2, E1) as separate legs.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import re
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

METRIC = "FWD+dX+dK ms & HBM GB/s (% peak), B16384 H128 L48 K48 fp32, 1 GPU"
WORKLOADS = {
    # the metric's workload.
    "primary": (16384, 128, 48, 48),
    # the other BASELINE configurations (legs).
    "short": (32768, 256, 48, 4),
    "odd_k": (16384, 128, 48, 47),
    "edge": (1000, 96, 37, 48),
}
PEAK_HBM_GBPS = 8000.0
PEAK_BF16_MFMA_TFLOPS = 2500.0  # MI355X dense BF16 matrix
# Published aggregate of the reference for this metric (README.md:96,
# A100 PCIe 40 GB): 11.283 ms.
REFERENCE_AGGREGATE_MS = 11.283
POLICY = ROOT / "pathtile_amd" / "tune" / "frozen_policy.json"
PROFILES = ROOT / "profiles"
FWD_TOL, DK_TOL = 1e-5, 1e-4


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=20)
    p.add_argument("--warmup", type=int, default=5)
    p.add_argument("--workload", choices=sorted(WORKLOADS), default="primary")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--trials", type=int, default=3, help="timing trials per path")
    p.add_argument("--path-warmup", type=int, default=50, help="warm-up launches per path and trial")
    p.add_argument("--path-runs", type=int, default=100, help="timed launches per path and trial")
    p.add_argument("--no-legs", action="store_true",
                   help="skip the other BASELINE configurations (S, E2, E1) and, unless "
                        "their counts are given, the MIOpen and S4ConvD comparisons")
    p.add_argument("--no-extras", action="store_true",
                   help="skip the BF16, channels-last, long-row and VALU-kernel legs")
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-runs", type=int, default=10)
    p.add_argument("--gpu-library-steps", type=int, default=None, metavar="N",
                   help="time N calls per path of PyTorch's GPU convolution (MIOpen) on "
                        "the same tensors (default 3; 0 skips; off with --no-legs)")
    p.add_argument("--s4convd-steps", type=int, default=None, metavar="N",
                   help="time N S4ConvD training steps (the reference's Model() at "
                        "B16384 L48, SGD lr 1e-3 momentum 0.9) on each backend "
                        "(default 3; 0 skips; off with --no-legs)")
    p.add_argument("--copy-probe", type=int, default=0, metavar="N",
                   help="after timing, run N plain device copies of x into y "
                        "(known bytes: 2 * B*H*L*4 per copy) to calibrate "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE")
    a = p.parse_args(argv)
    if a.gpu_library_steps is None:
        a.gpu_library_steps = 0 if a.no_legs else 3
    if a.s4convd_steps is None:
        a.s4convd_steps = 0 if a.no_legs else 3
    return a


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def frozen_config() -> dict:
    from pathtile_amd import runtime

    cfg = {
        "fwd_waves_per_block": runtime.DEFAULT_WAVES_PER_BLOCK,
        "dx_waves_per_block": runtime.DEFAULT_DX_WAVES_PER_BLOCK,
        "dk_threads_per_block": runtime.DEFAULT_BWDK_BLOCK,
        "source": "runtime defaults",
    }
    if POLICY.exists():
        pol = json.loads(POLICY.read_text())
        sel = pol.get("selected", {})
        cfg.update({k: int(sel[k]) for k in ("fwd_waves_per_block", "dx_waves_per_block",
                                              "dk_threads_per_block") if k in sel})
        cfg["source"] = str(POLICY.relative_to(ROOT))
    return cfg


def make_inputs(B, H, L, K, seed):
    import torch

    g = torch.Generator().manual_seed(seed)
    x = torch.randn(B, H, L, generator=g, dtype=torch.float32)
    w = torch.randn(H, K, generator=g, dtype=torch.float32) / math.sqrt(K)
    dy = torch.randn(B, H, L, generator=g, dtype=torch.float32)
    return x, w, dy


def mean(v):
    return sum(v) / len(v) if v else float("nan")


def stdev(v):
    if len(v) < 2:
        return 0.0
    m = mean(v)
    return math.sqrt(sum((a - m) ** 2 for a in v) / (len(v) - 1))


# --------------------------------------------------------------------------
# FP64 references on the GPU (PyTorch), for the checks of the timed outputs
# --------------------------------------------------------------------------
def fp64_fwd(x, w):
    """y[b,h,t] = sum_j w[h,j] x[b,h,t+j-p], p = K // 2, in FP64
    (benchmark/benchmark_shape_sweep_ampere.py:220-239)."""
    import torch.nn.functional as F

    K = w.shape[1]
    p = K // 2
    return F.conv1d(F.pad(x.double(), (p, K - 1 - p)), w.double().unsqueeze(1),
                    groups=x.shape[1])


def fp64_dx(dy, w):
    """dx[b,h,s] = sum_j w[h,j] dy[b,h,s-j+p]: a correlation with the
    flipped taps, padded (K-1-p, p), in FP64."""
    import torch.nn.functional as F

    K = w.shape[1]
    p = K // 2
    return F.conv1d(F.pad(dy.double(), (K - 1 - p, p)), w.double().flip(-1).unsqueeze(1),
                    groups=dy.shape[1])


def fp64_dk(dy, x, K):
    """dK[h,j] = sum_b sum_t dy[b,h,t] x[b,h,t+j-p] in FP64 over the whole
    batch (benchmark/check_dk_fp64_comparison.py:29-39)."""
    import torch
    import torch.nn.functional as F

    L = x.shape[2]
    p = K // 2
    xp = F.pad(x.double(), (p, K - 1 - p))
    dyd = dy.double()
    out = torch.stack([(dyd * xp[..., j:j + L]).sum(dim=(0, 2)) for j in range(K)], dim=1)
    del xp, dyd
    return out


def nerr(a, ref) -> float:
    """max |a - ref| / max |ref| (kernels/warp_tiled_ampere.py:182-184)."""
    return float((a.double() - ref).abs().max() / ref.abs().max().clamp_min(1e-30))


def device_warmup(fns: dict, seconds: float = 0.3) -> None:
    """Launch every path round-robin for about `seconds` of wall time before
    the first timed trial: the first ~0.1 s of launches after the inputs are
    written run a few percent slow (measured on MI355X: the first trial of
    the first path 144 us against 135.6 us after), which the per-path warm-up
    of the protocol alone does not cover."""
    import torch

    t0 = time.perf_counter()
    while time.perf_counter() - t0 < seconds:
        for fn in fns.values():
            fn()
        torch.cuda.synchronize()


def time_paths(fns: dict, stream, trials: int, warmup: int, runs: int) -> dict:
    """The reference's protocol per path: `trials` trials, each `warmup`
    launches then `runs` launches back to back between two events on the
    launch stream; path order reversed on even trials. Returns per path the
    trial means (ms per launch), their mean and their standard deviation."""
    import torch

    per = {k: [] for k in fns}
    for t in range(1, trials + 1):
        order = list(fns) if t % 2 else list(reversed(list(fns)))
        for k in order:
            fn = fns[k]
            for _ in range(warmup):
                fn()
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            e0.record(stream)
            for _ in range(runs):
                fn()
            e1.record(stream)
            e1.synchronize()
            per[k].append(e0.elapsed_time(e1) / runs)
    return {k: {"ms": mean(v), "std_ms": stdev(v), "trials_ms": v} for k, v in per.items()}


def rows_kernel_name(B: int, H: int, L: int, K: int, dx: bool) -> str:
    """The FWD/DX kernel the library runs for this call on 16-byte aligned
    tensors, as its own dispatch reports it (pt_rows_kernel_id; the
    PATHTILE_ROWS_* environment included)."""
    from pathtile_amd import runtime

    return runtime.rows_kernel_name(B, H, L, K, dx=dx)


def dk_kernel_name(H: int, L: int, threads: int) -> str:
    """The DK kernel the library picks: the channel-group matrix-core kernel
    when H is a multiple of the channel group (at most 8 waves per
    workgroup, one channel per wave for rows of 33-48 columns, two below;
    any L), else the per-channel matrix-core kernel (or the VALU kernel on
    request)."""
    if os.environ.get("PATHTILE_DK_ALGO") == "valu":
        return "dwconv_dk_kernel"
    wpb = threads // 64
    cpw = 1 if L > 32 else 2
    if wpb <= 8 and H % (cpw * wpb) == 0:
        return "dwconv_dk_cg_kernel"
    return "dwconv_dk_mfma_kernel"


def read_profile_numbers(name: str, keys: tuple[str, ...]) -> dict | None:
    """`KEY: number` lines from a committed rocprofv3 summary under
    profiles/ (None if the file or a key is missing)."""
    f = PROFILES / name
    if not f.exists():
        return None
    text = f.read_text()
    out = {}
    for k in keys:
        m = re.search(rf"{k}:\s*([0-9.eE+]+)", text)
        if not m:
            return None
        out[k] = float(m.group(1))
    return out


def read_traffic(kernel_tag: str) -> dict | None:
    """HBM bytes per launch of `kernel_tag` from the committed rocprofv3 PMC
    summary (profiles/pmc_traffic_<kernel_tag>.md)."""
    r = read_profile_numbers(f"pmc_traffic_{kernel_tag}.md",
                             ("FETCH_BYTES_PER_LAUNCH", "WRITE_BYTES_PER_LAUNCH"))
    return None if r is None else {"fetch": r["FETCH_BYTES_PER_LAUNCH"],
                                   "write": r["WRITE_BYTES_PER_LAUNCH"]}


def workload_leg(rt, name: str, args, dev, stream, keep: bool = False) -> dict:
    """One BASELINE configuration: per-path timing with the reference's
    protocol, then the checks of the timed outputs against FP64 (sampled
    batch rows for FWD/dX, the whole batch for dK; the deterministic dK
    bitwise equal across two runs)."""
    import torch

    from pathtile_amd import runtime

    B, H, L, K = WORKLOADS[name]
    log(f"{name}: B={B} H={H} L={L} K={K}")
    x_cpu, w_cpu, dy_cpu = make_inputs(B, H, L, K, args.seed)
    x, w, dy = x_cpu.to(dev), w_cpu.to(dev), dy_cpu.to(dev)
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    gk = torch.zeros(H, K, device=dev)
    gd = torch.zeros(H, K, device=dev)
    fns = {
        "fwd": lambda: rt.launch_fwd(x, w, y),
        "bwd_input": lambda: rt.launch_bwd_input(dy, w, dx),
        "bwd_weight": lambda: rt.launch_bwd_weight(dy, x, gk, K),
        "bwd_weight_zero": lambda: rt.launch_bwd_weight(dy, x, gk, K, zero_first=True),
        "bwd_weight_det": lambda: rt.launch_bwd_weight_deterministic(dy, x, gd, K),
    }
    device_warmup(fns)
    timing = time_paths(fns, stream, args.trials, args.path_warmup, args.path_runs)

    # Checks of the timed launches' outputs: y and dx hold the last timed
    # launch's results; dK is launched once more on the same tensors (the
    # timed atomic launches accumulate into gk).
    # Sampled batch rows: the first and the last sample (the ragged tail
    # steps) and distinct others.
    g = torch.Generator().manual_seed(args.seed + 1)
    n_rows = min(B, 256)
    inner = (torch.randperm(B - 2, generator=g)[: max(0, n_rows - 2)] + 1 if B > 2
             else torch.empty(0, dtype=torch.long))
    idx = torch.cat([torch.tensor([0]), inner, torch.tensor([B - 1] if B > 1 else [])]).long()
    idx = idx.to(dev)
    gate = {
        "fwd": nerr(y[idx], fp64_fwd(x[idx], w)),
        "bwd_input": nerr(dx[idx], fp64_dx(dy[idx], w)),
    }
    ref = fp64_dk(dy, x, K)
    rt.launch_bwd_weight(dy, x, gk, K, zero_first=True)
    gate["bwd_weight"] = nerr(gk, ref)
    gd2 = torch.empty_like(gd)
    rt.launch_bwd_weight_deterministic(dy, x, gd2, K)
    gate["bwd_weight_det"] = nerr(gd2, ref)
    torch.cuda.synchronize()
    det_bitwise = bool(torch.equal(gd, gd2))
    ok = (gate["fwd"] < FWD_TOL and gate["bwd_input"] < FWD_TOL and gate["bwd_weight"] < DK_TOL
          and gate["bwd_weight_det"] < DK_TOL and det_bitwise)
    if not ok:
        raise SystemExit(f"{name}: check of the timed outputs failed: {gate}, "
                         f"deterministic dK bitwise={det_bitwise}")
    nbytes = runtime.minimum_algorithmic_bytes(B, H, L, K)
    kernels = {"fwd": rows_kernel_name(B, H, L, K, False), "bwd_input": rows_kernel_name(B, H, L, K, True),
               "bwd_weight": dk_kernel_name(H, L, rt.bwdk_block)}
    paths = {}
    for ph, t in timing.items():
        gbps = runtime.algorithmic_bandwidth_gbps(nbytes, t["ms"])
        paths[ph] = {"ms": round(t["ms"], 5), "std_ms": round(t["std_ms"], 5),
                     "trials_ms": [round(v, 5) for v in t["trials_ms"]],
                     "gbps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_HBM_GBPS, 2),
                     "kernel": kernels[{"bwd_weight_zero": "bwd_weight",
                                        "bwd_weight_det": "bwd_weight"}.get(ph, ph)]}
    agg = paths["fwd"]["ms"] + paths["bwd_input"]["ms"] + paths["bwd_weight"]["ms"]
    agg_std = math.sqrt(sum(timing[p]["std_ms"] ** 2 for p in ("fwd", "bwd_input", "bwd_weight")))
    leg = {
        "config": {"B": B, "H": H, "L": L, "K": K},
        "fwd_dx_dk_ms": round(agg, 5),
        "fwd_dx_dk_std_ms": round(agg_std, 5),
        "aggregate_pct_peak": round(100 * 3 * nbytes / (agg / 1e3) / 1e9 / PEAK_HBM_GBPS, 2),
        "algorithmic_bytes_per_path": nbytes,
        "paths": paths,
        "check_of_timed_outputs": {k: float(f"{v:.3e}") for k, v in gate.items()}
        | {"deterministic_dk_bitwise_repeat": det_bitwise,
           "sampled_rows": int(idx.numel()),
           "bars": "FWD/dX <= 1e-5, dK <= 1e-4 max-abs-scaled vs PyTorch FP64 on the GPU"},
    }
    log(f"{name}: {path_line(paths)}; FWD+dX+dK {agg:.4f} ms "
        f"({leg['aggregate_pct_peak']:.1f}%)")
    if not keep and args.gpu_library_steps:
        leg["gpu_library_baseline"] = gpu_library_baseline(x, w, dy, args.gpu_library_steps)
    if keep:
        leg["_tensors"] = (x_cpu, w_cpu, dy_cpu, x, w, dy, y, dx, gk)
    else:
        del x, w, dy, y, dx, gk, gd, gd2, ref
        torch.cuda.empty_cache()
    return leg


PATH_TAGS = {"fwd": "FWD", "bwd_input": "dX", "bwd_weight": "dK",
             "bwd_weight_zero": "dK+zero", "bwd_weight_det": "dK det"}


def path_line(paths: dict) -> str:
    """One stderr line of per-path ms and % of the 8 TB/s peak."""
    return ", ".join(f"{PATH_TAGS.get(k, k)} {v['ms']:.4f} ms ({v['pct_peak']:.1f}%)"
                     for k, v in paths.items())


def compact_leg(leg: dict) -> dict:
    """A configuration leg for the JSON line: per path [ms, between-trial std
    ms, % of 8 TB/s], the kernels, the aggregate and the check errors."""
    p = leg["paths"]
    chk = leg["check_of_timed_outputs"]
    out = {
        "config": leg["config"],
        "fwd_dx_dk_ms": leg["fwd_dx_dk_ms"],
        "aggregate_pct_peak": leg["aggregate_pct_peak"],
        "paths": {k: [v["ms"], v["std_ms"], v["pct_peak"]] for k, v in p.items()},
        "kernels": sorted({v["kernel"] for v in p.values()}),
        "check_max_err": {k: v for k, v in chk.items() if isinstance(v, float)},
        "det_dk_bitwise_repeat": chk["deterministic_dk_bitwise_repeat"],
    }
    if "gpu_library_baseline" in leg:
        out["miopen_ms"] = leg["gpu_library_baseline"]["paths_ms"]
    return out


def rotated_paths(rt, args, stream, x, w, dy, K, gk) -> dict:
    """FWD, dX and dK timed over rotated buffer sets (the cold control): each
    launch reads tensors that at least one other set's launch has streamed
    past since their last use (2 x 403 MB at P, past the 256 MB MALL), so
    no launch can find its inputs in the MALL."""
    import torch

    nsets = max(2, -(-(512 << 20) // (2 * x.numel() * 4)) + 1)
    sets = [(x, dy, torch.empty_like(x), torch.empty_like(dy))]
    sets += [(x.clone(), dy.clone(), torch.empty_like(x), torch.empty_like(dy))
             for _ in range(nsets - 1)]
    cur = {"fwd": 0, "bwd_input": 0, "bwd_weight": 0}

    def rotated(ph, call):
        def fn():
            i = cur[ph] = (cur[ph] + 1) % nsets
            call(*sets[i])
        return fn

    fns = {
        "fwd": rotated("fwd", lambda xs, dys, ys, dxs: rt.launch_fwd(xs, w, ys)),
        "bwd_input": rotated("bwd_input", lambda xs, dys, ys, dxs: rt.launch_bwd_input(dys, w, dxs)),
        "bwd_weight": rotated("bwd_weight", lambda xs, dys, ys, dxs: rt.launch_bwd_weight(dys, xs, gk, K)),
    }
    device_warmup(fns)
    t = time_paths(fns, stream, args.trials, args.path_warmup, args.path_runs)
    del sets
    torch.cuda.empty_cache()
    return {"sets": nsets, "timing": t}


def cpu_baseline(x, w, dy, runs: int) -> dict:
    """PyTorch CPU with the reference's PyTorch timing boundaries
    (benchmark/benchmark_shape_sweep_ampere.py:349-407): FWD = F.pad +
    F.conv1d(groups=H); dX = autograd.grad(y, x); dK = autograd.grad(y, w);
    graph construction outside the timer."""
    import torch

    import oracle  # CPU restatement of the reference's PyTorch boundary

    try:
        cores = len(os.sched_getaffinity(0))
    except AttributeError:  # pragma: no cover
        cores = os.cpu_count() or 1
    threads = max(1, min(cores, int(os.environ.get("OMP_NUM_THREADS", cores))))
    torch.set_num_threads(threads)
    f = oracle.pytorch_depthwise_same
    out = {}
    t_all = time.perf_counter()
    for phase in ("fwd", "dx", "dk"):
        ts = []
        for r in range(runs + 1):
            if phase == "fwd":
                t0 = time.perf_counter()
                f(x, w)
                t1 = time.perf_counter()
            elif phase == "dx":
                xr = x.detach().requires_grad_(True)
                y = f(xr, w)
                t0 = time.perf_counter()
                torch.autograd.grad(y, xr, dy)
                t1 = time.perf_counter()
            else:
                wr = w.detach().requires_grad_(True)
                y = f(x, wr)
                t0 = time.perf_counter()
                torch.autograd.grad(y, wr, dy)
                t1 = time.perf_counter()
            if r > 0:  # first run is the warm-up
                ts.append((t1 - t0) * 1e3)
        out[phase] = mean(ts)
        log(f"cpu {phase}: {out[phase]:.1f} ms")
    total = out["fwd"] + out["dx"] + out["dk"]
    try:
        cpu_model = next(l.split(":", 1)[1].strip() for l in open("/proc/cpuinfo")
                         if l.startswith("model name"))
    except Exception:
        cpu_model = "unknown"
    B, H, L = x.shape
    return {
        "value": round(total, 3),
        "unit": "ms",
        "cores": threads,
        "kind": "port",
        "sample": (f"full workload B={B} H={H} L={L} K={w.shape[1]}, PyTorch {torch.__version__} "
                   f"CPU F.pad+F.conv1d(groups=H) / autograd.grad (reference PyTorch boundary), "
                   f"1 warm-up + {runs} timed runs per path, {threads} threads on {cpu_model}"),
        "paths_ms": {k: round(v, 3) for k, v in out.items()},
        "wall_s": round(time.perf_counter() - t_all, 1),
    }


def gpu_library_baseline(x, w, dy, steps: int) -> dict:
    """PyTorch's own GPU path for the same op on the same tensors (grouped
    F.conv1d, MIOpen on ROCm), with the reference's PyTorch boundaries: FWD =
    the convolution, dX = autograd.grad(y, x), dK = autograd.grad(y, w), the
    graph built outside the events; one event pair per call, mean over
    `steps` calls after one warm-up call."""
    import torch

    from pathtile_amd.runtime import reference_depthwise_conv as conv

    out = {}
    for phase in ("fwd", "dx", "dk"):
        ts = []
        for r in range(steps + 1):
            e0 = torch.cuda.Event(enable_timing=True)
            e1 = torch.cuda.Event(enable_timing=True)
            if phase == "fwd":
                e0.record()
                conv(x, w)
                e1.record()
            else:
                xr = x.detach().requires_grad_(phase == "dx")
                wr = w.detach().requires_grad_(phase == "dk")
                y = conv(xr, wr)
                e0.record()
                torch.autograd.grad(y, xr if phase == "dx" else wr, dy)
                e1.record()
            e1.synchronize()
            if r > 0:
                ts.append(e0.elapsed_time(e1))
        out[phase] = round(mean(ts), 4)
    return {"what": "torch.nn.functional.conv1d(groups=H) on the GPU (MIOpen), same tensors",
            "paths_ms": out, "total_ms": round(sum(out.values()), 4), "calls_per_path": steps}


def s4convd_training_steps(steps: int, warmup: int, dev) -> dict:
    """Time S4ConvD training steps (forward, backward, SGD) of the reference's
    default Model() on a synthetic batch shaped like its training batches
    (B=16384 windows of L=48 steps, 4 features; kernels/warp_tiled_ampere.py:
    1193-1215, 1345-1354, 1442-1446), on the "warp" backend (HIP path, skip
    term fused) and the "pytorch" backend (PyTorch's GPU convolution)."""
    import torch

    from pathtile_amd import runtime, s4convd
    from pathtile_amd.kernels import warp_tiled_ampere as wta

    runtime.get_or_create_runtime()  # the frozen policy's launch config
    out = {}
    prev = wta.TRAIN_CONV_BACKEND
    try:
        for name in ("warp", "pytorch"):
            wta.TRAIN_CONV_BACKEND = name
            torch.manual_seed(0)
            model = s4convd.Model().to(dev)
            opt = torch.optim.SGD(model.parameters(), lr=1e-3, momentum=0.9)
            g = torch.Generator().manual_seed(1)
            x = torch.randn(16384, 48, 4, generator=g).to(dev)
            target = torch.rand(16384, 1, generator=g).to(dev)

            def step():
                opt.zero_grad(set_to_none=True)
                loss = s4convd.rmsle(model(x), target)
                loss.backward()
                opt.step()
                return loss

            for _ in range(warmup):
                step()
            torch.cuda.synchronize()
            t0 = time.perf_counter()
            for _ in range(steps):
                loss = step()
            torch.cuda.synchronize()
            out[name] = {"ms_per_step": round((time.perf_counter() - t0) * 1e3 / steps, 4),
                         "final_loss": float(loss.detach())}
            del model, opt, x, target
            torch.cuda.empty_cache()
    finally:
        wta.TRAIN_CONV_BACKEND = prev
    return {"workload": "S4ConvD Model() (4 blocks, H128, state 64), B16384 L48 synthetic, "
                        "SGD lr 1e-3 momentum 0.9, dropout 0.01",
            "steps": steps, "warmup": warmup, **out,
            "speedup_vs_pytorch": round(out["pytorch"]["ms_per_step"] / out["warp"]["ms_per_step"], 3)}


def extras(rt, args, dev, stream, x, w, dy, y, gk) -> dict:
    """Legs beyond the metric on the primary tensors (no reference
    counterpart for BF16; the reference's Flash-DWC bridge ABI for
    channels-last dK; the reference's long-row module at its benchmark
    shape; the VALU FWD/dX kernel that reproduces the reference's bits)."""
    import torch

    from pathtile_amd import runtime

    B, H, L = x.shape
    K = w.shape[1]
    out = {}
    prot = dict(stream=stream, trials=args.trials, warmup=args.path_warmup, runs=args.path_runs)

    # BF16 I/O: x, dY and the FWD/dX outputs in bfloat16, taps and dK in
    # FP32; algorithmic bytes (2 B H L * 2 + H K * 4) per path. Served for
    # the channel-group layout only.
    dk_channels = 2 * (rt.bwdk_block // 64)
    if L % 4 == 0 and H % 8 == 0 and H % dk_channels == 0 and rt.bwdk_block <= 512:
        xb, dyb = x.to(torch.bfloat16), dy.to(torch.bfloat16)
        yb, dxb = torch.empty_like(xb), torch.empty_like(dyb)
        t = time_paths({
            "fwd": lambda: rt.launch_fwd_bf16(xb, w, yb),
            "bwd_input": lambda: rt.launch_bwd_input_bf16(dyb, w, dxb),
            "bwd_weight": lambda: rt.launch_bwd_weight_bf16(dyb, xb, gk, K),
            "bwd_weight_det": lambda: rt.launch_bwd_weight_deterministic_bf16(dyb, xb, gk, K),
        }, **prot)
        rows_b = min(512, B)
        y32 = torch.empty(rows_b, H, L, device=dev)
        rt.launch_fwd(xb[:rows_b].float().contiguous(), w, y32)
        torch.cuda.synchronize()
        bf16_gate = nerr(yb[:rows_b].float(), y32.double())
        if not bf16_gate < 2.0 ** -8:
            raise SystemExit(f"BF16 gate failed: {bf16_gate}")
        # The BF16 tensors at P (201 MB) fit the 256 MB MALL, so back-to-back
        # launches on one tensor read part of it from there. The same paths
        # over rotated buffer sets (each launch reads tensors that at least
        # 512 MiB of other traffic has passed since their last use) give
        # the time from HBM.
        nsets = max(1, -(-(512 << 20) // (2 * B * H * L * 2)) + 1)
        sets = [(xb.clone(), dyb.clone(), torch.empty_like(yb), torch.empty_like(dxb))
                for _ in range(nsets - 1)] + [(xb, dyb, yb, dxb)]
        cur = {"fwd": 0, "bwd_input": 0, "bwd_weight": 0}

        def rotated(ph, call):
            def fn():
                i = cur[ph] = (cur[ph] + 1) % nsets
                call(*sets[i])
            return fn
        t_cold = time_paths({
            "fwd": rotated("fwd", lambda xs, dys, ys, dxs: rt.launch_fwd_bf16(xs, w, ys)),
            "bwd_input": rotated("bwd_input", lambda xs, dys, ys, dxs: rt.launch_bwd_input_bf16(dys, w, dxs)),
            "bwd_weight": rotated("bwd_weight", lambda xs, dys, ys, dxs: rt.launch_bwd_weight_bf16(dys, xs, gk, K)),
        }, **prot)
        del xb, dyb, yb, dxb, y32, sets
        nb = 2 * B * H * L * 2 + H * K * 4
        def rows3(tt):
            return {ph: [round(v["ms"], 5), round(v["std_ms"], 5),
                         round(100 * nb / (v["ms"] / 1e3) / 1e9 / PEAK_HBM_GBPS, 2)]
                    for ph, v in tt.items()}
        out["bf16_io"] = {
            "paths": rows3(t),
            "fwd_dx_dk_ms": round(t["fwd"]["ms"] + t["bwd_input"]["ms"] + t["bwd_weight"]["ms"], 5),
            "paths_rotated": rows3(t_cold),
            "rotated_sets": nsets,
            "gate_vs_fp32_path": float(f"{bf16_gate:.3e}"),
            "note": "[ms, std, % of 8 TB/s]; x, dY, y, dX bf16, taps and dK fp32; bytes 2BHL*2 + HK*4",
        }

    # Channels-last dK through the Flash-DWC bridge ABI (flash_dk_fp32).
    if B % 16 == 0 and H % 32 == 0:
        xc = x.permute(0, 2, 1).unsqueeze(1).contiguous()
        dyc = dy.permute(0, 2, 1).unsqueeze(1).contiguous()
        dwc = torch.zeros(1, K, H, device=dev)
        t = time_paths({"dk": lambda: rt.launch_bwd_weight_channels_last(xc, dyc, dwc, 1)}, **prot)
        rt.launch_bwd_weight_deterministic(dy, x, gk, K)
        rt.launch_bwd_weight_channels_last(xc, dyc, dwc, 1, zero_first=True)
        torch.cuda.synchronize()
        cl_gate = nerr(dwc[0].T, gk.double())
        if not cl_gate < 1e-5:
            raise SystemExit(f"channels-last dK gate failed: {cl_gate}")
        gb = runtime.algorithmic_bandwidth_gbps(runtime.minimum_algorithmic_bytes(B, H, L, K),
                                                t["dk"]["ms"])
        out["channels_last_dk"] = {
            "ms": round(t["dk"]["ms"], 5), "std_ms": round(t["dk"]["std_ms"], 5),
            "gbps": round(gb, 1), "pct_peak": round(100 * gb / PEAK_HBM_GBPS, 2),
            "kernel": ("dwconv_dk_cl_kernel<48, 4, 2>" if L > 32
                       else f"dwconv_dk_cl_kernel<{16 * ((L + 15) // 16)}>"),
            "gate_vs_row_major": float(f"{cl_gate:.3e}"),
            "note": "flash_dk_fp32, x/dY [B,1,L,H], GZ=1"}
        del xc, dyc, dwc

    # The VALU rows kernel (the reference's lane-per-row structure, bit-exact
    # with its fmaf chain), forced beside the default FWD/DX kernel.
    prev = os.environ.get("PATHTILE_ROWS_ALGO")
    os.environ["PATHTILE_ROWS_ALGO"] = "valu"
    try:
        dxv = torch.empty_like(x)
        t = time_paths({"fwd": lambda: rt.launch_fwd(x, w, y),
                        "bwd_input": lambda: rt.launch_bwd_input(dy, w, dxv)}, **prot)
        idx = torch.arange(0, B, max(1, B // 256), device=dev)
        valu_gate = {"fwd": nerr(y[idx], fp64_fwd(x[idx], w)),
                     "bwd_input": nerr(dxv[idx], fp64_dx(dy[idx], w))}
        kern = {"fwd": rows_kernel_name(B, H, L, K, False), "bwd_input": rows_kernel_name(B, H, L, K, True)}
        del dxv
    finally:
        if prev is None:
            del os.environ["PATHTILE_ROWS_ALGO"]
        else:
            os.environ["PATHTILE_ROWS_ALGO"] = prev
    if not all(v < FWD_TOL for v in valu_gate.values()):
        raise SystemExit(f"VALU rows kernel gate failed: {valu_gate}")
    nbytes = runtime.minimum_algorithmic_bytes(B, H, L, K)
    out["rows_valu"] = {
        ph: {"ms": round(v["ms"], 5), "std_ms": round(v["std_ms"], 5),
             "pct_peak": round(100 * runtime.algorithmic_bandwidth_gbps(nbytes, v["ms"])
                               / PEAK_HBM_GBPS, 2), "kernel": kern[ph]}
        for ph, v in t.items()
    } | {"check_vs_fp64": {k: float(f"{v:.3e}") for k, v in valu_gate.items()},
         "note": "PATHTILE_ROWS_ALGO=valu (bit-exact VALU kernel)"}
    return out


def long_rows_leg(rt, args, dev, stream) -> dict:
    """Long rows at the reference's long-row benchmark shape (kernels/
    shared_l192.py, benchmarked at B16384 H128 L192 K192 by
    benchmark/benchmark_gmc_vs_shared_l192.py:14-17). The default kernels run
    on the BF16 matrix cores with three-way split FP32 operands; the FP32
    matrix-core kernels (PATHTILE_LONG_ALGO=fp32) are timed beside them."""
    import torch

    from pathtile_amd.tune.baselines import useful_products

    LB, LH, LL, LK = 16384, 128, 192, 192
    xl = torch.randn(LB, LH, LL, generator=torch.Generator().manual_seed(args.seed + 3)).to(dev)
    dyl = torch.randn(LB, LH, LL, generator=torch.Generator().manual_seed(args.seed + 4)).to(dev)
    wl = (torch.randn(LH, LK, generator=torch.Generator().manual_seed(args.seed + 5)) / LK ** 0.5).to(dev)
    yl, dxl, gkl = torch.empty_like(xl), torch.empty_like(dyl), torch.empty(LH, LK, device=dev)
    fns = {
        "fwd": lambda: rt.launch_fwd_long(xl, wl, yl),
        "bwd_input": lambda: rt.launch_bwd_input_long(dyl, wl, dxl),
        "bwd_weight": lambda: rt.launch_bwd_weight_long(dyl, xl, gkl, LK),
    }
    prot = dict(stream=stream, trials=args.trials, warmup=args.path_warmup, runs=args.path_runs)
    useful = 2 * useful_products(LB, LH, LL, LK)
    nbytes = 2 * LB * LH * LL * 4 + LH * LK * 4
    # Issued BF16 matrix flops per launch of the split kernels, from the
    # committed rocprofv3 counter summary (SQ_INSTS_VALU_MFMA_MOPS_BF16).
    issued = read_profile_numbers("pmc_mfma_long_l192_k192.md",
                                  ("BF16_MFMA_FLOP_FWD", "BF16_MFMA_FLOP_DX", "BF16_MFMA_FLOP_DK"))
    issued_key = {"fwd": "BF16_MFMA_FLOP_FWD", "bwd_input": "BF16_MFMA_FLOP_DX",
                  "bwd_weight": "BF16_MFMA_FLOP_DK"}

    def paths(t, split):
        # [ms, std ms, useful TFLOP/s, % of 8 TB/s, fraction of the BF16
        # matrix peak the split kernels issue]
        out = {}
        for ph, v in t.items():
            s = v["ms"] / 1e3
            row = [round(v["ms"], 5), round(v["std_ms"], 5), round(useful / s / 1e12, 2),
                   round(100 * nbytes / s / 1e9 / PEAK_HBM_GBPS, 2)]
            if split and issued:
                row.append(round(issued[issued_key[ph]] / s / 1e12 / PEAK_BF16_MFMA_TFLOPS, 4))
            out[ph] = row
        return out

    prev = os.environ.pop("PATHTILE_LONG_ALGO", None)
    try:
        t_split = time_paths(fns, **prot)
        y_split = yl[:256].clone()
        os.environ["PATHTILE_LONG_ALGO"] = "fp32"
        t_fp32 = time_paths(fns, **prot)
        rt.launch_fwd_long(xl, wl, yl)
        torch.cuda.synchronize()
    finally:
        if prev is None:
            os.environ.pop("PATHTILE_LONG_ALGO", None)
        else:
            os.environ["PATHTILE_LONG_ALGO"] = prev
    gate = {"split_vs_fp64": nerr(y_split, fp64_fwd(xl[:256], wl)),
            "fp32_vs_fp64": nerr(yl[:256], fp64_fwd(xl[:256], wl))}
    if not all(v < FWD_TOL for v in gate.values()):
        raise SystemExit(f"long-row gate failed: {gate}")
    del xl, dyl, wl, yl, dxl, gkl
    torch.cuda.empty_cache()
    return {
        "config": {"B": LB, "H": LH, "L": LL, "K": LK},
        "paths": paths(t_split, True),
        "fwd_dx_dk_ms": round(sum(v["ms"] for v in t_split.values()), 5),
        "fp32_mfma_kernels_ms": {k: round(v["ms"], 5) for k, v in t_fp32.items()},
        "check_fwd_first_256_samples": {k: float(f"{v:.3e}") for k, v in gate.items()},
        "note": "[ms, std, useful TFLOP/s, % of 8 TB/s, issued BF16 / 2.5 PFLOP/s "
                "(profiles/pmc_mfma_long_l192_k192.md)]; BF16 matrix cores on 3-way split "
                "FP32 operands; fp32_mfma_kernels_ms: PATHTILE_LONG_ALGO=fp32",
    }


def main(argv=None) -> int:
    args = parse_args(argv)
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (--gpus {args.gpus} requested): the "
              "path is built and measured as a single-GPU kernel; across GPUs it would "
              "shard by samples (FWD/dX independent, one H*K all-reduce for dK) or by "
              "channels (no exchange).",
              file=sys.stderr, flush=True)
        return 2
    import torch

    from pathtile_amd import runtime

    if not torch.cuda.is_available():
        print("bench.py needs a ROCm GPU", file=sys.stderr)
        return 1
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream(dev)
    B, H, L, K = WORKLOADS[args.workload]
    cfg = frozen_config()
    rt = runtime.HipWarpRuntime(waves_per_block=cfg["fwd_waves_per_block"],
                                dx_waves_per_block=cfg["dx_waves_per_block"],
                                bwdk_block=cfg["dk_threads_per_block"])
    log(f"workload {args.workload} config={cfg}")
    main_leg = workload_leg(rt, args.workload, args, dev, stream, keep=True)
    x_cpu, w_cpu, dy_cpu, x, w, dy, y, dx, gk = main_leg.pop("_tensors")
    log(f"{args.workload}: checks {main_leg['check_of_timed_outputs']}")
    nbytes = main_leg["algorithmic_bytes_per_path"]
    cold = rotated_paths(rt, args, stream, x, w, dy, K, gk)
    cold_paths = {}
    for ph, t in cold["timing"].items():
        gbps = runtime.algorithmic_bandwidth_gbps(nbytes, t["ms"])
        cold_paths[ph] = {"ms": round(t["ms"], 5), "std_ms": round(t["std_ms"], 5),
                          "gbps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_HBM_GBPS, 2)}
    log(f"{args.workload} over {cold['sets']} rotated buffer sets: {path_line(cold_paths)}")

    def step():
        rt.launch_fwd(x, w, y)
        rt.launch_bwd_input(dy, w, dx)
        gk.zero_()
        rt.launch_bwd_weight(dy, x, gk, K)

    # The contract's steps: `warmup` untimed, then exactly `steps` interleaved
    # FWD / dX / zero + dK steps, wall-clocked between two synchronisations,
    # with an event pair on the launch stream beside the wall clock. Before
    # the warm-up steps the GPU runs 0.3 s of steps: on MI355X bursts of
    # ~10 ms from a quiet GPU run these steps at 0.470-0.480 ms and after
    # 0.3 s of sustained work at 0.388 ms (the per-path sum), which a 1 s
    # pause followed by 0.1 s of work keeps (a clock ramp, not host time:
    # the host enqueues a launch in ~10 us).
    device_warmup({"step": step})
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    e0 = torch.cuda.Event(enable_timing=True)
    e1 = torch.cuda.Event(enable_timing=True)
    t0 = time.perf_counter()
    e0.record(stream)
    for _ in range(args.steps):
        step()
    e1.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3
    gpu_step_ms = e0.elapsed_time(e1) / args.steps

    # The reference's per-launch protocol (kernels/warp_tiled_ampere.py:
    # 1059-1070): an event pair around every launch; dK re-zeroed outside.
    coll = runtime.KernelEventCollector()
    coll.enabled = True
    n_ev = args.path_runs
    for _ in range(n_ev):
        rt.launch_fwd(x, w, y, coll)
    for _ in range(n_ev):
        rt.launch_bwd_input(dy, w, dx, coll)
    for _ in range(n_ev):
        gk.zero_()
        rt.launch_bwd_weight(dy, x, gk, K, coll)
    ev = {}
    for r in coll.rows(synchronize=True):
        ev.setdefault(r["phase"], []).append(r["runtime_ms"])
    for ph, v in ev.items():
        main_leg["paths"][ph]["per_launch_event_ms"] = round(mean(v), 5)

    paths = main_leg["paths"]
    agg = main_leg["fwd_dx_dk_ms"]
    dominant = max(("fwd", "bwd_input", "bwd_weight"), key=lambda k: paths[k]["ms"])
    tag = {"fwd": "fwd", "bwd_input": "dx", "bwd_weight": "dk"}[dominant]
    # The roofline takes the slower of the back-to-back and the rotated
    # (cold) timing of the dominant path.
    cold_slower = cold_paths[dominant]["ms"] > paths[dominant]["ms"]
    ach = (cold_paths if cold_slower else paths)[dominant]["gbps"]
    traffic = read_traffic(f"{tag}_{args.workload}")
    line = {
        "metric": METRIC,
        "value": round(agg, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms / args.steps, 5),
        "ms_per_step_gpu": round(gpu_step_ms, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(agg / REFERENCE_AGGREGATE_MS, 5),
        "vs_baseline_ref": "A100 PCIe aggregate 11.283 ms (README.md:96); value/ref",
        "dtype": "f32",
        "data": "synthetic (CPU torch.Generator: x, w, dY; x,dY~N(0,1), w~N(0,1/K))",
        "config": {
            "workload": f"B{B} H{H} L{L} K{K} fp32 ({args.workload}; BASELINE.json configs[1])"
            if args.workload == "primary" else f"B{B} H{H} L{L} K{K} fp32 ({args.workload})",
            "B": B, "H": H, "L": L, "K": K,
            "fwd_waves_per_block": cfg["fwd_waves_per_block"],
            "dx_waves_per_block": cfg["dx_waves_per_block"],
            "dk_threads_per_block": cfg["dk_threads_per_block"],
            "launch_config_source": cfg["source"],
        },
        "protocol": (f"value = FWD + dX + dK (atomic, excl. zero-init); per path {args.trials} trials "
                     f"x ({args.path_warmup} warm-up + {args.path_runs} launches back to back between "
                     "two events on the launch stream), order reversed on even trials, mean of trial "
                     "means; paths_rotated: the same over rotated buffer sets (no MALL reuse); "
                     "ms_per_step: wall time of `steps` FWD/dX/zero+dK steps after 0.3 s and "
                     "`warmup` warm-up steps (ms_per_step_gpu: event pair); legs: [ms, std_ms, "
                     "% of 8 TB/s]"),
        "value_std_ms": main_leg["fwd_dx_dk_std_ms"],
        "aggregate_gbps": round(3 * nbytes / (agg / 1e3) / 1e9, 1),
        "aggregate_pct_peak": main_leg["aggregate_pct_peak"],
        "algorithmic_bytes_per_path": nbytes,
        "paths": paths,
        "paths_rotated": cold_paths | {"sets": cold["sets"]},
        "check_of_timed_outputs": main_leg["check_of_timed_outputs"],
        "roofline": {
            "kernel": paths[dominant]["kernel"],
            "timing": "rotated buffers" if cold_slower else "back to back",
            "bound": "hbm",
            "achieved": ach,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBPS, 4),
            "traffic": (traffic["fetch"] + traffic["write"]) if traffic else None,
            "algorithmic_bytes": nbytes,
        },
    }
    log(f"{args.workload} contract steps: {line['ms_per_step']:.4f} ms per step (wall), "
        f"{line['ms_per_step_gpu']:.4f} ms (events)")
    if not args.no_extras:
        log("extras: BF16, channels-last, VALU FWD/dX ...")
        line.update(extras(rt, args, dev, stream, x, w, dy, y, gk))
    if args.gpu_library_steps:
        log("GPU library baseline ...")
        line["gpu_library_baseline"] = gpu_library_baseline(x, w, dy, args.gpu_library_steps)
    if args.copy_probe:
        for _ in range(args.copy_probe):
            y.copy_(x)
        torch.cuda.synchronize()
        line["copy_probe"] = {"copies": args.copy_probe, "bytes_read_per_copy": x.numel() * 4,
                              "bytes_written_per_copy": x.numel() * 4}
    del x, w, dy, y, dx, gk
    torch.cuda.empty_cache()
    if not args.no_legs:
        legs = {}
        for name in WORKLOADS:
            if name != args.workload:
                legs[name] = compact_leg(workload_leg(rt, name, args, dev, stream))
        line["baseline_configs"] = legs
    if not args.no_extras:
        log("long rows ...")
        line["long_rows"] = long_rows_leg(rt, args, dev, stream)
    if args.s4convd_steps:
        log("S4ConvD training steps ...")
        line["s4convd"] = s4convd_training_steps(args.s4convd_steps, max(3, args.warmup), dev)
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        line["cpu_baseline"] = cpu_baseline(x_cpu, w_cpu, dy_cpu, args.cpu_runs)
    rt.close()
    # The key blocks last: a reader that keeps only the end of the output
    # still sees P's per-path numbers, the rotated control and the checks.
    last = ("protocol", "baseline_configs", "paths_rotated", "paths", "check_of_timed_outputs",
            "cpu_baseline")
    line = {k: v for k, v in line.items() if k not in last} | \
        {k: line[k] for k in last if k in line}
    summary = [f"{args.workload} {path_line(paths)}"]
    for name, leg in line.get("baseline_configs", {}).items():
        summary.append(name + " " + ", ".join(
            f"{PATH_TAGS.get(k, k)} {v[0]:.4f} ms ({v[2]:.1f}%)" for k, v in leg["paths"].items()
            if k in ("fwd", "bwd_input", "bwd_weight")))
    log("summary: " + " | ".join(summary))
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
