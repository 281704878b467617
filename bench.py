"""Benchmark of the MI355X depthwise Conv1D hot path (one JSON line).

Metric: "FWD+dX+dK ms & HBM GB/s (% peak), B16384 H128 L48
K48 fp32, 1 GPU". A step is one pass of the hot path over one batch:
FWD, dX and dK (atomic, zero-init outside the dK event as in the reference's
protocol, README.md:136-140). Inputs are synthetic, drawn on a CPU
torch.Generator in the order x, w, dY (x, dY ~ N(0,1), w ~ N(0,1/K)) and
copied to HBM before timing.

    python bench.py [--gpus 1] [--steps 100] [--warmup 20] [--no-cpu-baseline]

``value`` = mean FWD + mean dX + mean dK kernel ms over the K timed steps
(HIP events on the launch stream; the reference sums separately timed path
means, kernels/warp_tiled_ampere.py:1059-1096). ``ms_per_step`` is the wall
time of the K steps / K between two device synchronisations.
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
    # parity cases, benchmarked only on request.
    "short": (32768, 256, 48, 4),
    "odd_k": (16384, 128, 48, 47),
    "edge": (1000, 96, 37, 48),
}
PEAK_HBM_GBPS = 8000.0
PEAK_FP32_MFMA_TFLOPS = 157.3  # MI355X dense FP32 matrix
# Published aggregate of the reference for this metric (README.md:96,
# A100 PCIe 40 GB): 11.283 ms.
REFERENCE_AGGREGATE_MS = 11.283
POLICY = ROOT / "pathtile_amd" / "tune" / "frozen_policy.json"
PROFILES = ROOT / "profiles"


def parse_args(argv=None):
    p = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    p.add_argument("--gpus", type=int, default=1)
    p.add_argument("--steps", type=int, default=100)
    p.add_argument("--warmup", type=int, default=20)
    p.add_argument("--workload", choices=sorted(WORKLOADS), default="primary")
    p.add_argument("--seed", type=int, default=0)
    p.add_argument("--no-cpu-baseline", action="store_true")
    p.add_argument("--cpu-runs", type=int, default=5)
    p.add_argument("--gpu-library-steps", type=int, default=0, metavar="N",
                   help="also time N calls per path of PyTorch's GPU convolution (MIOpen) "
                        "on the same tensors")
    p.add_argument("--s4convd-steps", type=int, default=0, metavar="N",
                   help="also time N S4ConvD training steps (the reference's Model() at "
                        "B16384 L48, SGD lr 1e-3 momentum 0.9) on each backend")
    p.add_argument("--copy-probe", type=int, default=0, metavar="N",
                   help="after timing, run N plain device copies of x into y "
                        "(known bytes: 2 * B*H*L*4 per copy) to calibrate "
                        "rocprofv3 FETCH_SIZE / WRITE_SIZE")
    return p.parse_args(argv)


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


def correctness_gate(rt, x, w, dy, rows: int = 512) -> dict:
    """Refuse to time a wrong kernel (benchmark/benchmark_dk_fairness.py:149-170):
    compare the HIP paths with PyTorch's own conv1d/autograd on the GPU for the
    first `rows` batch entries."""
    import torch
    import torch.nn.functional as F

    B, H, L = x.shape
    K = w.shape[1]
    xs, dys = x[:rows].contiguous(), dy[:rows].contiguous()
    y = torch.empty_like(xs)
    dx = torch.empty_like(xs)
    gk = torch.empty(H, K, device=x.device)
    rt.launch_fwd(xs, w, y)
    rt.launch_bwd_input(dys, w, dx)
    rt.launch_bwd_weight(dys, xs, gk, K, zero_first=True)
    xr = xs.double().requires_grad_(True)
    wr = w.double().requires_grad_(True)
    left = K // 2
    yr = F.conv1d(F.pad(xr, (left, K - 1 - left)), wr.unsqueeze(1), groups=H)
    gx_r, gk_r = torch.autograd.grad(yr, (xr, wr), dys.double())

    def err(a, b):
        return float((a.double() - b).abs().max() / b.abs().max().clamp_min(1e-12))

    e = {"fwd": err(y, yr.detach()), "dx": err(dx, gx_r), "dk": err(gk, gk_r)}
    ok = e["fwd"] < 1e-5 and e["dx"] < 1e-5 and e["dk"] < 1e-4
    if not ok:
        raise SystemExit(f"correctness gate failed: {e}")
    return e


def mean(v):
    return sum(v) / len(v) if v else float("nan")


def rows_kernel_name(H: int, L: int, K: int, dx: bool) -> str:
    """The FWD/DX kernel the library picks for 16-byte aligned rows: the
    channel-group matrix-core kernel where the layout allows it (L % 4 == 0,
    H % 8 == 0) and a row needs >= 10.5 (LMAX / L)^2 useful FMAs per output
    (LMAX = 16 ceil(L / 16)), else the VALU rows kernel (or either on
    request through PATHTILE_ROWS_ALGO)."""
    tag = "DX" if dx else "FWD"
    algo = os.environ.get("PATHTILE_ROWS_ALGO")
    p = K // 2
    useful = sum(max(0, min(L, L - (j - p)) - max(0, p - j)) for j in range(K))
    lmax = 16 * ((L + 15) // 16)
    mfma = algo == "mfma" or (algo != "valu" and 2 * useful * L >= 21 * lmax * lmax)
    if mfma and L % 4 == 0 and H % 8 == 0:
        return f"dwconv_rows_cg_kernel<{tag}>"
    return f"dwconv_rows_kernel<{tag}>"


def dk_kernel_name(H: int, L: int, threads: int) -> str:
    """The DK kernel the library picks for 16-byte aligned inputs: the
    channel-group matrix-core kernel when rows are whole float4 (L % 4 == 0)
    and H is a multiple of 2 x waves per workgroup (at most 8 waves), else
    the per-channel matrix-core kernel (or the VALU kernel on request)."""
    if os.environ.get("PATHTILE_DK_ALGO") == "valu":
        return "dwconv_dk_kernel"
    wpb = threads // 64
    if L % 4 == 0 and wpb <= 8 and H % (2 * wpb) == 0:
        return "dwconv_dk_cg_kernel"
    return "dwconv_dk_mfma_kernel"


def read_traffic(kernel_tag: str) -> dict | None:
    """HBM bytes per launch of `kernel_tag` from the committed rocprofv3 PMC
    summary (profiles/pmc_traffic_<kernel_tag>.md, lines
    'FETCH_BYTES_PER_LAUNCH: <n>' and 'WRITE_BYTES_PER_LAUNCH: <n>')."""
    f = PROFILES / f"pmc_traffic_{kernel_tag}.md"
    if not f.exists():
        return None
    text = f.read_text()
    m1 = re.search(r"FETCH_BYTES_PER_LAUNCH:\s*([0-9.eE+]+)", text)
    m2 = re.search(r"WRITE_BYTES_PER_LAUNCH:\s*([0-9.eE+]+)", text)
    if not (m1 and m2):
        return None
    return {"fetch": float(m1.group(1)), "write": float(m2.group(1))}


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
    B, H, L, K = WORKLOADS[args.workload]
    cfg = frozen_config()
    rt = runtime.HipWarpRuntime(waves_per_block=cfg["fwd_waves_per_block"],
                                dx_waves_per_block=cfg["dx_waves_per_block"],
                                bwdk_block=cfg["dk_threads_per_block"])
    log(f"workload B={B} H={H} L={L} K={K} config={cfg}")
    x_cpu, w_cpu, dy_cpu = make_inputs(B, H, L, K, args.seed)
    x, w, dy = x_cpu.to(dev), w_cpu.to(dev), dy_cpu.to(dev)
    y = torch.empty_like(x)
    dx = torch.empty_like(x)
    gk = torch.zeros(H, K, device=dev)
    gate = correctness_gate(rt, x, w, dy)
    log(f"correctness gate vs torch (first 512 rows): {gate}")

    def step():
        rt.launch_fwd(x, w, y)
        rt.launch_bwd_input(dy, w, dx)
        gk.zero_()
        rt.launch_bwd_weight(dy, x, gk, K)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()
    # The contract's K steps (FWD, dX, zero + dK interleaved), wall-clocked
    # between two synchronisations.
    t0 = time.perf_counter()
    for _ in range(args.steps):
        step()
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3

    # Per-path loops: `steps` back-to-back launches of one path between two
    # events recorded on the launch stream (torch's current stream, where the
    # runtime enqueues), mean = elapsed / steps. The atomic dK loop does not
    # re-zero gk (the kernel's work is the same; the zero-init is timed as its
    # own path, "bwd_weight_zero", where it is part of the call).
    stream = torch.cuda.current_stream(dev)
    loops = {
        "fwd": lambda: rt.launch_fwd(x, w, y),
        "bwd_input": lambda: rt.launch_bwd_input(dy, w, dx),
        "bwd_weight": lambda: rt.launch_bwd_weight(dy, x, gk, K),
        "bwd_weight_zero": lambda: rt.launch_bwd_weight(dy, x, gk, K, zero_first=True),
        "bwd_weight_det": lambda: rt.launch_bwd_weight_deterministic(dy, x, gk, K),
    }
    def time_loop(fn):
        for _ in range(max(1, args.warmup // 4)):
            fn()
        ev0 = torch.cuda.Event(enable_timing=True)
        ev1 = torch.cuda.Event(enable_timing=True)
        ev0.record(stream)
        for _ in range(args.steps):
            fn()
        ev1.record(stream)
        ev1.synchronize()
        return ev0.elapsed_time(ev1) / args.steps

    loop_ms = {ph: time_loop(fn) for ph, fn in loops.items()}

    # BF16 I/O (no reference counterpart): the same workload with x, dY and
    # the FWD/dX outputs in bfloat16, taps and dK in FP32, same loops. Its
    # algorithmic bytes are (2 B H L * 2 + H K * 4) per path. The BF16 entry
    # points serve the channel-group layout only (L % 4 == 0, H % 8 == 0 and
    # the dK block's channel rule), so other shapes skip the leg.
    bf16_leg = None
    dk_channels = 2 * (rt.bwdk_block // 64)
    if L % 4 == 0 and H % 8 == 0 and H % dk_channels == 0 and rt.bwdk_block <= 512:
        xb, dyb = x.to(torch.bfloat16), dy.to(torch.bfloat16)
        yb, dxb = torch.empty_like(xb), torch.empty_like(dyb)
        bf16_loops = {
            "fwd": lambda: rt.launch_fwd_bf16(xb, w, yb),
            "bwd_input": lambda: rt.launch_bwd_input_bf16(dyb, w, dxb),
            "bwd_weight": lambda: rt.launch_bwd_weight_bf16(dyb, xb, gk, K),
            "bwd_weight_det": lambda: rt.launch_bwd_weight_deterministic_bf16(dyb, xb, gk, K),
        }
        bf16_ms = {ph: time_loop(fn) for ph, fn in bf16_loops.items()}
        # gate: BF16 FWD against the FP32 path on the same (BF16-valued) input
        rows_b = min(512, B)
        y32 = torch.empty(rows_b, H, L, device=dev)
        rt.launch_fwd(xb[:rows_b].float().contiguous(), w, y32)
        torch.cuda.synchronize()
        bf16_gate = float((yb[:rows_b].float() - y32).abs().max() / y32.abs().max().clamp_min(1e-30))
        if not bf16_gate < 2.0 ** -8:
            raise SystemExit(f"BF16 gate failed: {bf16_gate}")
        del xb, dyb, yb, dxb, y32
        bf16_bytes = 2 * B * H * L * 2 + H * K * 4
        bf16_leg = {
            "paths": {
                ph: {"ms": round(ms, 5),
                     "gbps": round(bf16_bytes / (ms / 1e3) / 1e9, 1),
                     "pct_peak": round(100 * bf16_bytes / (ms / 1e3) / 1e9 / PEAK_HBM_GBPS, 2)}
                for ph, ms in bf16_ms.items()
            },
            "fwd_dx_dk_ms": round(bf16_ms["fwd"] + bf16_ms["bwd_input"] + bf16_ms["bwd_weight"], 5),
            "gate_vs_fp32_path": float(f"{bf16_gate:.3e}"),
            "note": "x, dY, y, dX bfloat16; taps and dK FP32; FP32 accumulation; "
                    "algorithmic bytes (2 B H L * 2 + H K * 4) per path",
        }

    # Channels-last dK through the Flash-DWC bridge ABI (flash_dk_fp32): x and
    # dY permuted to [B, 1, L, H] outside the timed region, dw [1, K, H]
    # accumulated into, same loop; GZ = 1 (B % 16 == 0 and H % 32 == 0 are the
    # bridge's own rules, so other shapes skip the leg). Gate: the row-major
    # deterministic dK of the same data.
    cl_leg = None
    if B % 16 == 0 and H % 32 == 0:
        xc = x.permute(0, 2, 1).unsqueeze(1).contiguous()
        dyc = dy.permute(0, 2, 1).unsqueeze(1).contiguous()
        dwc = torch.zeros(1, K, H, device=dev)
        cl_ms = time_loop(lambda: rt.launch_bwd_weight_channels_last(xc, dyc, dwc, 1))
        rt.launch_bwd_weight_deterministic(dy, x, gk, K)
        rt.launch_bwd_weight_channels_last(xc, dyc, dwc, 1, zero_first=True)
        torch.cuda.synchronize()
        cl_gate = float((dwc[0].T - gk).abs().max() / gk.abs().max().clamp_min(1e-30))
        if not cl_gate < 1e-5:
            raise SystemExit(f"channels-last dK gate failed: {cl_gate}")
        cl_gbps = runtime.algorithmic_bandwidth_gbps(runtime.minimum_algorithmic_bytes(B, H, L, K), cl_ms)
        cl_leg = {"ms": round(cl_ms, 5), "gbps": round(cl_gbps, 1),
                  "pct_peak": round(100 * cl_gbps / PEAK_HBM_GBPS, 2),
                  "kernel": f"dwconv_dk_cl_kernel<{16 * ((L + 15) // 16)}>",
                  "gate_vs_row_major": float(f"{cl_gate:.3e}"),
                  "note": "flash_dk_fp32 (x, dY [B,1,L,H]; dw [1,K,H] accumulated), GZ=1; "
                          "algorithmic bytes as the row-major dK"}
        del xc, dyc, dwc

    # Long rows at the reference's long-row benchmark shape (kernels/
    # shared_l192.py, benchmarked at B16384 H128 L192 K192 by
    # benchmark/benchmark_gmc_vs_shared_l192.py:14-17). The default kernels
    # run on the BF16 matrix cores with three-way split FP32 operands (six
    # part products); the FP32 matrix-core kernels (PATHTILE_LONG_ALGO=fp32)
    # are timed beside them. Useful flops: 2 per multiply-add that touches a
    # real element. Same loop.
    LB, LH, LL, LK = 16384, 128, 192, 192
    xl = torch.randn(LB, LH, LL, generator=torch.Generator().manual_seed(args.seed + 3)).to(dev)
    dyl = torch.randn(LB, LH, LL, generator=torch.Generator().manual_seed(args.seed + 4)).to(dev)
    wl = (torch.randn(LH, LK, generator=torch.Generator().manual_seed(args.seed + 5)) / LK ** 0.5).to(dev)
    yl, dxl, gkl = torch.empty_like(xl), torch.empty_like(dyl), torch.empty(LH, LK, device=dev)
    long_loops = {
        "fwd": lambda: rt.launch_fwd_long(xl, wl, yl),
        "bwd_input": lambda: rt.launch_bwd_input_long(dyl, wl, dxl),
        "bwd_weight": lambda: rt.launch_bwd_weight_long(dyl, xl, gkl, LK),
    }
    from pathtile_amd.tune.baselines import useful_products
    long_flops = 2 * useful_products(LB, LH, LL, LK)
    long_bytes = 2 * LB * LH * LL * 4 + LH * LK * 4

    def long_paths(ms_by_path):
        return {ph: {"ms": round(ms, 5),
                     "tflops_useful": round(long_flops / (ms / 1e3) / 1e12, 2),
                     "frac_fp32_mfma_peak": round(long_flops / (ms / 1e3) / 1e12 / PEAK_FP32_MFMA_TFLOPS, 4),
                     "hbm_pct_peak": round(100 * long_bytes / (ms / 1e3) / 1e9 / PEAK_HBM_GBPS, 2)}
                for ph, ms in ms_by_path.items()}

    prev_long = os.environ.pop("PATHTILE_LONG_ALGO", None)
    long_ms = {ph: time_loop(fn) for ph, fn in long_loops.items()}
    # gate on the first 256 samples (a small copy: the profiles' copy probe
    # is the largest plain copy of the run)
    y_split = yl[:256].clone()
    os.environ["PATHTILE_LONG_ALGO"] = "fp32"
    long_ms_fp32 = {ph: time_loop(fn) for ph, fn in long_loops.items()}
    rt.launch_fwd_long(xl, wl, yl)
    torch.cuda.synchronize()
    long_gate = float((y_split - yl[:256]).abs().max() / yl[:256].abs().max())
    if prev_long is None:
        del os.environ["PATHTILE_LONG_ALGO"]
    else:
        os.environ["PATHTILE_LONG_ALGO"] = prev_long
    if not long_gate < 1e-5:
        raise SystemExit(f"long-row split vs FP32 gate failed: {long_gate}")
    long_leg = {
        "config": {"B": LB, "H": LH, "L": LL, "K": LK},
        "paths": long_paths(long_ms),
        "fwd_dx_dk_ms": round(sum(long_ms.values()), 5),
        "kernels": {"fwd": "dwconv_rows_long_s3_kernel<192, 192, false, true>",
                    "bwd_input": "dwconv_rows_long_s3_kernel<192, 192, true, true>",
                    "bwd_weight": "dwconv_dk_long_s3_kernel<192, true>"},
        "fp32_mfma_kernels": {"paths": long_paths(long_ms_fp32),
                              "fwd_dx_dk_ms": round(sum(long_ms_fp32.values()), 5)},
        "gate_split_vs_fp32_fwd": float(f"{long_gate:.3e}"),
        "note": "pt_dwconv1d_{fwd,dx,dk}_long_f32; default = BF16 matrix cores on three-way split "
                "FP32 operands (FP32-accurate), fp32_mfma_kernels = PATHTILE_LONG_ALGO=fp32; useful "
                "flops 2 * sum over rows of real multiply-adds; FP32 matrix peak 157.3 TFLOP/s; "
                "HBM bytes 2 B H L 4 + H K 4 per path",
    }
    del xl, dyl, wl, yl, dxl, gkl

    # The VALU rows kernel (the reference's lane-per-row structure, bit-exact
    # with its fmaf chain) timed beside the default FWD/DX kernel, same loops.
    prev = os.environ.get("PATHTILE_ROWS_ALGO")
    os.environ["PATHTILE_ROWS_ALGO"] = "valu"
    valu_gate = correctness_gate(rt, x, w, dy)
    valu_ms = {"fwd": time_loop(loops["fwd"]), "bwd_input": time_loop(loops["bwd_input"])}
    valu_kernels = {"fwd": rows_kernel_name(H, L, K, False), "bwd_input": rows_kernel_name(H, L, K, True)}
    if prev is None:
        del os.environ["PATHTILE_ROWS_ALGO"]
    else:
        os.environ["PATHTILE_ROWS_ALGO"] = prev

    # The reference's per-launch protocol (kernels/warp_tiled_ampere.py:
    # 1059-1070; benchmark/benchmark_pathtile_candidate_sweep.py:274-317):
    # an event pair around every launch; dK re-zeroed outside the events.
    coll = runtime.KernelEventCollector()
    coll.enabled = True
    for _ in range(args.steps):
        rt.launch_fwd(x, w, y, coll)
    for _ in range(args.steps):
        rt.launch_bwd_input(dy, w, dx, coll)
    for _ in range(args.steps):
        gk.zero_()
        rt.launch_bwd_weight(dy, x, gk, K, coll)
    for _ in range(args.steps):
        rt.launch_bwd_weight(dy, x, gk, K, coll, zero_first=True)
    for _ in range(args.steps):
        rt.launch_bwd_weight_deterministic(dy, x, gk, K, coll)
    rows = coll.rows(synchronize=True)
    per = {ph: [r["runtime_ms"] for r in rows if r["phase"] == ph]
           for ph in ("fwd", "bwd_input", "bwd_weight", "bwd_weight_zero", "bwd_weight_det")}
    assert all(len(v) == args.steps for v in per.values())

    nbytes = runtime.minimum_algorithmic_bytes(B, H, L, K)
    paths = {}
    for ph, v in per.items():
        ms = loop_ms[ph]
        gbps = runtime.algorithmic_bandwidth_gbps(nbytes, ms)
        paths[ph] = {"ms": round(ms, 5),
                     "gbps": round(gbps, 1), "pct_peak": round(100 * gbps / PEAK_HBM_GBPS, 2),
                     "per_launch_event_ms": round(mean(v), 5),
                     "per_launch_event_min_ms": round(min(v), 5)}
    agg = paths["fwd"]["ms"] + paths["bwd_input"]["ms"] + paths["bwd_weight"]["ms"]
    kernels = {"fwd": rows_kernel_name(H, L, K, False), "bwd_input": rows_kernel_name(H, L, K, True),
               "bwd_weight": dk_kernel_name(H, L, cfg["dk_threads_per_block"])}
    for ph in paths:
        paths[ph]["kernel"] = kernels[{"bwd_weight_zero": "bwd_weight",
                                       "bwd_weight_det": "bwd_weight"}.get(ph, ph)]
    dominant = max(("fwd", "bwd_input", "bwd_weight"), key=lambda k: paths[k]["ms"])
    tag = {"fwd": "fwd", "bwd_input": "dx", "bwd_weight": "dk"}[dominant]
    ach = paths[dominant]["gbps"]
    traffic = read_traffic(f"{tag}_{args.workload}")
    line = {
        "metric": METRIC,
        "value": round(agg, 5),
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(wall_ms / args.steps, 5),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": round(agg / REFERENCE_AGGREGATE_MS, 5),
        "vs_baseline_ref": "reference aggregate 11.283 ms on A100 PCIe (README.md:96); value/ref, lower is better",
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
        "protocol": ("value = FWD + dX + dK (atomic, excl. zero-init) mean launch times; "
                     "each path runs `steps` back-to-back launches between two HIP events on "
                     "the launch stream; paths.*.per_launch_event_ms = the reference's "
                     "protocol (an event pair per launch); ms_per_step = wall time of "
                     "`steps` interleaved FWD/dX/zero+dK steps"),
        "aggregate_gbps": round(3 * nbytes / (agg / 1e3) / 1e9, 1),
        "aggregate_pct_peak": round(100 * 3 * nbytes / (agg / 1e3) / 1e9 / PEAK_HBM_GBPS, 2),
        "algorithmic_bytes_per_path": nbytes,
        "paths": paths,
        "correctness_gate": {k: float(f"{v:.3e}") for k, v in gate.items()},
        "bf16_io": bf16_leg,
        "channels_last_dk": cl_leg,
        "long_rows": long_leg,
        "rows_valu": {
            ph: {"ms": round(ms, 5), "pct_peak": round(100 * runtime.algorithmic_bandwidth_gbps(nbytes, ms)
                                                     / PEAK_HBM_GBPS, 2),
                 "kernel": valu_kernels[ph]}
            for ph, ms in valu_ms.items()
        } | {"correctness_gate": {k: float(f"{v:.3e}") for k, v in valu_gate.items()},
             "note": "PATHTILE_ROWS_ALGO=valu: the bit-exact VALU FWD/DX kernel, same loops"},
        "roofline": {
            "kernel": kernels[dominant],
            "bound": "hbm",
            "achieved": ach,
            "peak": PEAK_HBM_GBPS,
            "unit": "GB/s",
            "frac": round(ach / PEAK_HBM_GBPS, 4),
            "traffic": (traffic["fetch"] + traffic["write"]) if traffic else None,
            "algorithmic_bytes": nbytes,
        },
    }
    if args.gpu_library_steps:
        log("GPU library baseline ...")
        line["gpu_library_baseline"] = gpu_library_baseline(x, w, dy, args.gpu_library_steps)
    if args.s4convd_steps:
        log("S4ConvD training steps ...")
        line["s4convd"] = s4convd_training_steps(args.s4convd_steps, max(3, args.warmup // 4), dev)
    if args.copy_probe:
        for _ in range(args.copy_probe):
            y.copy_(x)
        torch.cuda.synchronize()
        line["copy_probe"] = {"copies": args.copy_probe, "bytes_read_per_copy": x.numel() * 4,
                              "bytes_written_per_copy": x.numel() * 4}
    if not args.no_cpu_baseline:
        log("cpu baseline ...")
        line["cpu_baseline"] = cpu_baseline(x_cpu, w_cpu, dy_cpu, args.cpu_runs)
    rt.close()
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
