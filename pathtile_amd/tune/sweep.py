"""PathTile candidate sweep on one MI355X (needs a GPU).

Follows the reference's measurement contract
(benchmark/benchmark_pathtile_candidate_sweep.py:153-317, 493-712;
artifact/REPRODUCIBILITY.md:81-93, 130-131):
* candidates: FWD/dX wavefronts per workgroup, dK threads per workgroup;
  every candidate is validated against PyTorch on the GPU at
  B = min(B, 128) with full H, L, K before it is timed;
* per (shape, candidate): warm-up launches, then `runs` launches each
  bracketed by events on the launch stream; dK's output is zeroed outside
  the event;
* trials repeat the sweep with candidate and shape order reversed on even
  trials; the summary is the mean of trial means.
Unlike the reference (a fresh nvcc JIT per candidate), every candidate is a
runtime argument of the one prebuilt library, so a sweep compiles nothing.
"""

from __future__ import annotations

import math
import platform
import socket
import time
import zlib
from datetime import datetime, timezone

import torch
import torch.nn.functional as F

from .. import runtime as rt
from .shapes import ShapeCase

FWD_DX_KIND = "waves_per_block"
DK_KIND = "dk_threads_per_block"
# 64-lane wavefronts per workgroup. 16 waves (1024 threads) does not fit the
# LDS tile of rows longer than 32, which the grid contains, so it is not a
# candidate (it would be missing on those shapes).
FWD_DX_CANDIDATES = (1, 2, 4, 8)
DK_CANDIDATES = (64, 128, 192, 256, 384, 512)


def control_specs() -> list[tuple[str, int]]:
    """Duplicate control: the runtime's current launch values (the installed
    frozen policy), timed a second time per shape after every candidate, so
    two measurements of one configuration give the regret's noise floor
    (scripts/aggregate_pathtile_results.py:223-240 reads regret against such
    a floor). Their rows never enter the selection."""
    return [(FWD_DX_KIND, int(rt.DEFAULT_WAVES_PER_BLOCK)),
            (DK_KIND, int(rt.DEFAULT_BWDK_BLOCK))]


def utc_now() -> str:
    return datetime.now(timezone.utc).isoformat()


def stats(values) -> dict:
    """benchmark/benchmark_pathtile_candidate_sweep.py:77-106."""
    v = sorted(float(x) for x in values)
    n = len(v)
    if n == 0:
        raise ValueError("Cannot summarize an empty measurement group")
    mean = sum(v) / n
    std = math.sqrt(sum((x - mean) ** 2 for x in v) / (n - 1)) if n > 1 else 0.0
    sem = std / math.sqrt(n) if n > 1 else 0.0

    def q(p):
        pos = p * (n - 1)
        lo, hi = math.floor(pos), math.ceil(pos)
        return v[lo] + (v[hi] - v[lo]) * (pos - lo)

    return {"n": n, "mean_ms": mean, "median_ms": q(0.5), "std_ms": std, "sem_ms": sem,
            "ci95_low_ms": mean - 1.96 * sem, "ci95_high_ms": mean + 1.96 * sem,
            "min_ms": v[0], "p05_ms": q(0.05), "p95_ms": q(0.95), "max_ms": v[-1]}


def case_seed(base_seed: int, case: ShapeCase) -> int:
    """benchmark/benchmark_pathtile_candidate_sweep.py:109-110."""
    return int(base_seed + zlib.crc32(case.config_id.encode("utf-8")))


def make_inputs(case: ShapeCase, seed: int, batch_override: int | None = None):
    """x, w, dY on the GPU from a seeded generator: x, dY ~ N(0,1),
    w ~ N(0, 1/K) (the reference draws w ~ N(0,1), :113-124)."""
    g = torch.Generator(device="cuda").manual_seed(seed)
    B = int(case.B if batch_override is None else batch_override)
    x = torch.randn(B, case.H, case.L, device="cuda", generator=g)
    w = torch.randn(case.H, case.K, device="cuda", generator=g) / math.sqrt(case.K)
    dy = torch.randn(B, case.H, case.L, device="cuda", generator=g)
    return x, w, dy


def _torch_same(x, k):
    K = int(k.shape[1])
    left = K // 2
    return F.conv1d(F.pad(x, (left, K - 1 - left)), k.unsqueeze(1), groups=int(x.shape[1]))


def make_runtime(kind: str, value: int) -> rt.HipWarpRuntime:
    if kind == FWD_DX_KIND:
        return rt.HipWarpRuntime(waves_per_block=value, dx_waves_per_block=value)
    return rt.HipWarpRuntime(bwdk_block=value)


def validate_candidate(runtime, case: ShapeCase, seed: int, kind: str, value: int) -> list[dict]:
    """Candidate vs PyTorch (FP64 on the GPU) at B = min(B, 128)
    (benchmark/benchmark_pathtile_candidate_sweep.py:153-243). Tolerances:
    the reference's allclose bars and the build's own bars (FWD/dX <= 1e-5,
    dK <= 1e-4 max-abs-scaled)."""
    vb = min(case.B, 128)
    x, k, gy = make_inputs(case, seed, batch_override=vb)
    xr = x.double().requires_grad_(True)
    kr = k.double().requires_grad_(True)
    yr = _torch_same(xr, kr)
    gx_r, gk_r = torch.autograd.grad(yr, (xr, kr), gy.double())
    rows = []

    def row(phase, actual, expected, atol, rtol, bar):
        err = float((actual.double() - expected).abs().max() / expected.abs().max().clamp_min(1e-12))
        ok = bool(torch.allclose(actual.double(), expected, atol=atol, rtol=rtol)) and err <= bar
        rows.append({**case.as_dict(), "candidate_kind": kind, "candidate_value": value,
                     "validation_B": vb, "phase": phase, "normalized_max_abs": err, "allclose": ok})

    if kind == FWD_DX_KIND:
        y = torch.empty_like(x)
        gx = torch.empty_like(x)
        runtime.launch_fwd(x, k, y)
        runtime.launch_bwd_input(gy, k, gx)
        row("fwd", y, yr.detach(), 2e-3, 2e-3, 1e-5)
        row("bwd_input", gx, gx_r, 2e-3, 2e-3, 1e-5)
    else:
        gk = torch.zeros_like(k)
        runtime.launch_bwd_weight(gy, x, gk, case.K)
        row("bwd_weight", gk, gk_r, 1e-2, 5e-4, 1e-4)
    torch.cuda.synchronize()
    return rows


# MI355X has a 256 MiB memory-side cache (MALL). Tensors of the smaller
# tuning shapes fit in it, and back-to-back launches on the same buffers would
# then time the cache, not HBM. Each candidate therefore cycles through enough
# buffer sets (x, dY, y, dX) to exceed this footprint, so every launch streams
# from HBM and pays for evicting the previous launches' outputs, as it does in
# a training step.
ROTATION_BYTES = 1 << 29


def buffer_sets(x, gy) -> list[tuple]:
    """(x, dY, y, dX) sets: the seeded inputs plus copies, enough to exceed
    ROTATION_BYTES; copies hold the same values."""
    per_set = 4 * x.numel() * x.element_size()
    n = max(1, -(-ROTATION_BYTES // per_set))
    sets = [(x, gy, torch.empty_like(x), torch.empty_like(x))]
    for _ in range(n - 1):
        sets.append((x.clone(), gy.clone(), torch.empty_like(x), torch.empty_like(x)))
    return sets


def measure_candidate(runtime, kind: str, sets: list[tuple], k, warmup: int,
                      runs: int, outputs: dict | None = None) -> dict[str, list[float]]:
    """Warm-up, then `runs` event-timed launches per path, cycling through the
    buffer sets (benchmark/benchmark_pathtile_candidate_sweep.py:246-317).
    With `outputs`, the FWD/dX outputs start as NaN and the last timed
    launches' results are returned in it ("fwd", "bwd_input": one buffer
    set's y and dX; "bwd_weight": dK of the last timed launch)."""
    K = int(k.shape[1])
    coll = rt.KernelEventCollector()
    coll.enabled = True
    n = len(sets)
    if kind == FWD_DX_KIND:
        if outputs is not None:
            for _, _, y, gx in sets:
                y.fill_(float("nan"))
                gx.fill_(float("nan"))
        for i in range(warmup):
            x, gy, y, gx = sets[i % n]
            runtime.launch_fwd(x, k, y)
            runtime.launch_bwd_input(gy, k, gx)
        torch.cuda.synchronize()
        for i in range(runs):
            x, gy, y, gx = sets[i % n]
            runtime.launch_fwd(x, k, y, coll)
        for i in range(runs):
            x, gy, y, gx = sets[i % n]
            runtime.launch_bwd_input(gy, k, gx, coll)
        if outputs is not None:
            last = sets[(runs - 1) % n]
            outputs["fwd"], outputs["bwd_input"] = last[2], last[3]
    else:
        gk = torch.zeros_like(k)
        for i in range(warmup):
            x, gy, _, _ = sets[i % n]
            gk.zero_()
            runtime.launch_bwd_weight(gy, x, gk, K)
        torch.cuda.synchronize()
        for i in range(runs):
            x, gy, _, _ = sets[i % n]
            gk.zero_()
            runtime.launch_bwd_weight(gy, x, gk, K, coll)
        if outputs is not None:
            outputs["bwd_weight"] = gk
    out: dict[str, list[float]] = {}
    for r in coll.rows(synchronize=True):
        out.setdefault(r["phase"], []).append(r["runtime_ms"])
    return out


# Batch rows of the timed FWD/dX outputs compared against FP64 (the first
# and last sample among them: the ragged tail steps).
TIMED_CHECK_ROWS = 64


class TimedCheck:
    """FP64 references of one shape's full-size inputs on the GPU, and the
    check of a candidate's timed outputs against them: FWD and dX on sampled
    batch rows (all channels), dK over the whole batch, each within the
    build's bars (1e-5, 1e-5, 1e-4 max-abs-scaled). This gates the timing on
    correctness at the size that is timed, as the reference's sweep gates
    each schedule (benchmark/benchmark_pathtile_candidate_sweep.py:
    153-243), not only at the validation size."""

    def __init__(self, case: ShapeCase, seed: int, x, k, gy):
        self.case = case
        B, K = case.B, case.K
        g = torch.Generator().manual_seed(seed + 1)
        n = min(B, TIMED_CHECK_ROWS)
        inner = torch.randperm(B - 2, generator=g)[:max(0, n - 2)] + 1 if B > 2 else \
            torch.empty(0, dtype=torch.long)
        idx = torch.cat([torch.tensor([0]), inner, torch.tensor([B - 1] if B > 1 else [])]).long()
        self.idx = idx.to(x.device)
        kd = k.double()
        self.y = _torch_same(x[self.idx].double(), kd)
        # dX[b,h,s] = sum_j w[h,j] dY[b,h,s-j+p]: a correlation with the
        # flipped taps, padded (K-1-p, p)
        p = K // 2
        self.gx = F.conv1d(F.pad(gy[self.idx].double(), (K - 1 - p, p)),
                           kd.flip(-1).unsqueeze(1), groups=case.H)
        L = case.L
        xp = F.pad(x.double(), (p, K - 1 - p))
        gyd = gy.double()
        self.gk = torch.stack([(gyd * xp[..., j:j + L]).sum(dim=(0, 2)) for j in range(K)], dim=1)
        del xp, gyd

    @staticmethod
    def _err(a, ref) -> float:
        return float((a.double() - ref).abs().max() / ref.abs().max().clamp_min(1e-12))

    def rows(self, kind: str, value: int, outputs: dict) -> list[dict]:
        got = {}
        if "fwd" in outputs:
            got["fwd"] = (self._err(outputs["fwd"][self.idx], self.y), 1e-5)
            got["bwd_input"] = (self._err(outputs["bwd_input"][self.idx], self.gx), 1e-5)
        if "bwd_weight" in outputs:
            got["bwd_weight"] = (self._err(outputs["bwd_weight"], self.gk), 1e-4)
        return [{**self.case.as_dict(), "candidate_kind": kind, "candidate_value": value,
                 "validation_B": self.case.B, "phase": ph, "normalized_max_abs": err,
                 "allclose": bool(err <= bar), "source": "timed launches"}
                for ph, (err, bar) in got.items()]


def candidate_specs(trial_id: int) -> list[tuple[str, int]]:
    """benchmark/benchmark_pathtile_candidate_sweep.py:485-490."""
    specs = [(FWD_DX_KIND, v) for v in FWD_DX_CANDIDATES]
    specs += [(DK_KIND, v) for v in DK_CANDIDATES]
    if trial_id % 2 == 0:
        specs.reverse()
    return specs


def run_trial(cases: list[ShapeCase], trial_id: int, warmup: int, runs: int,
              base_seed: int = 0, log=print) -> dict:
    """One trial over all cases and candidates; returns summary rows,
    validation rows and metadata (benchmark/benchmark_pathtile_candidate_
    sweep.py:493-712)."""
    if trial_id <= 0:
        raise ValueError("trial_id must be positive")
    created = utc_now()
    order = list(reversed(cases)) if trial_id % 2 == 0 else list(cases)
    specs = candidate_specs(trial_id)
    controls = control_specs()
    runtimes = {(k, v): make_runtime(k, v) for k, v in specs}
    summary, control, validation = [], [], []
    t0 = time.time()
    for case in order:
        seed = case_seed(base_seed, case)
        for kind, value in specs:
            validation += validate_candidate(runtimes[(kind, value)], case, seed, kind, value)
        x, k, gy = make_inputs(case, seed)
        check = TimedCheck(case, seed, x, k, gy)
        sets = buffer_sets(x, gy)
        for kind, value in specs:
            outputs: dict = {}
            times = measure_candidate(runtimes[(kind, value)], kind, sets, k, warmup, runs,
                                      outputs)
            validation += check.rows(kind, value, outputs)
            for phase, vals in times.items():
                summary.append({**case.as_dict(), "trial_id": trial_id, "candidate_kind": kind,
                                "candidate_value": value, "phase": phase,
                                "buffer_sets": len(sets), **stats(vals)})
        for kind, value in controls:
            times = measure_candidate(runtimes[(kind, value)], kind, sets, k, warmup, runs)
            for phase, vals in times.items():
                control.append({**case.as_dict(), "trial_id": trial_id, "candidate_kind": kind,
                                "candidate_value": value, "phase": phase,
                                "buffer_sets": len(sets), **stats(vals)})
        del x, k, gy, sets, check
        torch.cuda.empty_cache()
        log(f"[tune] trial {trial_id} {case.config_id} done ({time.time() - t0:.1f}s)")
    bad = [v for v in validation if not v["allclose"]]
    if bad:
        raise AssertionError(f"candidate correctness failure: {bad[:3]}")
    meta = {
        "trial_id": trial_id, "created_at_utc": created, "finished_at_utc": utc_now(),
        "device_name": torch.cuda.get_device_name(0), "hostname": socket.gethostname(),
        "python": platform.python_version(), "torch": torch.__version__,
        "hip": torch.version.hip, "warmup": warmup, "runs": runs, "base_seed": base_seed,
        "candidates": {"fwd_dx_waves_per_block": list(FWD_DX_CANDIDATES),
                       "dk_threads_per_block": list(DK_CANDIDATES)},
        "measurement_contract": "warm-up then event-timed launches per path on the launch "
                                "stream, cycling buffer sets past the 256 MiB MALL; dK "
                                "zero-fill outside the event; mean of trial means",
    }
    meta["control"] = {kind: value for kind, value in controls}
    return {"summary": summary, "control": control, "validation": validation, "metadata": meta}
