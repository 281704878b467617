"""PathTile selection and regret arithmetic (CPU only, no device).

Restates, on plain row dicts instead of pandas frames:
* per-shape / per-path oracle: fastest candidate, ties kept in row order
  (benchmark/benchmark_pathtile_candidate_sweep.py:354-424, 427-474);
* the frozen per-path policy: sum of mean_ms over the tuning shapes per
  candidate value, argmin, ties to the smaller value
  (scripts/aggregate_pathtile_results.py:223-240);
* held-out regret of the frozen policy against the per-shape oracle total
  (scripts/aggregate_pathtile_results.py:376-527) and the frozen-before-
  holdout timestamp check (:258-284).

A row is {"config_id", "B", "H", "L", "K", "phase", "candidate_value",
"mean_ms", ...}; phases are "fwd", "bwd_input", "bwd_weight".
"""

from __future__ import annotations

import math
from datetime import datetime
from typing import Iterable


PHASES = ("fwd", "bwd_input", "bwd_weight")
POLICY_KEYS = {
    "fwd": "fwd_waves_per_block",
    "bwd_input": "dx_waves_per_block",
    "bwd_weight": "dk_threads_per_block",
}


def normalize_roundoff(value: float, tolerance: float = 1e-12) -> float:
    """scripts/artifact_common.py:48-49."""
    return 0.0 if math.isfinite(value) and abs(value) < tolerance else float(value)


def geometric_mean(values: Iterable[float]) -> float:
    vals = [float(v) for v in values]
    if not vals or any((not math.isfinite(v)) or v <= 0.0 for v in vals):
        raise ValueError(f"Invalid geometric-mean values: {vals}")
    return math.exp(sum(math.log(v) for v in vals) / len(vals))


def mean_of_trials(rows: list[dict]) -> list[dict]:
    """Average trial means per (config, phase, candidate): the reference's
    'mean of trial means' (artifact/REPRODUCIBILITY.md:81-93)."""
    groups: dict[tuple, list[dict]] = {}
    for r in rows:
        key = (r["config_id"], r["phase"], int(r["candidate_value"]))
        groups.setdefault(key, []).append(r)
    out = []
    for (cid, phase, value), g in groups.items():
        means = [float(r["mean_ms"]) for r in g]
        m = sum(means) / len(means)
        std = (math.sqrt(sum((x - m) ** 2 for x in means) / (len(means) - 1))
               if len(means) > 1 else 0.0)
        base = {k: g[0][k] for k in ("config_id", "B", "H", "L", "K") if k in g[0]}
        out.append({**base, "phase": phase, "candidate_value": value,
                    "mean_ms": m, "between_trial_std_ms": std, "trials": len(means)})
    return out


def oracle(rows: list[dict]) -> dict[tuple[str, str], dict]:
    """Fastest candidate per (config_id, phase); a stable sort keeps the
    first of equal means (the reference sorts by mean_ms, kind='stable')."""
    by: dict[tuple[str, str], list[dict]] = {}
    for r in rows:
        by.setdefault((r["config_id"], r["phase"]), []).append(r)
    out = {}
    for key, g in by.items():
        ordered = sorted(g, key=lambda r: float(r["mean_ms"]))
        best = ordered[0]
        second = ordered[1] if len(ordered) > 1 else best
        out[key] = {
            "winner_value": int(best["candidate_value"]),
            "winner_mean_ms": float(best["mean_ms"]),
            "second_value": int(second["candidate_value"]),
            "second_mean_ms": float(second["mean_ms"]),
            "winner_margin_vs_second_pct": (float(second["mean_ms"]) / float(best["mean_ms"]) - 1.0) * 100.0,
        }
    return out


def combined_oracle(rows: list[dict]) -> dict[str, dict]:
    """Per shape: per-path winners and the oracle total FWD + dX + dK."""
    orc = oracle(rows)
    shapes = sorted({r["config_id"] for r in rows})
    out = {}
    for cid in shapes:
        phases = {ph for (c, ph) in orc if c == cid}
        if phases != set(PHASES):
            raise RuntimeError(f"Missing path result for {cid}: found={sorted(phases)}")
        out[cid] = {
            "fwd_winner": orc[(cid, "fwd")]["winner_value"],
            "bwd_input_winner": orc[(cid, "bwd_input")]["winner_value"],
            "bwd_weight_winner": orc[(cid, "bwd_weight")]["winner_value"],
            "oracle_total_ms": sum(orc[(cid, ph)]["winner_mean_ms"] for ph in PHASES),
        }
    return out


def select_policy(training: list[dict]) -> dict[str, int]:
    """Per path: the candidate value minimising the sum of mean_ms over the
    tuning shapes; ties go to the smaller value
    (scripts/aggregate_pathtile_results.py:223-240). Only candidates measured
    on every tuning shape of the path compete."""
    selected = {}
    for phase, name in POLICY_KEYS.items():
        rows = [r for r in training if r["phase"] == phase]
        if not rows:
            raise ValueError(f"No training candidates for {phase}")
        shapes = {r["config_id"] for r in rows}
        totals: dict[int, float] = {}
        seen: dict[int, set] = {}
        for r in rows:
            v = int(r["candidate_value"])
            totals[v] = totals.get(v, 0.0) + float(r["mean_ms"])
            seen.setdefault(v, set()).add(r["config_id"])
        complete = [(t, v) for v, t in totals.items() if seen[v] == shapes]
        if not complete:
            raise ValueError(f"No candidate of {phase} covers every tuning shape")
        selected[name] = sorted(complete)[0][1]
    return selected


def selected_time(rows: list[dict], config_id: str, phase: str, value: int) -> float:
    """scripts/aggregate_pathtile_results.py:243-255."""
    hits = [r for r in rows if r["config_id"] == config_id and r["phase"] == phase
            and int(r["candidate_value"]) == int(value)]
    if len(hits) != 1:
        raise RuntimeError(f"Expected one row for {config_id}/{phase}/{value}, found {len(hits)}")
    return float(hits[0]["mean_ms"])


def holdout_regret(rows: list[dict], policy: dict[str, int]) -> tuple[list[dict], dict]:
    """Per held-out shape: frozen total vs oracle total, regret in percent;
    plus the summary the reference reports (mean/median/max regret,
    runtime-weighted regret, shapes within 1% and 2%, exact-oracle shapes)."""
    comb = combined_oracle(rows)
    per_shape = []
    for cid, orc in sorted(comb.items()):
        base = next(r for r in rows if r["config_id"] == cid)
        fwd = selected_time(rows, cid, "fwd", policy["fwd_waves_per_block"])
        dx = selected_time(rows, cid, "bwd_input", policy["dx_waves_per_block"])
        dk = selected_time(rows, cid, "bwd_weight", policy["dk_threads_per_block"])
        frozen = fwd + dx + dk
        oracle_total = orc["oracle_total_ms"]
        per_shape.append({
            "config_id": cid, "B": base.get("B"), "H": base.get("H"),
            "L": base.get("L"), "K": base.get("K"),
            "frozen_fwd_ms": fwd, "frozen_bwd_input_ms": dx, "frozen_bwd_weight_ms": dk,
            "frozen_total_ms": frozen, "oracle_total_ms": oracle_total,
            "absolute_gap_us": normalize_roundoff((frozen - oracle_total) * 1000.0),
            "regret_pct": normalize_roundoff((frozen / oracle_total - 1.0) * 100.0),
            "exact_oracle_schedule": (
                policy["fwd_waves_per_block"] == orc["fwd_winner"]
                and policy["dx_waves_per_block"] == orc["bwd_input_winner"]
                and policy["dk_threads_per_block"] == orc["bwd_weight_winner"]),
            "fwd_winner": orc["fwd_winner"], "bwd_input_winner": orc["bwd_input_winner"],
            "bwd_weight_winner": orc["bwd_weight_winner"],
        })
    regrets = sorted(r["regret_pct"] for r in per_shape)
    n = len(regrets)
    median = (regrets[n // 2] if n % 2 else 0.5 * (regrets[n // 2 - 1] + regrets[n // 2])) if n else float("nan")
    summary = {
        "shapes": n,
        "mean_regret_pct": sum(regrets) / n if n else float("nan"),
        "median_regret_pct": median,
        "max_regret_pct": max(regrets) if n else float("nan"),
        "runtime_weighted_regret_pct": (
            sum(r["frozen_total_ms"] for r in per_shape)
            / sum(r["oracle_total_ms"] for r in per_shape) - 1.0) * 100.0 if n else float("nan"),
        "shapes_within_1pct": sum(1 for r in regrets if r <= 1.0),
        "shapes_within_2pct": sum(1 for r in regrets if r <= 2.0),
        "exact_oracle_schedule_shapes": sum(1 for r in per_shape if r["exact_oracle_schedule"]),
        "oracle_geomean_speedup_vs_frozen": geometric_mean(
            r["frozen_total_ms"] / r["oracle_total_ms"] for r in per_shape) if n else float("nan"),
    }
    return per_shape, summary


def verify_frozen_before_holdout(policy: dict, holdout_created_at: Iterable[str]) -> None:
    """The frozen policy must predate every held-out trial
    (scripts/aggregate_pathtile_results.py:258-284)."""
    if policy.get("frozen_before_holdout") is not True:
        raise AssertionError("Frozen-policy marker is missing")
    frozen_at = datetime.fromisoformat(str(policy["frozen_at_utc"]))
    for stamp in holdout_created_at:
        if not frozen_at < datetime.fromisoformat(str(stamp)):
            raise AssertionError(f"Policy timestamp {frozen_at} is not before holdout trial {stamp}")


# --------------------------------------------------------------------------
# Additions on MI355X: per-path regret, the pairs where a knob cannot act,
# and the noise floor of two measurements of one configuration.
# --------------------------------------------------------------------------
KNOB_INERT_RULE = (
    "FWD/dX waves per workgroup cannot change the kernel where the matrix-core "
    "FWD/dX kernel serves (H % 8 == 0 and, for L % 4 == 0 with 16 <= L <= 48, K at "
    "least a threshold by L: 5 at L = 16, 9 at L = 20-32 and 44, 17 at L = 36 and 40, "
    "9 at L = 48 on tensors of at most 256 MiB with H <= 128 and 17 otherwise, higher "
    "on calls of fewer than 2^17 rows; for L < 16 >= 10.5 (16 / L)^2 useful FMAs per "
    "output; for L % 4 != 0 every call of >= 2^18 rows and smaller ones from 5 "
    "(LMAX / L)^2, LMAX = 16 ceil(L / 16)): it always runs 8- or 16-wave workgroups. "
    "There the FWD/dX candidates differ only by measurement noise.")


def fwd_dx_knob_inert(H: int, L: int, K: int, B: int) -> bool:
    """True where the FWD/dX knob cannot change the kernel: where the
    library's matrix-core rule serves a 16-byte aligned call (the tuner's
    tensors are torch allocations), as the library's dispatch reports it
    (pt_rows_kernel_id)."""
    from .. import runtime

    return runtime.rows_on_matrix_cores(B, H, L, K)


def path_regret(rows: list[dict], policy: dict[str, int]) -> dict[str, dict]:
    """Per path: sum over shapes of the frozen candidate's time against the
    per-shape fastest, and the mean of the per-shape path regrets."""
    orc = oracle(rows)
    out = {}
    for phase, key in POLICY_KEYS.items():
        shapes = sorted({c for (c, ph) in orc if ph == phase})
        frozen = [selected_time(rows, c, phase, policy[key]) for c in shapes]
        best = [orc[(c, phase)]["winner_mean_ms"] for c in shapes]
        regs = [(f / b - 1.0) * 100.0 for f, b in zip(frozen, best)]
        out[phase] = {
            "shapes": len(shapes),
            "sum_regret_pct": normalize_roundoff((sum(frozen) / sum(best) - 1.0) * 100.0),
            "mean_regret_pct": normalize_roundoff(sum(regs) / len(regs)),
            "max_regret_pct": normalize_roundoff(max(regs)),
        }
        if phase != "bwd_weight":
            inert = [c for c in shapes if fwd_dx_knob_inert(*_hlkb(rows, c))]
            out[phase]["shapes_knob_inert"] = len(inert)
    return out


def _hlkb(rows: list[dict], config_id: str) -> tuple[int, int, int, int]:
    r = next(r for r in rows if r["config_id"] == config_id)
    return int(r["H"]), int(r["L"]), int(r["K"]), int(r["B"])


def active_knob_regret(rows: list[dict], policy: dict[str, int]) -> dict:
    """Regret of the frozen policy when the FWD/dX paths whose knob cannot
    act count at the frozen candidate's time on both sides (their spread is
    measurement noise, not a choice the policy could improve)."""
    orc = oracle(rows)
    regs = []
    for cid in sorted({r["config_id"] for r in rows}):
        inert = fwd_dx_knob_inert(*_hlkb(rows, cid))
        frozen = best = 0.0
        for phase, key in POLICY_KEYS.items():
            f = selected_time(rows, cid, phase, policy[key])
            frozen += f
            best += f if (inert and phase != "bwd_weight") else orc[(cid, phase)]["winner_mean_ms"]
        regs.append((frozen / best - 1.0) * 100.0)
    return {"shapes": len(regs), "mean_regret_pct": normalize_roundoff(sum(regs) / len(regs)),
            "max_regret_pct": normalize_roundoff(max(regs))}


def noise_floor(rows: list[dict], control: list[dict]) -> dict:
    """Two measurements of one configuration per (shape, path): the control
    rows repeat a candidate that the sweep also measured. Reported: the mean
    relative difference per path, and the regret that the repeated
    configuration shows against the faster of its two measurements (a policy
    can show this much regret from noise alone)."""
    per_path: dict[str, list[float]] = {}
    regs = []
    shapes = sorted({r["config_id"] for r in control})
    for cid in shapes:
        first = second = 0.0
        for phase in PHASES:
            c = next(r for r in control if r["config_id"] == cid and r["phase"] == phase)
            a = selected_time(rows, cid, phase, int(c["candidate_value"]))
            b = float(c["mean_ms"])
            per_path.setdefault(phase, []).append(abs(a - b) / a * 100.0)
            first += a
            second += min(a, b)
        regs.append((first / second - 1.0) * 100.0)
    return {
        "control_values": {ph: int(next(r for r in control if r["phase"] == ph)["candidate_value"])
                           for ph in PHASES},
        "shapes": len(shapes),
        "mean_abs_diff_pct": {ph: normalize_roundoff(sum(v) / len(v)) for ph, v in per_path.items()},
        "mean_regret_pct": normalize_roundoff(sum(regs) / len(regs)),
        "max_regret_pct": normalize_roundoff(max(regs)),
    }

