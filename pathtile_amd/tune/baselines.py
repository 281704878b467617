"""Selector baselines and the shape-coverage budget of the PathTile tuner
(CPU only, from the tuning/held-out trial CSVs; no device).

Restates, on plain row dicts:

* the majority-winner policy: per path, the candidate that is fastest on the
  most tuning shapes (each shape's winner by mean_ms, ties to the smaller
  value; the count's ties to the smaller value)
  (``scripts/evaluate_selector_baselines.py:261-307``);
* the global-static table: every (FWD, dX, dK) combination scored over the
  tuning shapes by raw summed latency and by mean, geometric-mean and max
  regret against the per-shape oracle total
  (``scripts/check_global_static_objective.py:56-123``; one GPU here, so
  nothing is pooled across devices);
* the coverage-budget policy: ``budget`` tuning shapes chosen from metadata
  alone (largest useful work first, then repeatedly the shape farthest from
  those chosen in standardised log2(B, H, L, K)), then per path the candidate
  minimising the latency summed over those shapes
  (``scripts/compare_pathtile_shape_coverage.py:35-64``,
  ``scripts/freeze_pathtile_coverage_policy.py:27``, budget 6).

Every policy is then scored on the held-out shapes with the same regret
arithmetic as the frozen policy (``select.holdout_regret``).
"""

from __future__ import annotations

import itertools
import math

from . import select
from .select import PHASES, POLICY_KEYS


def useful_products(B: int, H: int, L: int, K: int) -> int:
    """Non-padding multiply-adds of one path
    (``scripts/prototype_pathtile_shape_queries.py:62-68``)."""
    terms = 0
    for j in range(K):
        s = j - K // 2
        terms += max(0, min(L, L - s) - max(0, -s))
    return B * H * terms


def _shapes(rows: list[dict]) -> list[str]:
    return sorted({r["config_id"] for r in rows})


def _table(rows: list[dict], phase: str) -> dict[str, dict[int, float]]:
    """config_id -> {candidate value -> mean_ms} for one path."""
    out: dict[str, dict[int, float]] = {}
    for r in rows:
        if r["phase"] == phase:
            out.setdefault(r["config_id"], {})[int(r["candidate_value"])] = float(r["mean_ms"])
    return out


def majority_winner_policy(training: list[dict]) -> dict[str, int]:
    policy = {}
    for phase, name in POLICY_KEYS.items():
        wins: dict[int, int] = {}
        for cid, cand in sorted(_table(training, phase).items()):
            best = min(cand.items(), key=lambda kv: (kv[1], kv[0]))[0]
            wins[best] = wins.get(best, 0) + 1
        if not wins:
            raise ValueError(f"No training candidates for {phase}")
        policy[name] = min(wins.items(), key=lambda kv: (-kv[1], kv[0]))[0]
    return policy


def global_static_table(training: list[dict]) -> list[dict]:
    """Every (FWD, dX, dK) combination measured on every tuning shape, scored
    against the per-shape oracle total."""
    tables = {ph: _table(training, ph) for ph in PHASES}
    shapes = _shapes(training)
    values = {ph: sorted(set.intersection(*(set(tables[ph][c]) for c in shapes))) for ph in PHASES}
    oracle_total = {c: sum(min(tables[ph][c].values()) for ph in PHASES) for c in shapes}
    out = []
    for combo in itertools.product(*(values[ph] for ph in PHASES)):
        ratios, raw = [], 0.0
        for c in shapes:
            t = sum(tables[ph][c][v] for ph, v in zip(PHASES, combo))
            raw += t
            ratios.append(t / oracle_total[c])
        regrets = [(r - 1.0) * 100.0 for r in ratios]
        out.append({
            POLICY_KEYS[PHASES[0]]: combo[0],
            POLICY_KEYS[PHASES[1]]: combo[1],
            POLICY_KEYS[PHASES[2]]: combo[2],
            "raw_total_ms": raw,
            "mean_regret_pct": sum(regrets) / len(regrets),
            "geomean_regret_pct": (math.exp(sum(math.log(r) for r in ratios) / len(ratios)) - 1.0) * 100.0,
            "max_regret_pct": max(regrets),
        })
    return out


def best_by(table: list[dict], key: str) -> dict[str, int]:
    """The combination minimising `key`; ties to the smaller (FWD, dX, dK)."""
    names = [POLICY_KEYS[ph] for ph in PHASES]
    row = min(table, key=lambda r: (r[key], *(r[n] for n in names)))
    return {n: row[n] for n in names}


def coverage_queries(dims: list[tuple[int, int, int, int]], budget: int) -> list[int]:
    """Indices of `budget` shapes: the one with the most useful work first,
    then repeatedly the shape whose nearest chosen shape is farthest, in
    log2(B, H, L, K) standardised per dimension (population std; a constant
    dimension keeps scale 1); ties go to the lower index."""
    n = len(dims)
    if not 2 <= budget <= n:
        raise ValueError("Invalid shape budget")
    geo = [[math.log2(v) for v in d] for d in dims]
    cols = list(zip(*geo))
    mean = [sum(c) / n for c in cols]
    std = [math.sqrt(sum((v - m) ** 2 for v in c) / n) for c, m in zip(cols, mean)]
    std = [s if s >= 1e-12 else 1.0 for s in std]
    z = [[(v - m) / s for v, m, s in zip(row, mean, std)] for row in geo]
    work = [useful_products(*d) for d in dims]
    picked = [max(range(n), key=lambda i: (work[i], -i))]
    while len(picked) < budget:
        def nearest(i):
            return min(sum((a - b) ** 2 for a, b in zip(z[i], z[j])) for j in picked)
        rest = [i for i in range(n) if i not in picked]
        picked.append(max(rest, key=lambda i: (nearest(i), -i)))
    return picked


def coverage_policy(training: list[dict], budget: int = 6) -> tuple[list[str], dict[str, int]]:
    """The coverage-selected tuning shapes and, per path, the candidate with
    the least latency summed over them (ties to the smaller value)."""
    shapes = _shapes(training)
    dims = []
    for c in shapes:
        r = next(r for r in training if r["config_id"] == c)
        dims.append((int(r["B"]), int(r["H"]), int(r["L"]), int(r["K"])))
    chosen = [shapes[i] for i in coverage_queries(dims, budget)]
    subset = [r for r in training if r["config_id"] in set(chosen)]
    return chosen, select.select_policy(subset)


def evaluate(training: list[dict], holdout: list[dict], frozen: dict[str, int],
             budget: int = 6) -> dict:
    """Held-out (and tuning-shape) regret of the frozen policy and of each
    baseline policy."""
    table = global_static_table(training)
    chosen, cov = coverage_policy(training, budget)
    policies = {
        "frozen_sum_latency": frozen,
        "majority_winner": majority_winner_policy(training),
        "global_static_raw_sum": best_by(table, "raw_total_ms"),
        "global_static_geomean_regret": best_by(table, "geomean_regret_pct"),
        f"coverage_{budget}_shapes": cov,
    }
    out = {"coverage_shapes": chosen, "policies": {}}
    for name, pol in policies.items():
        _, tr = select.holdout_regret(training, pol)
        _, ho = select.holdout_regret(holdout, pol)
        out["policies"][name] = {"policy": pol, "train": tr, "holdout": ho}
    out["global_static_top5_by_raw_sum"] = sorted(
        table, key=lambda r: (r["raw_total_ms"],))[:5]
    # How the held-out regret depends on the tuning budget (the tuning cost
    # grows with the number of measured shapes).
    sweep = []
    for b in range(2, len(_shapes(training)) + 1):
        shapes_b, pol_b = coverage_policy(training, b)
        _, ho = select.holdout_regret(holdout, pol_b)
        sweep.append({"budget": b, "policy": pol_b,
                      "holdout_mean_regret_pct": ho["mean_regret_pct"],
                      "holdout_max_regret_pct": ho["max_regret_pct"]})
    out["coverage_budget_sweep"] = sweep
    return out
