"""CLI of the PathTile tuner.

    python -m pathtile_amd.tune all    [--trials 3 --warmup 50 --runs 100]
        GPU: tuning trials -> freeze the per-path policy -> held-out trials
        -> regret report; with --install the policy becomes the runtime's
        launch default (pathtile_amd/tune/frozen_policy.json).
    python -m pathtile_amd.tune report [--out DIR]
        CPU: recompute the policy from the tuning CSVs, verify it matches the
        frozen one and predates every held-out trial, rewrite the report.
    python -m pathtile_amd.tune baselines [--out DIR] [--budget 6]
        CPU: score the selector baselines (majority winner, global static,
        a coverage-selected shape budget) beside the frozen policy on the
        same CSVs; writes DIR/baselines.json.
"""

from __future__ import annotations

import argparse
import csv
import json
import subprocess
import sys
from pathlib import Path

from . import baselines, select
from .shapes import SEED, draw_shapes

PKG = Path(__file__).resolve().parent
DEFAULT_OUT = PKG / "results"
INSTALLED_POLICY = PKG / "frozen_policy.json"


def _write_csv(path: Path, rows: list[dict]) -> None:
    if not rows:
        path.write_text("")
        return
    keys = list(rows[0].keys())
    for r in rows[1:]:
        for k in r:
            if k not in keys:
                keys.append(k)
    with path.open("w", newline="") as f:
        w = csv.DictWriter(f, fieldnames=keys)
        w.writeheader()
        w.writerows(rows)


def _read_csv(path: Path) -> list[dict]:
    with path.open() as f:
        rows = list(csv.DictReader(f))
    for r in rows:
        for k in ("B", "H", "L", "K", "candidate_value", "trial_id", "n"):
            if k in r and r[k] != "":
                r[k] = int(float(r[k]))
        for k in ("mean_ms",):
            if k in r:
                r[k] = float(r[k])
    return rows


def _git_rev() -> str:
    """The checkout's HEAD; where the tree was copied without its .git (a
    GPU box), the PATHTILE_GIT_REV the caller passes along."""
    import os

    try:
        return subprocess.run(["git", "rev-parse", "HEAD"], cwd=PKG, capture_output=True,
                              text=True, check=True).stdout.strip()
    except Exception:
        return os.environ.get("PATHTILE_GIT_REV", "unknown")


def _run_phase(name, cases, args, out: Path, log) -> list[dict]:
    from .sweep import run_trial

    rows, validation, metas = [], [], []
    for trial in range(1, args.trials + 1):
        res = run_trial(cases, trial, args.warmup, args.runs, args.seed, log=log)
        _write_csv(out / f"{name}_trial{trial}.csv", res["summary"])
        _write_csv(out / f"{name}_control_trial{trial}.csv", res["control"])
        rows += res["summary"]
        validation += res["validation"]
        metas.append(res["metadata"])
    _write_csv(out / f"{name}_validation.csv", validation)
    (out / f"{name}_metadata.json").write_text(json.dumps(metas, indent=2))
    return rows


def _phase_rows(out: Path, name: str) -> tuple[list[dict], list[dict]]:
    rows = sum((_read_csv(p) for p in sorted(out.glob(f"{name}_trial*.csv"))), [])
    ctrl = sum((_read_csv(p) for p in sorted(out.glob(f"{name}_control_trial*.csv"))), [])
    return select.mean_of_trials(rows), select.mean_of_trials(ctrl)


def build_report(out: Path, policy: dict) -> dict:
    """Regret tables from the CSVs in `out` (no device needed): the
    reference's summary per phase, per-path regret, the (shape, path) pairs
    where the FWD/dX knob cannot change the kernel, the regret over the
    knobs that can, and the noise floor from the duplicate control."""
    train, train_ctrl = _phase_rows(out, "train")
    hold, hold_ctrl = _phase_rows(out, "holdout")
    recomputed = select.select_policy(train)
    if recomputed != policy["selected"]:
        raise AssertionError(f"frozen policy {policy['selected']} != training-only reconstruction {recomputed}")
    metas = json.loads((out / "holdout_metadata.json").read_text())
    select.verify_frozen_before_holdout(policy, [m["created_at_utc"] for m in metas])
    report = {"policy": recomputed, "device_name": policy.get("device_name"),
              "knob_inert_rule": select.KNOB_INERT_RULE}
    for name, rows, ctrl in (("train", train, train_ctrl), ("holdout", hold, hold_ctrl)):
        per, summary = select.holdout_regret(rows, recomputed)
        for r in per:
            r["fwd_dx_knob_inert"] = select.fwd_dx_knob_inert(r["H"], r["L"], r["K"], r["B"])
        _write_csv(out / f"{name}_per_shape.csv", per)
        summary["per_path"] = select.path_regret(rows, recomputed)
        summary["knob_active_paths"] = select.active_knob_regret(rows, recomputed)
        if ctrl:
            summary["noise_floor"] = select.noise_floor(rows, ctrl)
        report[name] = summary
    (out / "report.json").write_text(json.dumps(report, indent=2))
    return report


def main(argv=None) -> int:
    p = argparse.ArgumentParser(prog="python -m pathtile_amd.tune")
    p.add_argument("command", choices=["all", "report", "baselines"])
    p.add_argument("--budget", type=int, default=6,
                   help="tuning shapes of the coverage-budget baseline")
    p.add_argument("--out", type=Path, default=DEFAULT_OUT)
    p.add_argument("--trials", type=int, default=3)
    p.add_argument("--warmup", type=int, default=50)
    p.add_argument("--runs", type=int, default=100)
    p.add_argument("--seed", type=int, default=0, help="base input seed (shapes use a fixed seed)")
    p.add_argument("--install", action="store_true",
                   help="write the frozen policy to pathtile_amd/tune/frozen_policy.json")
    args = p.parse_args(argv)
    out = args.out
    out.mkdir(parents=True, exist_ok=True)

    def log(msg):
        print(msg, flush=True)

    if args.command == "all":
        if args.trials < 1 or args.warmup < 1 or args.runs < 2:
            raise SystemExit("Use at least one trial, one warm-up and two measured runs")
        import torch

        train_cases, holdout_cases = draw_shapes()
        log(f"[tune] {len(train_cases)} tuning shapes, {len(holdout_cases)} held out (shape seed {SEED})")
        train_rows = _run_phase("train", train_cases, args, out, log)
        selected = select.select_policy(select.mean_of_trials(train_rows))
        policy = {
            "selected": selected,
            "frozen_before_holdout": True,
            "frozen_at_utc": __import__("datetime").datetime.now(
                __import__("datetime").timezone.utc).isoformat(),
            "device_name": torch.cuda.get_device_name(0),
            "git_rev": _git_rev(),
            "shape_seed": SEED,
            "train_shapes": [c.config_id for c in train_cases],
            "holdout_shapes": [c.config_id for c in holdout_cases],
            "objective": "per path: argmin over candidates of the sum of mean kernel ms over the "
                         "tuning shapes; ties to the smaller value",
            "protocol": {"trials": args.trials, "warmup": args.warmup, "runs": args.runs},
        }
        (out / "frozen_policy.json").write_text(json.dumps(policy, indent=2))
        log(f"[tune] frozen policy {selected}")
        _run_phase("holdout", holdout_cases, args, out, log)
        report = build_report(out, policy)
        log(json.dumps(report, indent=2))
        if args.install:
            INSTALLED_POLICY.write_text(json.dumps(policy, indent=2))
        return 0

    policy = json.loads((out / "frozen_policy.json").read_text())
    if args.command == "baselines":
        train = select.mean_of_trials(sum((_read_csv(q) for q in sorted(out.glob("train_trial*.csv"))), []))
        hold = select.mean_of_trials(sum((_read_csv(q) for q in sorted(out.glob("holdout_trial*.csv"))), []))
        result = baselines.evaluate(train, hold, policy["selected"], args.budget)
        (out / "baselines.json").write_text(json.dumps(result, indent=2))
        for name, r in result["policies"].items():
            print(f"{name:32s} {r['policy']}  held-out mean regret {r['holdout']['mean_regret_pct']:.3f}%  "
                  f"tuning {r['train']['mean_regret_pct']:.3f}%")
        return 0
    report = build_report(out, policy)
    print(json.dumps(report, indent=2))
    return 0


if __name__ == "__main__":
    sys.exit(main())
