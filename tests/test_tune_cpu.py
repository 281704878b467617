"""PathTile tuner arithmetic on hand-built tables (CPU only): the selection
rule and regret formulas of scripts/aggregate_pathtile_results.py:223-527."""

from __future__ import annotations

import pytest

from pathtile_amd.tune import select, shapes


def _row(cid, phase, value, ms, trial=1):
    return {"config_id": cid, "B": 1, "H": 1, "L": 8, "K": 3, "phase": phase,
            "candidate_value": value, "mean_ms": ms, "trial_id": trial}


def test_shape_draw_is_deterministic_and_on_grid():
    a_tr, a_ho = shapes.draw_shapes()
    b_tr, b_ho = shapes.draw_shapes()
    assert [c.config_id for c in a_tr + a_ho] == [c.config_id for c in b_tr + b_ho]
    assert len(a_tr) == 20 and len(a_ho) == 10
    dims = [(c.B, c.H, c.L, c.K) for c in a_tr + a_ho]
    assert len(set(dims)) == 30
    for B, H, L, K in dims:
        assert B in shapes.GRID_B and H in shapes.GRID_H
        assert L in shapes.GRID_L and K in shapes.GRID_K
    other = shapes.draw_shapes(seed=1)[0]
    assert [c.config_id for c in other] != [c.config_id for c in a_tr]


def test_select_sums_then_argmins_with_ties_to_smaller():
    rows = []
    # fwd: value 4 wins on total (1+1) vs 2 (0.5+2) ; dx: tie 2 vs 8 -> 2
    rows += [_row("s1", "fwd", 2, 0.5), _row("s2", "fwd", 2, 2.0),
             _row("s1", "fwd", 4, 1.0), _row("s2", "fwd", 4, 1.0)]
    rows += [_row("s1", "bwd_input", 8, 1.0), _row("s2", "bwd_input", 8, 1.0),
             _row("s1", "bwd_input", 2, 1.5), _row("s2", "bwd_input", 2, 0.5)]
    rows += [_row("s1", "bwd_weight", 128, 3.0), _row("s2", "bwd_weight", 128, 3.0),
             _row("s1", "bwd_weight", 256, 2.0)]  # 256 lacks s2 -> cannot compete
    pol = select.select_policy(rows)
    assert pol == {"fwd_waves_per_block": 4, "dx_waves_per_block": 2,
                   "dk_threads_per_block": 128}


def test_mean_of_trials():
    rows = [_row("s1", "fwd", 2, 1.0, 1), _row("s1", "fwd", 2, 3.0, 2)]
    m = select.mean_of_trials(rows)
    assert len(m) == 1 and m[0]["mean_ms"] == 2.0 and m[0]["trials"] == 2
    assert m[0]["between_trial_std_ms"] == pytest.approx(2 ** 0.5)


def test_regret_against_per_path_oracle():
    rows = []
    for cid, f, d, k in (("a", (1.0, 0.8), (1.0, 1.0), (2.0, 1.0)),
                         ("b", (1.0, 1.2), (1.0, 1.0), (2.0, 2.0))):
        rows += [_row(cid, "fwd", 2, f[0]), _row(cid, "fwd", 4, f[1]),
                 _row(cid, "bwd_input", 2, d[0]), _row(cid, "bwd_input", 4, d[1]),
                 _row(cid, "bwd_weight", 128, k[0]), _row(cid, "bwd_weight", 256, k[1])]
    policy = {"fwd_waves_per_block": 2, "dx_waves_per_block": 2, "dk_threads_per_block": 128}
    per, summ = select.holdout_regret(rows, policy)
    a = next(r for r in per if r["config_id"] == "a")
    b = next(r for r in per if r["config_id"] == "b")
    # a: frozen 1+1+2 = 4, oracle 0.8+1+1 = 2.8 ; b: frozen 4, oracle 1+1+2 = 4
    assert a["frozen_total_ms"] == pytest.approx(4.0)
    assert a["oracle_total_ms"] == pytest.approx(2.8)
    assert a["regret_pct"] == pytest.approx((4 / 2.8 - 1) * 100)
    assert b["regret_pct"] == 0.0 and b["exact_oracle_schedule"] in (True, False)
    assert summ["shapes"] == 2
    assert summ["mean_regret_pct"] == pytest.approx(((4 / 2.8 - 1) * 100) / 2)
    assert summ["runtime_weighted_regret_pct"] == pytest.approx((8 / 6.8 - 1) * 100)
    assert summ["shapes_within_1pct"] == 1


def test_missing_path_is_an_error():
    rows = [_row("a", "fwd", 2, 1.0), _row("a", "bwd_input", 2, 1.0)]
    with pytest.raises(RuntimeError, match="Missing path result"):
        select.combined_oracle(rows)


def test_frozen_policy_must_predate_holdout():
    pol = {"frozen_before_holdout": True, "frozen_at_utc": "2026-12-01T10:00:00+00:00"}
    select.verify_frozen_before_holdout(pol, ["2026-12-01T10:00:01+00:00"])
    with pytest.raises(AssertionError):
        select.verify_frozen_before_holdout(pol, ["2026-12-01T09:59:59+00:00"])
    with pytest.raises(AssertionError, match="marker"):
        select.verify_frozen_before_holdout({"frozen_at_utc": pol["frozen_at_utc"]}, [])


def test_normalize_roundoff_and_geomean():
    assert select.normalize_roundoff(1e-13) == 0.0
    assert select.normalize_roundoff(1e-3) == 1e-3
    assert select.geometric_mean([1.0, 4.0]) == pytest.approx(2.0)
    with pytest.raises(ValueError):
        select.geometric_mean([1.0, 0.0])
