"""PathTile tuner arithmetic on hand-built tables (CPU only): the selection
rule and regret formulas of scripts/aggregate_pathtile_results.py:223-527."""

from __future__ import annotations

import pytest

from pathtile_amd import rows_rule
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


# ---------------------------------------------------------------------------
# Selector baselines and the coverage budget (pathtile_amd/tune/baselines.py)
# ---------------------------------------------------------------------------
from pathtile_amd.tune import baselines  # noqa: E402


def _full(table):
    """rows from {phase: {cid: {value: ms}}}"""
    rows = []
    for ph, per in table.items():
        for cid, cand in per.items():
            for v, ms in cand.items():
                rows.append(_row(cid, ph, v, ms))
    return rows


def test_majority_winner_counts_shape_wins():
    """fwd: 2 wins s1, s2 and 4 wins s3 -> 2, although 4 has the smaller sum;
    dx: one win each for 1 and 8 -> the smaller value; dk: a tie within a
    shape goes to the smaller value (128 wins s1 and s2)."""
    t = {
        "fwd": {"s1": {2: 1.0, 4: 1.1}, "s2": {2: 1.0, 4: 1.2}, "s3": {2: 9.0, 4: 1.0}},
        "bwd_input": {"s1": {1: 1.0, 8: 2.0}, "s2": {1: 2.0, 8: 1.0}, "s3": {1: 1.0, 8: 1.0}},
        "bwd_weight": {"s1": {128: 1.0, 256: 1.0}, "s2": {128: 1.0, 256: 1.0}, "s3": {128: 2.0, 256: 1.0}},
    }
    rows = _full(t)
    pol = baselines.majority_winner_policy(rows)
    assert pol == {"fwd_waves_per_block": 2, "dx_waves_per_block": 1, "dk_threads_per_block": 128}
    assert select.select_policy(rows)["fwd_waves_per_block"] == 4


def test_global_static_raw_sum_is_the_per_path_choice_and_geomean_can_differ():
    """Summed latency separates over the paths, so its best combination is
    select_policy's; the geometric-mean regret weighs shapes equally and can
    prefer another value (here fwd 2: 10% worse on the big shape s1, a third
    faster on the small shape s2)."""
    t = {
        "fwd": {"s1": {2: 11.0, 4: 10.0}, "s2": {2: 0.1, 4: 0.15}},
        "bwd_input": {"s1": {1: 0.01, 2: 0.02}, "s2": {1: 0.01, 2: 0.02}},
        "bwd_weight": {"s1": {64: 0.01}, "s2": {64: 0.01}},
    }
    rows = _full(t)
    table = baselines.global_static_table(rows)
    assert len(table) == 2 * 2 * 1
    raw = baselines.best_by(table, "raw_total_ms")
    assert raw == select.select_policy(rows)
    assert raw["fwd_waves_per_block"] == 4
    assert baselines.best_by(table, "geomean_regret_pct")["fwd_waves_per_block"] == 2
    r = next(x for x in table if x["fwd_waves_per_block"] == 4 and x["dx_waves_per_block"] == 1)
    # s1 is at its oracle (10.02); s2 takes 0.17 against 0.12
    assert r["max_regret_pct"] == pytest.approx((0.17 / 0.12 - 1) * 100)
    assert r["mean_regret_pct"] == pytest.approx((0.17 / 0.12 - 1) * 50)
    assert r["geomean_regret_pct"] == pytest.approx(((0.17 / 0.12) ** 0.5 - 1) * 100)


def test_coverage_queries_on_a_line():
    """Shapes that differ only in B = 2, 4, 8, 16, 32: the most work first
    (B = 32), then the farthest (B = 2), then the middle (B = 8), then of the
    two equidistant gaps the lower index (B = 4)."""
    dims = [(b, 64, 16, 8) for b in (2, 4, 8, 16, 32)]
    assert baselines.coverage_queries(dims, 4) == [4, 0, 2, 1]
    assert baselines.coverage_queries(dims, 5) == [4, 0, 2, 1, 3]
    with pytest.raises(ValueError):
        baselines.coverage_queries(dims, 1)


def test_coverage_queries_standardise_each_dimension():
    """Without standardisation B (range 2^4) would dominate L (range 2^1.6);
    standardised, each spans the same distance, so after the largest-work
    shape the farthest pick is the corner opposite in both."""
    dims = [(32768, 64, 48, 8), (2048, 64, 48, 8), (32768, 64, 16, 8), (2048, 64, 16, 8)]
    assert baselines.useful_products(*dims[0]) == max(baselines.useful_products(*d) for d in dims)
    assert baselines.coverage_queries(dims, 2) == [0, 3]


def test_useful_products_matches_the_path_count():
    from pathtile_amd import runtime

    for B, H, L, K in ((3, 5, 48, 48), (2, 7, 16, 3), (1, 1, 1, 1), (4, 2, 9, 40)):
        assert 2 * baselines.useful_products(B, H, L, K) == runtime.useful_flops(B, H, L, K)


def test_baselines_on_the_committed_tuner_results():
    """On the committed MI355X trial CSVs: the summed-latency baseline is the
    frozen policy, every budget's coverage policy is a valid candidate
    combination, and the full budget gives the frozen policy."""
    import json
    from pathlib import Path

    from pathtile_amd.tune.__main__ import _read_csv

    res = Path(__file__).resolve().parents[1] / "pathtile_amd" / "tune" / "results"
    train = select.mean_of_trials(sum((_read_csv(p) for p in sorted(res.glob("train_trial*.csv"))), []))
    hold = select.mean_of_trials(sum((_read_csv(p) for p in sorted(res.glob("holdout_trial*.csv"))), []))
    frozen = json.loads((res / "frozen_policy.json").read_text())["selected"]
    out = baselines.evaluate(train, hold, frozen, 6)
    assert out["policies"]["global_static_raw_sum"]["policy"] == frozen
    assert len(out["coverage_shapes"]) == 6
    assert out["coverage_budget_sweep"][-1]["policy"] == frozen
    for name, r in out["policies"].items():
        assert r["holdout"]["shapes"] == 10 and r["train"]["shapes"] == 20, name


def _shape_rows(cid, H, L, K, times):
    """times: {phase: {value: ms}} for one shape."""
    out = []
    for phase, by_value in times.items():
        for v, ms in by_value.items():
            out.append({"config_id": cid, "B": 64, "H": H, "L": L, "K": K, "phase": phase,
                        "candidate_value": v, "mean_ms": ms})
    return out


def test_fwd_dx_knob_inert_follows_the_library_rule():
    # matrix cores: H % 8 == 0 and the library's thresholds
    assert select.fwd_dx_knob_inert(128, 48, 48, 16384)       # P
    assert select.fwd_dx_knob_inert(128, 48, 47, 16384)       # E2
    assert not select.fwd_dx_knob_inert(256, 48, 4, 32768)    # S: short chain, VALU kernel
    assert select.fwd_dx_knob_inert(96, 37, 48, 1000)         # E1: L % 4 != 0 is served too
    assert not select.fwd_dx_knob_inert(96, 37, 8, 1000)      # short chain, small call: VALU
    assert select.fwd_dx_knob_inert(96, 37, 8, 4096)          # L % 4 != 0 from 2^18 rows: matrix cores
    assert not select.fwd_dx_knob_inert(12, 48, 48, 16384)    # H % 8 != 0
    # rows of L % 4 == 0 from 16 to 48 columns: the matrix cores from a K
    # that depends on L, on calls of fewer than 2^17 rows (B * H) and, at
    # L = 48, on the load regime and H
    assert select.fwd_dx_knob_inert(128, 24, 9, 16384)        # L24 from K = 9
    assert not select.fwd_dx_knob_inert(128, 24, 8, 16384)
    assert select.fwd_dx_knob_inert(256, 24, 16, 32768)       # above 256 MiB too
    assert not select.fwd_dx_knob_inert(96, 24, 16, 1024)     # 98304 rows: from K = 17
    assert select.fwd_dx_knob_inert(96, 24, 17, 1024)
    assert select.fwd_dx_knob_inert(128, 16, 5, 16384)        # L16 from K = 5
    assert not select.fwd_dx_knob_inert(128, 16, 4, 16384)
    assert not select.fwd_dx_knob_inert(128, 40, 16, 16384)   # L40 from K = 17
    assert select.fwd_dx_knob_inert(128, 40, 17, 16384)
    assert not select.fwd_dx_knob_inert(64, 40, 24, 2000)     # 128000 rows: from K = 25
    assert select.fwd_dx_knob_inert(64, 40, 25, 2000)
    assert select.fwd_dx_knob_inert(128, 48, 9, 8192)         # L48, 201 MB, H <= 128: K >= 9
    assert not select.fwd_dx_knob_inert(128, 48, 16, 16384)   # above 256 MiB: K >= 17
    assert not select.fwd_dx_knob_inert(256, 48, 16, 4096)    # H > 128: K >= 17
    assert select.fwd_dx_knob_inert(256, 48, 17, 4096)
    # rows of fewer than 16 columns: >= 10.5 (16 / L)^2 useful FMAs per
    # output, with the useful count against brute force
    L, K = 12, 24
    useful = sum(1 for t in range(L) for j in range(K) if 0 <= t + j - K // 2 < L)
    assert rows_rule.useful_fma_per_row(L, K) == useful
    assert select.fwd_dx_knob_inert(64, L, K, 2048) == (2 * useful * L >= 21 * 16 * 16)
    L, K = 40, 32
    useful = sum(1 for t in range(L) for j in range(K) if 0 <= t + j - K // 2 < L)
    assert rows_rule.useful_fma_per_row(L, K) == useful


def test_per_path_and_active_knob_regret():
    pol = {"fwd_waves_per_block": 2, "dx_waves_per_block": 2, "dk_threads_per_block": 128}
    rows = []
    # shape a: FWD/dX knob inert (P-like); fwd candidate 4 is 10% faster by noise
    rows += _shape_rows("a", 128, 48, 48, {"fwd": {2: 1.1, 4: 1.0}, "bwd_input": {2: 1.0, 4: 1.0},
                                           "bwd_weight": {128: 2.0, 256: 2.0}})
    # shape b: VALU shapes (knob active); dk candidate 256 is 25% faster
    rows += _shape_rows("b", 256, 48, 4, {"fwd": {2: 1.0, 4: 1.5}, "bwd_input": {2: 1.0, 4: 1.0},
                                          "bwd_weight": {128: 2.5, 256: 2.0}})
    per = select.path_regret(rows, pol)
    assert per["fwd"]["sum_regret_pct"] == pytest.approx((2.1 / 2.0 - 1) * 100)
    assert per["fwd"]["mean_regret_pct"] == pytest.approx(5.0)
    assert per["fwd"]["shapes_knob_inert"] == 1 and "shapes_knob_inert" not in per["bwd_weight"]
    assert per["bwd_weight"]["max_regret_pct"] == pytest.approx(25.0)
    _, total = select.holdout_regret(rows, pol)
    act = select.active_knob_regret(rows, pol)
    # a: the inert FWD noise no longer counts -> 0; b: 4.5 / 4.0 -> 12.5%
    assert act["mean_regret_pct"] == pytest.approx(6.25)
    assert total["mean_regret_pct"] == pytest.approx(((4.1 / 4.0 - 1) + (4.5 / 4.0 - 1)) * 50)


def test_noise_floor_from_the_duplicate_control():
    rows = _shape_rows("a", 128, 48, 48, {"fwd": {2: 1.0}, "bwd_input": {2: 1.0},
                                          "bwd_weight": {128: 2.0}})
    rows += _shape_rows("b", 128, 48, 48, {"fwd": {2: 1.0}, "bwd_input": {2: 1.0},
                                           "bwd_weight": {128: 2.0}})
    ctrl = _shape_rows("a", 128, 48, 48, {"fwd": {2: 0.9}, "bwd_input": {2: 1.1},
                                          "bwd_weight": {128: 2.0}})
    ctrl += _shape_rows("b", 128, 48, 48, {"fwd": {2: 1.0}, "bwd_input": {2: 1.0},
                                           "bwd_weight": {128: 2.2}})
    nf = select.noise_floor(rows, ctrl)
    assert nf["control_values"] == {"fwd": 2, "bwd_input": 2, "bwd_weight": 128}
    assert nf["mean_abs_diff_pct"]["fwd"] == pytest.approx(5.0)
    assert nf["mean_abs_diff_pct"]["bwd_weight"] == pytest.approx(5.0)
    # a: 4.0 against 3.9 (the faster of each pair); b: 4.0 against 4.0
    assert nf["mean_regret_pct"] == pytest.approx((4.0 / 3.9 - 1) * 50)
    assert nf["max_regret_pct"] == pytest.approx((4.0 / 3.9 - 1) * 100)


def test_timed_check_references_and_verdicts():
    """The sweep's check of the timed outputs (sweep.TimedCheck): its FP64
    references equal the oracle's (FWD and dX on the sampled rows, which
    include the first and last sample; dK over the whole batch), correct
    outputs pass the build's bars, and NaN (an unwritten tile) or a
    perturbed output fail them."""
    import numpy as np
    import torch

    import oracle
    from pathtile_amd.tune import sweep
    from pathtile_amd.tune.shapes import ShapeCase

    B, H, L, K = 70, 6, 13, 5
    case = ShapeCase("t", B, H, L, K, "t")
    x, w, dy = oracle.make_inputs(B, H, L, K, 3)
    tc = sweep.TimedCheck(case, 1, x, w, dy)
    idx = tc.idx.numpy()
    assert idx[0] == 0 and idx[-1] == B - 1 and len(set(idx)) == min(B, sweep.TIMED_CHECK_ROWS)
    assert np.abs(tc.y.numpy() - oracle.fwd_f64(x[idx], w)).max() < 1e-12
    assert np.abs(tc.gx.numpy() - oracle.dx_f64(dy[idx], w)).max() < 1e-12
    assert np.abs(tc.gk.numpy() - oracle.dk_f64(dy, x, K)).max() < 1e-9
    good = {"fwd": torch.from_numpy(oracle.fwd_f64(x, w)).float(),
            "bwd_input": torch.from_numpy(oracle.dx_f64(dy, w)).float(),
            "bwd_weight": torch.from_numpy(oracle.dk_f64(dy, x, K)).float()}
    rows = tc.rows("waves_per_block", 4, {k: good[k] for k in ("fwd", "bwd_input")})
    rows += tc.rows("dk_threads_per_block", 128, {"bwd_weight": good["bwd_weight"]})
    assert [r["phase"] for r in rows] == ["fwd", "bwd_input", "bwd_weight"]
    assert all(r["allclose"] and r["validation_B"] == B for r in rows)
    bad_y = good["fwd"].clone()
    bad_y[B - 1, 0, 0] = float("nan")   # the last sample: a tile the launch missed
    bad_k = good["bwd_weight"] * (1 + 1e-3)
    rows = tc.rows("waves_per_block", 4, {"fwd": bad_y, "bwd_input": good["bwd_input"]})
    rows += tc.rows("dk_threads_per_block", 128, {"bwd_weight": bad_k})
    assert [r["allclose"] for r in rows] == [False, True, False]
