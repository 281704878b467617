"""Shape sets of the PathTile tuner on MI355X.

The reference tunes on hand-listed shapes (benchmark/benchmark_shape_sweep_
ampere.py:92-178: 20 "pathtile-train", 10 "pathtile-holdout"). This re-run
draws 30 distinct shapes with a fixed seed from the grid
B in {2048, 4096, 8192, 16384, 32768}, H in {64, 128, 256},
L in {16, 24, 32, 40, 48}, K in {3, 8, 16, 24, 32, 48}, and splits them by a
seeded permutation into 20 tuning and 10 held-out shapes.
"""

from __future__ import annotations

from dataclasses import asdict, dataclass

import numpy as np

GRID_B = (2048, 4096, 8192, 16384, 32768)
GRID_H = (64, 128, 256)
GRID_L = (16, 24, 32, 40, 48)
GRID_K = (3, 8, 16, 24, 32, 48)
SEED = 2026
N_TRAIN = 20
N_HOLDOUT = 10


@dataclass(frozen=True)
class ShapeCase:
    """One tuning shape (benchmark/benchmark_shape_sweep_ampere.py:61-75)."""

    config_id: str
    B: int
    H: int
    L: int
    K: int
    sweep_group: str

    def validate(self) -> None:
        if min(self.B, self.H, self.L, self.K) <= 0:
            raise ValueError(f"All dimensions must be positive: {self}")
        if self.L > 48 or self.K > 48:
            raise ValueError(f"{self.config_id}: kernels require L<=48 and K<=48")

    def as_dict(self) -> dict:
        return asdict(self)


def _case(B: int, H: int, L: int, K: int, group: str) -> ShapeCase:
    return ShapeCase(f"{group}_b{B}_h{H}_l{L}_k{K}", B, H, L, K, group)


def draw_shapes(seed: int = SEED, n_train: int = N_TRAIN,
                n_holdout: int = N_HOLDOUT) -> tuple[list[ShapeCase], list[ShapeCase]]:
    """30 distinct grid shapes from `seed`; the first 20 of a seeded
    permutation tune, the last 10 are held out."""
    grid = [(B, H, L, K) for B in GRID_B for H in GRID_H for L in GRID_L for K in GRID_K]
    rng = np.random.default_rng(seed)
    picks = rng.choice(len(grid), size=n_train + n_holdout, replace=False)
    order = rng.permutation(len(picks))
    chosen = [grid[int(picks[i])] for i in order]
    train = [_case(*s, "train") for s in chosen[:n_train]]
    holdout = [_case(*s, "holdout") for s in chosen[n_train:]]
    for c in train + holdout:
        c.validate()
    return train, holdout


# The BASELINE workloads, reported beside the tuned policy.
BASELINE_CASES = [
    _case(16384, 128, 48, 48, "primary"),
    _case(32768, 256, 48, 4, "short"),
    _case(16384, 128, 48, 47, "oddk"),
    _case(1000, 96, 37, 48, "edge"),
]
