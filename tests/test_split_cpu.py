"""The three-way BF16 split behind the long-row matrix-core kernels, checked
on the CPU (no GPU): each FP32 value v becomes hi = bf16(v),
mid = bf16(v - hi), lo = bf16(v - hi - mid) (round to nearest even), and the
kernels keep six of the nine part products of x w. These tests pin the
bounds the kernels rely on, over values with random mantissas and exponents:

* v - hi and v - hi - mid are exact in FP32;
* |mid| <= 2^-8 |v|, |lo| <= 2^-16 |v|, |v - hi - mid - lo| <= 2^-24 |v|;
* the six kept products differ from x w by at most 2^-22 |x w|.

The BF16 rounding is restated here from its definition (keep the top 16
bits of the FP32 pattern, ties to even), independently of the HIP code.
"""

from __future__ import annotations

import numpy as np


def bf16_rne(v: np.ndarray) -> np.ndarray:
    """FP32 -> nearest BF16 (ties to even), returned as FP32."""
    b = v.astype(np.float32).view(np.uint32).astype(np.uint64)
    r = (b + 0x7FFF + ((b >> 16) & 1)) >> 16 << 16
    return r.astype(np.uint32).view(np.float32)


def split3(v: np.ndarray):
    v = v.astype(np.float32)
    hi = bf16_rne(v)
    r1 = (v - hi).astype(np.float32)
    mid = bf16_rne(r1)
    r2 = (r1 - mid).astype(np.float32)
    lo = bf16_rne(r2)
    return hi, mid, lo, r1, r2


def _values(n: int, seed: int, emin: int = -60, emax: int = 60) -> np.ndarray:
    g = np.random.default_rng(seed)
    m = g.uniform(1.0, 2.0, n) * g.choice([-1.0, 1.0], n)
    return (m * np.exp2(g.integers(emin, emax + 1, n))).astype(np.float32)


def test_bf16_rounding_is_nearest_even():
    # exact BF16 values stay, halfway cases go to the even neighbour
    v = np.array([1.0, 1.0 + 2.0 ** -7, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8,
                  1.0 + 2.0 ** -8 + 2.0 ** -20, -1.5], dtype=np.float32)
    want = np.array([1.0, 1.0 + 2.0 ** -7, 1.0, 1.0 + 2.0 ** -6,
                     1.0 + 2.0 ** -7, -1.5], dtype=np.float32)
    assert np.array_equal(bf16_rne(v), want)


def test_split_parts_and_residual_bounds():
    v = _values(200_000, 1)
    hi, mid, lo, r1, r2 = split3(v)
    v64 = v.astype(np.float64)
    # both differences are exact in FP32
    assert np.array_equal(r1.astype(np.float64), v64 - hi.astype(np.float64))
    assert np.array_equal(r2.astype(np.float64), r1.astype(np.float64) - mid.astype(np.float64))
    a = np.abs(v64)
    assert np.all(np.abs(mid.astype(np.float64)) <= 2.0 ** -8 * a)
    assert np.all(np.abs(lo.astype(np.float64)) <= 2.0 ** -16 * a)
    res = v64 - hi.astype(np.float64) - mid.astype(np.float64) - lo.astype(np.float64)
    assert np.all(np.abs(res) <= 2.0 ** -24 * a)


def test_six_part_products_bound():
    x, w = _values(200_000, 2, -40, 40), _values(200_000, 3, -40, 40)
    xh, xm, xl, _, _ = (p.astype(np.float64) for p in split3(x))
    wh, wm, wl, _, _ = (p.astype(np.float64) for p in split3(w))
    six = xh * wh + xh * wm + xm * wh + xm * wm + xh * wl + xl * wh
    exact = x.astype(np.float64) * w.astype(np.float64)
    assert np.all(np.abs(six - exact) <= 2.0 ** -22 * np.abs(exact))
    # every kept product of two 8-bit parts is exact in FP32
    for a, b in ((xh, wh), (xh, wm), (xm, wh), (xm, wm), (xh, wl), (xl, wh)):
        p = a * b
        assert np.array_equal(p.astype(np.float32).astype(np.float64), p)


def test_dropping_a_kept_product_breaks_the_bound():
    """The bound is tight enough to notice a missing mid*mid term (2^-16)."""
    x, w = _values(50_000, 4, -10, 10), _values(50_000, 5, -10, 10)
    xh, xm, xl, _, _ = (p.astype(np.float64) for p in split3(x))
    wh, wm, wl, _, _ = (p.astype(np.float64) for p in split3(w))
    five = xh * wh + xh * wm + xm * wh + xh * wl + xl * wh
    exact = x.astype(np.float64) * w.astype(np.float64)
    assert np.any(np.abs(five - exact) > 2.0 ** -22 * np.abs(exact))
