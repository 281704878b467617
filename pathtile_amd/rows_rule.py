"""Which FWD/dX kernel the library runs for a 16-byte aligned call, as a
host-side predicate (the rule itself is rows_algo in csrc/dwconv1d_abi.hip;
this restates it for the bench's kernel names, the tuner's knob-inert flag
and the tests that pick their tolerance by kernel).

The channel-group matrix-core kernel serves when H % 8 == 0 and:
  * L % 4 == 0, 16 <= L <= 48: from the K of mfma_min_k (by L, with
    separate thresholds for calls of fewer than 2^17 rows B * H and, at
    L = 48, for tensors above 256 MiB or H > 128);
  * L % 4 == 0, L < 16: at least 10.5 (LMAX / L)^2 useful FMAs per output;
  * L % 4 != 0: every call of at least 2^18 rows (B * H), smaller ones from
    5 (LMAX / L)^2 useful FMAs per output;
with LMAX = 16 ceil(L / 16). The VALU kernels serve every other call.
"""

from __future__ import annotations

PLAIN_LOAD_BYTES = 256 * 2**20
ODD_MFMA_ROWS = 1 << 18
SMALL_CALL_ROWS = 1 << 17


def useful_fma_per_row(L: int, K: int) -> int:
    """Multiply-adds of one row that touch a real element (zero padding,
    p = K // 2)."""
    p = K // 2
    return sum(max(0, min(L, L - (j - p)) - max(0, p - j)) for j in range(K))


def plain_loads(B: int, H: int, L: int) -> bool:
    """FP32 FWD/dX input loads are plain (cached) up to 256 MiB."""
    return 4 * B * H * L <= PLAIN_LOAD_BYTES


def mfma_min_k(L: int, H: int, rows: int, plain: bool) -> int:
    """Smallest K from which the matrix cores serve rows of L % 4 == 0,
    16 <= L <= 48 columns (rows = B * H; plain: at most 256 MiB)."""
    small = rows < SMALL_CALL_ROWS
    if L == 16:
        return 12 if small else 5
    if L == 20:
        return 16 if small else 9
    if L == 24:
        return 17 if small else 9
    if L in (28, 32):
        return 13 if small else 9
    if L == 36:
        return 17
    if L == 40:
        return 25 if small else 17
    if L == 44:
        return 17 if small else 9
    return 17 if small or not plain or H > 128 else 9


def matrix_cores_serve(B: int, H: int, L: int, K: int) -> bool:
    """The library's default FWD/dX kernel choice for 16-byte aligned
    tensors (PATHTILE_ROWS_ALGO unset)."""
    B, H, L, K = int(B), int(H), int(L), int(K)
    if H % 8:
        return False
    lmax = 16 * ((L + 15) // 16)
    useful = useful_fma_per_row(L, K)
    if L % 4 == 0:
        if L >= 16:
            return K >= mfma_min_k(L, H, B * H, plain_loads(B, H, L))
        return 2 * useful * L >= 21 * lmax * lmax
    return B * H >= ODD_MFMA_ROWS or 2 * useful * L >= 10 * lmax * lmax
