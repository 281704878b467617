"""C-ABI and host-logic tests that need no GPU.

The library is loaded and every symbol ``include/pathtile_hip.h`` declares
must be exported; argument validation is exercised only on paths that
return before any HIP call (invalid shapes/configs/NULL pointers).
"""

from __future__ import annotations

import ctypes
import math
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "pathtile_hip.h"


def _declared_symbols() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b((?:pt_|flash_dk_)[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    from pathtile_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("libpathtile_hip.so not built (python -m pathtile_amd.build)")
    return _lib.load()


def test_header_declares_the_expected_entry_points():
    syms = _declared_symbols()
    for name in (
        "pt_dwconv1d_fwd_f32",
        "pt_dwconv1d_dx_f32",
        "pt_dwconv1d_fwd_f32_algo",
        "pt_dwconv1d_dx_f32_algo",
        "pt_dwconv1d_dk_atomic_f32",
        "pt_dwconv1d_dk_det_f32",
        "pt_dwconv1d_dk_det_workspace_bytes",
        "pt_kernel_attributes",
        "pt_status_string",
        "pt_abi_version",
        "flash_dk_fp32",
    ):
        assert name in syms


def test_library_exports_every_declared_symbol(lib):
    from pathtile_amd import _lib

    syms = _declared_symbols()
    out = subprocess.run(["nm", "-D", "--defined-only", str(_lib.LIB_PATH)],
                         capture_output=True, text=True, check=True).stdout
    exported = set(re.findall(r"\bT ((?:pt_|flash_dk_)[a-z0-9_]+)", out))
    assert set(syms) <= exported, set(syms) - exported
    assert set(syms) == set(_lib.SIGNATURES), set(syms) ^ set(_lib.SIGNATURES)
    for name in syms:
        assert getattr(lib, name) is not None


def test_status_codes(lib):
    from pathtile_amd import _lib

    assert lib.pt_abi_version() == 1
    assert _lib.status_string(0) == "ok"
    assert "shape" in _lib.status_string(_lib.PT_ERR_SHAPE)
    assert _lib.status_string(-99) == "unknown status"
    with pytest.raises(ValueError):
        _lib.check(_lib.PT_ERR_SHAPE, "x")
    with pytest.raises(_lib.PathTileLibraryError):
        _lib.check(_lib.PT_ERR_HIP, "x")


def _fake(n=64):
    # Host buffers stand in for device pointers: every call below must be
    # rejected before any pointer is dereferenced or any HIP call is made.
    return (ctypes.c_float * n)()


def test_argument_validation_before_launch(lib):
    from pathtile_amd import _lib

    a, b, c = _fake(), _fake(), _fake()
    P = ctypes.cast
    vp = ctypes.c_void_p
    pa, pb, pc = (vp(ctypes.addressof(t)) for t in (a, b, c))
    S = None
    # NULL pointers
    assert lib.pt_dwconv1d_fwd_f32(None, pb, pc, 1, 1, 8, 3, 4, S) == _lib.PT_ERR_NULL
    assert lib.pt_dwconv1d_dx_f32(pa, None, pc, 1, 1, 8, 3, 4, S) == _lib.PT_ERR_NULL
    assert lib.pt_dwconv1d_dk_atomic_f32(pa, pb, None, 1, 1, 8, 3, 256, 0, S) == _lib.PT_ERR_NULL
    # shapes: L, K in [1, 48]
    for L, K in ((49, 3), (0, 3), (8, 49), (8, 0)):
        assert lib.pt_dwconv1d_fwd_f32(pa, pb, pc, 1, 1, L, K, 4, S) == _lib.PT_ERR_SHAPE
        assert lib.pt_dwconv1d_dk_atomic_f32(pa, pb, pc, 1, 1, L, K, 256, 0, S) == _lib.PT_ERR_SHAPE
    assert lib.pt_dwconv1d_fwd_f32(pa, pb, pc, -1, 1, 8, 3, 4, S) == _lib.PT_ERR_SHAPE
    assert lib.pt_dwconv1d_fwd_f32(pa, pb, pc, 1 << 20, 1 << 10, 48, 3, 4, S) == _lib.PT_ERR_SHAPE
    # launch configs
    for w in (0, 3, 5, 32):
        assert lib.pt_dwconv1d_fwd_f32(pa, pb, pc, 1, 1, 8, 3, w, S) == _lib.PT_ERR_CONFIG
    for t in (0, 32, 96, 800, 1024):
        assert lib.pt_dwconv1d_dk_atomic_f32(pa, pb, pc, 1, 1, 8, 3, t, 0, S) == _lib.PT_ERR_CONFIG
    # alignment
    mis = vp(ctypes.addressof(a) + 2)
    assert lib.pt_dwconv1d_fwd_f32(mis, pb, pc, 1, 1, 8, 3, 4, S) == _lib.PT_ERR_ALIGN
    # empty batch / channels: nothing to launch
    assert lib.pt_dwconv1d_fwd_f32(pa, pb, pc, 0, 4, 8, 3, 4, S) == _lib.PT_OK
    assert lib.pt_dwconv1d_dx_f32(pa, pb, pc, 5, 0, 8, 3, 4, S) == _lib.PT_OK
    # the *_algo entry points: PT_ROWS_AUTO, PT_ROWS_VALU, PT_ROWS_MATRIX only
    for algo in (-1, 3, 7):
        assert lib.pt_dwconv1d_fwd_f32_algo(pa, pb, pc, 1, 1, 8, 3, 4, algo, S) == _lib.PT_ERR_CONFIG
        assert lib.pt_dwconv1d_dx_f32_algo(pa, pb, pc, 1, 1, 8, 3, 4, algo, S) == _lib.PT_ERR_CONFIG
    for algo in (_lib.PT_ROWS_AUTO, _lib.PT_ROWS_VALU, _lib.PT_ROWS_MATRIX):
        assert lib.pt_dwconv1d_fwd_f32_algo(None, pb, pc, 1, 1, 8, 3, 4, algo, S) == _lib.PT_ERR_NULL
        assert lib.pt_dwconv1d_dx_f32_algo(pa, pb, pc, 1, 1, 49, 3, 4, algo, S) == _lib.PT_ERR_SHAPE
        assert lib.pt_dwconv1d_fwd_f32_algo(pa, pb, pc, 0, 4, 8, 3, 4, algo, S) == _lib.PT_OK
    # workspace too small for the deterministic dK
    assert lib.pt_dwconv1d_dk_det_f32(pa, pb, pc, None, 0, 64, 2, 8, 3, 256, S) == _lib.PT_ERR_WORKSPACE
    del P


def test_bf16_argument_validation_before_launch(lib):
    """BF16 entry points: shape, then layout (PT_ERR_CONFIG: L % 4, H % 8 for
    FWD/DX, the channel-group block rule for DK), then empty tensors, NULL,
    and 16-byte alignment, all before any device work."""
    from pathtile_amd import _lib

    buf = (ctypes.c_ubyte * 4096)()
    base = ctypes.addressof(buf)
    al = base + (-base) % 16
    pa, pb, pc = (ctypes.c_void_p(al + o) for o in (0, 1024, 2048))
    mis = ctypes.c_void_p(al + 8)
    S = None
    for fn in (lib.pt_dwconv1d_fwd_bf16, lib.pt_dwconv1d_dx_bf16):
        assert fn(pa, pb, pc, 2, 8, 49, 5, S) == _lib.PT_ERR_SHAPE
        assert fn(pa, pb, pc, 2, 8, 18, 5, S) == _lib.PT_ERR_CONFIG   # L % 4
        assert fn(pa, pb, pc, 2, 12, 16, 5, S) == _lib.PT_ERR_CONFIG  # H % 8
        assert fn(pa, pb, pc, 0, 8, 16, 5, S) == _lib.PT_OK           # empty
        assert fn(None, pb, pc, 2, 8, 16, 5, S) == _lib.PT_ERR_NULL
        assert fn(mis, pb, pc, 2, 8, 16, 5, S) == _lib.PT_ERR_ALIGN
    dk = lib.pt_dwconv1d_dk_atomic_bf16
    assert dk(pa, pb, pc, 2, 8, 18, 5, 128, 0, S) == _lib.PT_ERR_CONFIG   # L % 4
    assert dk(pa, pb, pc, 2, 6, 16, 5, 256, 0, S) == _lib.PT_ERR_CONFIG   # H % (2 * 4)
    assert dk(pa, pb, pc, 2, 24, 16, 5, 768, 0, S) == _lib.PT_ERR_CONFIG  # > 8 waves
    assert dk(pa, pb, None, 2, 8, 16, 5, 128, 0, S) == _lib.PT_ERR_NULL
    assert dk(mis, pb, pc, 2, 8, 16, 5, 128, 0, S) == _lib.PT_ERR_ALIGN
    assert lib.pt_dwconv1d_dk_det_bf16(pa, pb, pc, None, 0, 2, 8, 16, 5, 128, S) == _lib.PT_ERR_WORKSPACE


def test_flash_dk_fp32_validation_before_launch(lib):
    """The Flash-DWC bridge ABI returns -2 for every argument the bridge
    rejects (benchmark/flashdwc_fp32_bridge.cu:14-19) and for the ones this
    library does not serve (L or K above 48, misaligned tensors), before any
    device work."""
    buf = (ctypes.c_ubyte * 4096)()
    base = ctypes.addressof(buf)
    al = base + (-base) % 16
    x, dy, dw = (ctypes.c_void_p(al + o) for o in (0, 1024, 2048))
    fn = lib.flash_dk_fp32
    S = None
    ok = (32, 32, 48, 48, 1)  # B, H, L, K, GZ that pass every check
    cases = [
        ((None, dy, dw), ok),
        ((x, None, dw), ok),
        ((x, dy, None), ok),
        ((x, dy, dw), (0, 32, 48, 48, 1)),        # B <= 0
        ((x, dy, dw), (32, 0, 48, 48, 1)),        # H <= 0
        ((x, dy, dw), (32, 48, 48, 48, 1)),       # H % 32
        ((x, dy, dw), (32, 32, 0, 48, 1)),        # L <= 0
        ((x, dy, dw), (32, 32, 48, 0, 1)),        # K <= 0
        ((x, dy, dw), (32, 32, 48, 48, 0)),       # GZ <= 0
        ((x, dy, dw), (32, 32, 48, 48, 3)),       # B % GZ
        ((x, dy, dw), (48, 32, 48, 48, 2)),       # (B / GZ) % 16
        ((x, dy, dw), (32, 32, 49, 48, 1)),       # L above 48
        ((x, dy, dw), (32, 32, 48, 49, 1)),       # K above 48
        ((ctypes.c_void_p(al + 4), dy, dw), ok),  # x not 16-byte aligned
        ((x, ctypes.c_void_p(al + 1032), dw), ok),
        ((x, dy, ctypes.c_void_p(al + 2050)), ok),
    ]
    for ptrs, (B, H, L, K, gz) in cases:
        assert fn(*ptrs, B, H, L, K, gz, S) == -2, (ptrs, B, H, L, K, gz)


def test_long_row_validation_and_workspace(lib):
    """Long-row entry points: L up to 192 and K up to 256, then NULL / 4-byte alignment
    / workspace checks before any device work; the DK workspace is
    [H, K, ranges] floats with ranges = ceil(512 / H), at most one per
    32 samples (a function of B and H only)."""
    from pathtile_amd import _lib

    buf = (ctypes.c_ubyte * 4096)()
    base = ctypes.addressof(buf)
    al = base + (-base) % 16
    pa, pb, pc = (ctypes.c_void_p(al + o) for o in (0, 1024, 2048))
    mis = ctypes.c_void_p(al + 2)
    S = None
    for fn in (lib.pt_dwconv1d_fwd_long_f32, lib.pt_dwconv1d_dx_long_f32):
        assert fn(pa, pb, pc, 2, 4, 193, 5, S) == _lib.PT_ERR_SHAPE
        assert fn(pa, pb, pc, 2, 4, 192, 257, S) == _lib.PT_ERR_SHAPE
        assert fn(pa, pb, pc, 2, 4, 0, 5, S) == _lib.PT_ERR_SHAPE
        assert fn(pa, pb, pc, -1, 4, 16, 5, S) == _lib.PT_ERR_SHAPE
        assert fn(pa, pb, pc, 1 << 16, 1 << 12, 192, 5, S) == _lib.PT_ERR_SHAPE  # 2^31 elements
        assert fn(pa, pb, pc, 0, 4, 192, 5, S) == _lib.PT_OK                      # empty
        assert fn(None, pb, pc, 2, 4, 192, 5, S) == _lib.PT_ERR_NULL
        assert fn(mis, pb, pc, 2, 4, 192, 5, S) == _lib.PT_ERR_ALIGN
    out = ctypes.c_size_t(0)

    def ranges(B, H):
        return max(1, min(-(-512 // H), -(-B // 32)))

    for (B, H, L, K) in [(16384, 128, 192, 192), (16384, 64, 192, 3), (100, 1000, 64, 64),
                         (40, 8, 176, 256), (1, 3, 1, 1), (4096, 512, 128, 48)]:
        assert lib.pt_dwconv1d_dk_long_workspace_bytes(B, H, L, K, ctypes.byref(out)) == _lib.PT_OK
        assert out.value == H * K * ranges(B, H) * 4, (B, H, L, K)
    lib.pt_dwconv1d_dk_long_workspace_bytes(16384, 128, 192, 192, ctypes.byref(out))
    assert out.value == 128 * 192 * 4 * 4  # 4 ranges
    lib.pt_dwconv1d_dk_long_workspace_bytes(40, 128, 192, 192, ctypes.byref(out))
    assert out.value == 128 * 192 * 2 * 4  # B = 40: two 32-sample steps, two ranges
    lib.pt_dwconv1d_dk_long_workspace_bytes(0, 128, 192, 192, ctypes.byref(out))
    assert out.value == 0
    dk = lib.pt_dwconv1d_dk_long_f32
    assert dk(pa, pb, pc, None, 0, 2, 4, 193, 5, S) == _lib.PT_ERR_SHAPE
    assert dk(pa, pb, pc, None, 0, 2, 4, 192, 257, S) == _lib.PT_ERR_SHAPE
    assert dk(pa, pb, None, None, 0, 2, 4, 192, 5, S) == _lib.PT_ERR_NULL
    assert dk(pa, pb, mis, None, 0, 2, 4, 192, 5, S) == _lib.PT_ERR_ALIGN
    assert dk(None, pb, pc, None, 0, 2, 4, 192, 5, S) == _lib.PT_ERR_NULL
    assert dk(pa, pb, pc, None, 0, 2, 4, 192, 5, S) == _lib.PT_ERR_WORKSPACE
    assert dk(pa, pb, pc, pa, 8, 2, 4, 192, 5, S) == _lib.PT_ERR_WORKSPACE   # needs 80 bytes
    assert dk(pa, pb, pc, None, 0, 2, 0, 192, 5, S) == _lib.PT_OK            # H == 0


def test_bf16_workspace_bytes(lib):
    """BF16 DK partials: [H, K, ranges] floats, one range per 16-sample step
    at most; the range count is, of 2^k and 3 * 2^(k-1) in [8, 256], the one
    nearest by ratio to 3 MiB / (16 * 2 * H * L bytes) (ties to the smaller),
    at every tensor size; independent of the block size."""
    from pathtile_amd import _lib

    out = ctypes.c_size_t(0)
    cands = sorted({c for k in range(3, 9) for c in (2**k, 3 * 2**(k - 1)) if 8 <= c <= 256})

    def ranges(B, H, L):
        want = 3 * 2**20 / (32 * H * L)
        n = min(cands, key=lambda c: (abs(math.log(c / want)), c))
        return max(1, min(n, -(-B // 16)))

    for (B, H, L, K) in [(16384, 128, 48, 48), (32768, 256, 48, 4), (4096, 128, 24, 48),
                         (2048, 64, 24, 48), (16384, 64, 16, 3), (40, 8, 16, 5), (1, 8, 4, 3)]:
        for threads in (64, 128, 256, 512):
            if H % (2 * threads // 64):
                continue
            st = lib.pt_dwconv1d_dk_det_bf16_workspace_bytes(B, H, L, K, threads, ctypes.byref(out))
            assert st == _lib.PT_OK
            assert out.value == H * K * ranges(B, H, L) * 4, (B, H, L, threads)
    # P in BF16: 192 KiB steps, 3 MiB / 192 KiB = 16 ranges
    lib.pt_dwconv1d_dk_det_bf16_workspace_bytes(16384, 128, 48, 48, 128, ctypes.byref(out))
    assert out.value == 128 * 48 * 16 * 4
    # B = 40: three 16-sample steps, so three ranges
    lib.pt_dwconv1d_dk_det_bf16_workspace_bytes(40, 8, 16, 5, 128, ctypes.byref(out))
    assert out.value == 8 * 5 * 3 * 4


def test_workspace_bytes(lib):
    from pathtile_amd import _lib

    out = ctypes.c_size_t(0)

    def nbt(B, H, L, K, threads):
        st = lib.pt_dwconv1d_dk_det_workspace_bytes(B, H, L, K, threads, ctypes.byref(out))
        assert st == _lib.PT_OK
        assert out.value % (H * K * 4) == 0  # [H, K, num_btiles] floats
        return out.value // (H * K * 4)

    # The kernel, and so the partial count, follows from the shape and block
    # size (alignment only sets the channel-group kernel's staging width):
    #  * channel-group interleaved sample ranges where the layout allows (at
    #    most 8 waves, H a multiple of the group: one channel per wave for
    #    rows of 33-48 columns, two below; any L), at most one per 4-sample
    #    step: for tensors of at least 256 MiB, of 2^k and 3 * 2^(k-1) in
    #    [8, 256] the one nearest by ratio to 3 MiB / (16 H L bytes) (ties to
    #    the smaller); below that, the power of two in [8, 256] nearest to
    #    2.5 MiB / (16 H L bytes);
    #  * otherwise per-channel batch tiles of (threads / 64) waves x
    #    rows-per-wave samples; rows per wave are whole load groups (48 / 24
    #    / 16 samples for rows of <= 16 / <= 32 / <= 48 floats), up to 128.
    # Both depend on the shape and block size only, never on the device.
    def per_channel(B, H, L, wpb):
        grp = 48 // (-(-L // 16))
        rpw = -(-(B * H) // 16384)
        rpw = min(max(-(-rpw // grp) * grp, grp), -(-128 // grp) * grp)
        rpw = min(rpw, -(-(-(-B // wpb)) // grp) * grp)
        return -(-B // (wpb * rpw))

    def channel_group(B, H, L, wpb):
        cpw = 1 if L > 32 else 2
        if wpb > 8 or H % (cpw * wpb):
            return 0
        if 4 * B * H * L >= 256 * 2**20:
            want = 3 * 2**20 / (16 * H * L)
            cands = sorted({c for k in range(3, 9) for c in (2**k, 3 * 2**(k - 1)) if 8 <= c <= 256})
            n = min(cands, key=lambda c: (abs(math.log(c / want)), c))
        else:
            want = 2.5 * 2**20 / (16 * H * L)
            n = 8
            while n < 256 and n * 2 <= want * 2**0.5:
                n *= 2
        return max(1, min(n, -(-B // 4)))

    for (B, H, L, K) in [(16384, 128, 48, 48), (16384, 64, 16, 3), (1000, 96, 37, 48),
                         (32768, 256, 48, 4), (20, 4, 8, 3), (4096, 128, 24, 8), (3, 16, 48, 5),
                         (1000, 7, 37, 48), (500, 12, 30, 9)]:
        for threads in (64, 128, 192, 256, 512, 768):
            wpb = threads // 64
            n = nbt(B, H, L, K, threads)
            assert n == (channel_group(B, H, L, wpb) or per_channel(B, H, L, wpb)), (B, H, L, threads)
    assert nbt(16384, 128, 48, 48, 256) == 32   # 32 ranges (96 KiB steps), 32 tiles
    assert nbt(16384, 64, 16, 3, 256) == 128    # 64 MiB tensors, 16 KiB steps: 128
    assert nbt(16384, 128, 40, 48, 256) == 32   # 80 KiB steps: 38.4 -> 32 (not 48)
    assert nbt(16384, 128, 32, 8, 256) == 48    # 256 MiB tensors, 64 KiB steps: 48 = 3 * 2^4
    assert nbt(8192, 128, 32, 8, 256) == 32     # 128 MiB tensors: 2.5 MiB rule, 32
    assert nbt(16384, 128, 48, 48, 192) == 43   # per-channel: 3 waves x 128 samples
    assert nbt(1000, 96, 37, 48, 64) == 64      # L % 4 != 0: channel-group, 2.5 MiB rule
    assert nbt(1000, 7, 37, 48, 128) == 32      # H % 2 != 0: per-channel, 2 waves x 16 samples
    st = lib.pt_dwconv1d_dk_det_workspace_bytes(0, 4, 8, 3, 256, ctypes.byref(out))
    assert st == _lib.PT_OK and out.value == 0
    lds = ctypes.c_int(0)
    assert lib.pt_dynamic_lds_bytes(_lib.PT_KERNEL_FWD, 48, 48, 8, ctypes.byref(lds)) == 0
    assert lds.value == 8 * 64 * (48 + 4) * 4  # 64-row tile, padded stride
    assert lib.pt_dynamic_lds_bytes(_lib.PT_KERNEL_FWD, 48, 48, 3, ctypes.byref(lds)) == _lib.PT_ERR_CONFIG
    # matrix-core FWD/DX: 8 channels x 16 samples, two input + two output stages
    for kid in (_lib.PT_KERNEL_FWD_CG, _lib.PT_KERNEL_DX_CG):
        for L in (4, 16, 32, 48):
            assert lib.pt_dynamic_lds_bytes(kid, L, 48, 1, ctypes.byref(lds)) == 0
            assert lds.value == 4 * 16 * (8 * L + 4) * 4
        assert lib.pt_dynamic_lds_bytes(kid, 48, 48, 3, ctypes.byref(lds)) == _lib.PT_ERR_CONFIG
    # 16-channel matrix-core FWD/DX: one input + two output stages
    for kid in (_lib.PT_KERNEL_FWD_CG16, _lib.PT_KERNEL_DX_CG16):
        assert lib.pt_dynamic_lds_bytes(kid, 48, 48, 4, ctypes.byref(lds)) == 0
        assert lds.value == 3 * 16 * (16 * 48 + 4) * 4
    # short-tap streaming FWD/DX: no LDS
    for kid in (_lib.PT_KERNEL_FWD_STREAM, _lib.PT_KERNEL_DX_STREAM):
        assert lib.pt_dynamic_lds_bytes(kid, 48, 4, 16, ctypes.byref(lds)) == 0
        assert lds.value == 0
        assert lib.pt_dynamic_lds_bytes(kid, 48, 4, 3, ctypes.byref(lds)) == _lib.PT_ERR_CONFIG


def test_library_is_not_linked_to_the_oracle():
    from pathtile_amd import _lib

    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    needed = subprocess.run(["readelf", "-d", str(_lib.LIB_PATH)], capture_output=True,
                            text=True, check=True).stdout
    assert "oracle" not in needed
    assert "libamdhip64.so" in needed


def test_flat_tile_row_magic_is_exact():
    """The FWD/DX kernels split a flat tile element e (< 64 * 48) into
    (row, col) as row = (e * ceil(2^20 / L)) >> 20; exact for every L <= 48."""
    for L in range(1, 49):
        magic = ((1 << 20) + L - 1) // L
        for e in range(64 * L):
            row = (e * magic) >> 20
            assert row == e // L, (L, e)
            assert (e * magic) < (1 << 32)


def test_xcd_remap_is_a_bijection():
    """Workgroup renumbering used by the dK kernels (8 XCDs, round-robin)."""
    import random

    def remap(p, n):
        q, r = divmod(n, 8)
        x, i = p % 8, p // 8
        return x * (q + 1) + i if x < r else r * (q + 1) + (x - r) * q + i

    for n in list(range(1, 130)) + [random.Random(1).randint(1, 50000) for _ in range(20)]:
        assert sorted(remap(p, n) for p in range(n)) == list(range(n))


def test_noalloc_dk_validation_and_scratch_limit_before_launch(lib):
    """pt_dwconv1d_dk_det_f32_noalloc checks shape, config, NULL, alignment
    and then its static scratch (PT_DK_SCRATCH_BYTES of partials) before any
    device query or launch: a shape whose workspace size (the shape-only
    partial count pt_dwconv1d_dk_det_workspace_bytes reports) exceeds it is
    refused with PT_ERR_SCRATCH, for 16-byte aligned (channel-group) and
    4-byte aligned (per-channel) inputs alike."""
    from pathtile_amd import _lib

    buf = (ctypes.c_ubyte * 4096)()
    base = ctypes.addressof(buf)
    al = base + (-base) % 16
    pa, pb, pc = (ctypes.c_void_p(al + o) for o in (0, 1024, 2048))
    mis = [ctypes.c_void_p(al + o) for o in (4, 1028)]
    fn = lib.pt_dwconv1d_dk_det_f32_noalloc
    S = None
    assert fn(pa, pb, pc, 1, 1, 49, 3, 128, S) == _lib.PT_ERR_SHAPE
    assert fn(pa, pb, pc, 1, 1, 8, 3, 96, S) == _lib.PT_ERR_CONFIG
    assert fn(pa, pb, None, 1, 1, 8, 3, 128, S) == _lib.PT_ERR_NULL
    assert fn(None, pb, pc, 1, 1, 8, 3, 128, S) == _lib.PT_ERR_NULL
    assert fn(ctypes.c_void_p(al + 2), pb, pc, 1, 1, 8, 3, 128, S) == _lib.PT_ERR_ALIGN
    B, H, L, K = 64, 65536, 48, 48  # 65536 * 48 taps * 4 bytes = 12 MiB per range
    need = ctypes.c_size_t(0)
    assert lib.pt_dwconv1d_dk_det_workspace_bytes(B, H, L, K, 128, ctypes.byref(need)) == 0
    assert need.value > _lib.PT_DK_SCRATCH_BYTES
    assert fn(pa, pb, pc, B, H, L, K, 128, S) == _lib.PT_ERR_SCRATCH
    assert fn(mis[0], mis[1], pc, B, H, L, K, 128, S) == _lib.PT_ERR_SCRATCH
    # The limit is the size the workspace query reports, whatever one range
    # needs: 8 ranges of 8192 * 48 taps (1.5 MiB each, 12 MiB in all) are
    # refused; 8 ranges of 4096 * 48 (6 MiB) pass the check (and then need a
    # device, which this host lacks).
    for H2, refused in ((8192, True), (4096, False)):
        assert lib.pt_dwconv1d_dk_det_workspace_bytes(64, H2, 8, 48, 128, ctypes.byref(need)) == 0
        assert (need.value > _lib.PT_DK_SCRATCH_BYTES) == refused
        st = fn(pa, pb, pc, 64, H2, 8, 48, 128, S)
        assert (st == _lib.PT_ERR_SCRATCH) == refused, st
    assert "static scratch" in _lib.status_string(_lib.PT_ERR_SCRATCH)
    with pytest.raises(ValueError, match="static scratch"):
        _lib.check(_lib.PT_ERR_SCRATCH, "pt_dwconv1d_dk_det_f32_noalloc")


def test_rows_kernel_query_matches_the_restated_rule(lib, monkeypatch):
    """pt_rows_kernel_id runs the library's own FWD/dX dispatch up to the
    launch. Its matrix-core / VALU answer must equal the Python restatement
    (pathtile_amd.rows_rule, used where no device is present) at every row
    length and tap count, in each size class the rule separates: calls of
    fewer than 2^17 rows, of at least 2^18 rows, tensors of at most and above
    256 MiB, H above 128, H not a multiple of 8. The matrix-core choice does
    not depend on device queries, so this holds without a GPU."""
    from pathtile_amd import rows_rule, runtime

    monkeypatch.delenv("PATHTILE_ROWS_ALGO", raising=False)
    monkeypatch.delenv("PATHTILE_ROWS_CHANNELS", raising=False)
    mismatches = []
    for B, H in ((1000, 96), (2048, 64), (16384, 128), (4096, 256), (32768, 256), (3000, 36)):
        for L in range(1, 49):
            for K in range(1, 49):
                lib_mfma = runtime.rows_on_matrix_cores(B, H, L, K)
                if lib_mfma != rows_rule.matrix_cores_serve(B, H, L, K):
                    mismatches.append((B, H, L, K, lib_mfma))
    assert not mismatches, mismatches[:20]


def test_rows_kernel_query_ids_and_errors(lib, monkeypatch):
    """The query names a kernel of its path, honours the forced choices,
    reports -1 for empty calls and returns the launch's error codes."""
    from pathtile_amd import _lib, runtime

    monkeypatch.delenv("PATHTILE_ROWS_ALGO", raising=False)
    fwd_ids = {_lib.PT_KERNEL_FWD, _lib.PT_KERNEL_FWD_STREAM, _lib.PT_KERNEL_FWD_CG,
               _lib.PT_KERNEL_FWD_CG16}
    dx_ids = {_lib.PT_KERNEL_DX, _lib.PT_KERNEL_DX_STREAM, _lib.PT_KERNEL_DX_CG,
              _lib.PT_KERNEL_DX_CG16}
    assert runtime.rows_kernel_id(16384, 128, 48, 48) in fwd_ids
    assert runtime.rows_kernel_id(16384, 128, 48, 48, dx=True) in dx_ids
    assert runtime.rows_kernel_id(16384, 128, 48, 48, algo="valu") == _lib.PT_KERNEL_FWD
    assert runtime.rows_kernel_id(257, 8, 48, 4, algo="mfma") == _lib.PT_KERNEL_FWD_CG
    # the matrix cores need H % 8 == 0 and 16-byte aligned tensors
    assert runtime.rows_kernel_id(257, 12, 48, 48, algo="mfma") == _lib.PT_KERNEL_FWD
    assert runtime.rows_kernel_id(16384, 128, 48, 48, aligned16=False) == _lib.PT_KERNEL_FWD
    assert runtime.rows_kernel_id(0, 128, 48, 48) == -1
    assert runtime.rows_kernel_name(0, 128, 48, 48) == "none"
    monkeypatch.setenv("PATHTILE_ROWS_ALGO", "valu")
    assert runtime.rows_kernel_name(16384, 128, 48, 48) == "dwconv_rows_kernel<FWD>"
    for bad in ((16, 8, 49, 4), (16, 8, 48, 49), (16, 8, 0, 4)):
        with pytest.raises(ValueError):
            runtime.rows_kernel_id(*bad)
    with pytest.raises(ValueError):
        runtime.rows_kernel_id(16, 8, 48, 4, waves_per_block=3)
    out = ctypes.c_int(0)
    assert lib.pt_rows_kernel_id(16, 8, 48, 4, 4, 0, 1, 0, None) == _lib.PT_ERR_NULL
    assert lib.pt_rows_kernel_id(16, 8, 48, 4, 4, 7, 1, 0, ctypes.byref(out)) == _lib.PT_ERR_CONFIG
