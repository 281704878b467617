"""The no-allocation deterministic dK (pt_dwconv1d_dk_det_f32_noalloc)
against the workspace entry point (pt_dwconv1d_dk_det_f32), through the C
ABI (marked ``gpu``).

The two entry points run the same kernels in the same order, so their
results must agree bit for bit. The workspace version gets a NaN-filled
workspace: any partial that the kernels read without writing first would
show up. Two no-allocation calls in a row, the second on a smaller input,
check that nothing of the first call's scratch leaks into the second. After
one eager call, a call allocates nothing (torch's allocation count and the
device's free memory unchanged) and runs under HIP graph capture: every
replay of the captured call gives the eager bits. (The refusal of shapes
beyond the static scratch depends on the shape alone, comes before any
device query, and is tested on the CPU, tests/test_abi_cpu.py.)
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

import oracle

pytestmark = pytest.mark.gpu


def _vp(t):
    return ctypes.c_void_p(t.data_ptr())


def _stream():
    return ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)


def _det_workspace(lib, dy, x, K, threads):
    from pathtile_amd import _lib

    B, H, L = map(int, x.shape)
    nbytes = ctypes.c_size_t(0)
    _lib.check(lib.pt_dwconv1d_dk_det_workspace_bytes(B, H, L, K, threads,
                                                      ctypes.byref(nbytes)), "ws bytes")
    ws = torch.full((max(nbytes.value, 4) // 4,), float("nan"), device=x.device)
    gk = torch.full((H, K), float("nan"), device=x.device)
    _lib.check(lib.pt_dwconv1d_dk_det_f32(_vp(dy), _vp(x), _vp(gk), _vp(ws), ws.numel() * 4,
                                          B, H, L, K, threads, _stream()), "det")
    return gk


def _det_noalloc(lib, dy, x, K, threads):
    from pathtile_amd import _lib

    B, H, L = map(int, x.shape)
    gk = torch.full((H, K), float("nan"), device=x.device)
    _lib.check(lib.pt_dwconv1d_dk_det_f32_noalloc(_vp(dy), _vp(x), _vp(gk), B, H, L, K,
                                                  threads, _stream()), "det noalloc")
    return gk


@pytest.mark.parametrize("threads", [128, 256])
@pytest.mark.parametrize("first,second", [
    ((16384, 128, 48, 48), (300, 16, 48, 47)),   # channel-group kernel, then a smaller one
    ((4096, 96, 37, 48), (1000, 8, 37, 5)),      # channel-group kernel, dword staging (L % 4 != 0)
    ((4096, 7, 37, 48), (1000, 5, 20, 5)),       # per-channel kernel (H not a multiple of the group)
])
def test_noalloc_matches_workspace_entry_point(first, second, threads):
    from pathtile_amd import _lib

    lib = _lib.load()
    for shape in (first, second):
        B, H, L, K = shape
        print(f"[case] noalloc B={B} H={H} L={L} K={K} threads={threads}", flush=True)
        x, w, dy = oracle.make_inputs(B, H, L, K, seed=B + H + L + K)
        xd, dyd = x.cuda(), dy.cuda()
        a = _det_noalloc(lib, dyd, xd, K, threads)
        b = _det_workspace(lib, dyd, xd, K, threads)
        torch.cuda.synchronize()
        a, b = a.cpu().numpy(), b.cpu().numpy()
        assert np.isfinite(a).all()
        assert np.array_equal(a, b)
        if B * H <= 2_000_000:
            assert oracle.normalized_max_abs(a, oracle.dk_f64(dy, x, K)) < 1e-4


def test_noalloc_allocates_nothing_and_replays_under_graph_capture():
    from pathtile_amd import _lib

    lib = _lib.load()
    B, H, L, K, threads = 4096, 128, 48, 48, 128
    print(f"[case] noalloc graph B={B} H={H} L={L} K={K} threads={threads}", flush=True)
    x, w, dy = oracle.make_inputs(B, H, L, K, seed=404)
    xd, dyd = x.cuda(), dy.cuda()
    gk = torch.full((H, K), float("nan"), device="cuda")

    def call():
        _lib.check(lib.pt_dwconv1d_dk_det_f32_noalloc(_vp(dyd), _vp(xd), _vp(gk), B, H, L, K,
                                                      threads, _stream()), "det noalloc")

    call()  # the warm-up call: scratch address and occupancy lookups
    torch.cuda.synchronize()
    eager = gk.clone()
    assert np.array_equal(eager.cpu().numpy(), _det_workspace(lib, dyd, xd, K, threads).cpu().numpy())
    torch.cuda.synchronize()
    alloc0 = torch.cuda.memory_allocated()
    free0, _ = torch.cuda.mem_get_info()
    gk.fill_(float("nan"))
    call()
    torch.cuda.synchronize()
    assert torch.cuda.memory_allocated() == alloc0
    assert torch.cuda.mem_get_info()[0] == free0
    assert torch.equal(gk, eager)

    graph = torch.cuda.CUDAGraph()
    gk.fill_(float("nan"))
    torch.cuda.synchronize()
    with torch.cuda.graph(graph):
        call()
    for i in range(4):
        gk.fill_(float("nan"))          # eager work between the replays
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(gk, eager), i
    del graph
