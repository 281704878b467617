"""The library's FWD/dX kernel choice on the GPU, on both sides of each
threshold of the rule (rows_algo / rows_mfma_min_k in csrc/dwconv1d_abi.hip,
restated in pathtile_amd/rows_rule.py): the library's own answer
(pt_rows_kernel_id) must equal the restatement; where they say the VALU
kernels serve, sampled rows must be the reference's fmaf chain bit for bit;
where they say the matrix cores serve, they must differ from that chain
somewhere (the matrix cores sum in their own order) and stay within 1e-5 of
FP64. The shapes cover every row length with a threshold of its own and the
size classes the rule separates: calls of fewer than 2^17 rows, tensors of at
most 256 MiB and above, H above 128 at L = 48, rows of L % 4 != 0 from 2^18
rows (B x H) and below, and rows shorter than 16."""

from __future__ import annotations

import numpy as np
import pytest
import torch

import oracle
from pathtile_amd import rows_rule, runtime

pytestmark = pytest.mark.gpu

FWD_TOL = 1e-5
SAMPLE = 48

# (B, H, L, K) pairs: the last K below a threshold, then the threshold
CASES = [
    (16384, 128, 16, 4), (16384, 128, 16, 5),      # >= 2^17 rows: L16 from K = 5
    (1024, 96, 16, 11), (1024, 96, 16, 12),        # small call: L16 from K = 12
    (16384, 128, 24, 8), (16384, 128, 24, 9),      # L24 from K = 9
    (1024, 96, 24, 16), (1024, 96, 24, 17),        # small call: L24 from K = 17
    (16384, 128, 40, 16), (16384, 128, 40, 17),    # L40 from K = 17
    (2000, 64, 40, 24), (2000, 64, 40, 25),        # small call: L40 from K = 25
    (8192, 128, 48, 8), (8192, 128, 48, 9),        # L48, <= 256 MiB, H <= 128: K = 9
    (4096, 256, 48, 16), (4096, 256, 48, 17),      # L48, H > 128: K = 17
    (16384, 128, 48, 16), (16384, 128, 48, 17),    # L48 above 256 MiB: K = 17
    (16384, 128, 20, 8), (16384, 128, 20, 9),      # L20 from K = 9
    (16384, 128, 28, 8), (16384, 128, 28, 9),      # L28 from K = 9
    (16384, 128, 32, 8), (16384, 128, 32, 9),      # L32 from K = 9
    (16384, 128, 36, 16), (16384, 128, 36, 17),    # L36 from K = 17
    (16384, 128, 44, 8), (16384, 128, 44, 9),      # L44 from K = 9
    (4095, 64, 37, 6), (4096, 64, 37, 6),          # L % 4 != 0: from 2^18 rows
    (1000, 96, 37, 8), (1000, 96, 37, 9),          # below: 5 (48 / 37)^2 FMAs per output
    (16384, 64, 12, 12),                           # L < 16, L % 4 == 0: VALU
]


@pytest.fixture(scope="module")
def rt():
    from pathtile_amd import runtime

    r = runtime.HipWarpRuntime()
    yield r
    r.close()


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}H{}L{}K{}".format(*c))
def test_kernel_choice_matches_the_restated_rule(rt, case):
    B, H, L, K = case
    mfma = rows_rule.matrix_cores_serve(B, H, L, K)
    assert runtime.rows_on_matrix_cores(B, H, L, K) == mfma
    assert runtime.rows_on_matrix_cores(B, H, L, K, dx=True) == mfma
    print(f"[case] rule B={B} H={H} L={L} K={K} matrix_cores={mfma}", flush=True)
    g = torch.Generator().manual_seed(1000 + B + H + L + K)
    x = torch.randn(B, H, L, generator=g)
    w = torch.randn(H, K, generator=g) / np.sqrt(K)
    idx = torch.from_numpy(np.random.default_rng(K).choice(B, SAMPLE, replace=False))
    idx[0], idx[-1] = 0, B - 1
    xd, wd = x.to("cuda:0"), w.to("cuda:0")
    for dx in (False, True):
        out = torch.empty_like(xd)
        (rt.launch_bwd_input if dx else rt.launch_fwd)(xd, wd, out)
        got = out[idx.to("cuda:0")].cpu().numpy()
        xs = x[idx]
        chain = (oracle.dx_f32_refchain if dx else oracle.fwd_f32_refchain)(xs, w)
        exact = (oracle.dx_f64 if dx else oracle.fwd_f64)(xs, w)
        assert oracle.normalized_max_abs(got, exact) < FWD_TOL
        if mfma:
            assert not np.array_equal(got, chain), "expected the matrix cores' summation order"
        else:
            assert np.array_equal(got, chain), "expected the VALU kernels' fmaf chain"
    del xd, out
    torch.cuda.empty_cache()
