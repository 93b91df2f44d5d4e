"""Seeded sweep over the forward kernels' shape classes against the CPU oracle.

Each case draws its own shape from a fixed seed list so the sweep is
deterministic. It covers the kernel selection boundaries: streaming (a single
query within one pass, per-query docs), tiled (batched queries over shared
docs, single queries past one streaming pass; row blocks of 128 to 1024 rows,
DMA-staged exact-width rows and VGPR-staged masked widths), split-d (d > 256),
single and batched queries,
shared and per-query docs, ragged lengths (0, 1, Ld, > Ld), fp16 and bf16,
and uint8 docs in one- and two-doc workgroups. Scores within 1e-2 of the
float64 oracle on the same input values.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flash_maxsim_amd as fm
from conftest import sim, to_np32

pytestmark = pytest.mark.gpu

DEV = "cuda"
ATOL = 1e-2

# (Nq, Lq, B, Ld, d, dtype, shared_docs)
CASES = [
    (1, 32, 37, 300, 128, torch.float16, True),     # stream, metric shape class
    (1, 17, 9, 65, 64, torch.bfloat16, True),       # stream, bf16, odd sizes
    (1, 256, 12, 200, 128, torch.float16, True),    # tiled, single query, exact width (DMA)
    (1, 300, 10, 130, 96, torch.float16, True),     # tiled, masked width (VGPR staging)
    (1, 257, 11, 77, 256, torch.bfloat16, True),    # tiled KS = 8, straddling row blocks
    (12, 32, 40, 150, 128, torch.float16, True),    # tiled batched, 384 rows
    (9, 40, 13, 90, 128, torch.bfloat16, True),     # tiled batched, queries straddle blocks
    (3, 32, 7, 50, 128, torch.float16, False),      # stream, per-query docs
    (5, 70, 6, 40, 128, torch.float16, False),      # per-query docs, 350 rows
    (1, 64, 8, 100, 512, torch.float16, True),      # split-d
    (4, 20, 6, 33, 768, torch.bfloat16, True),      # split-d batched, bf16
    (1, 130, 5, 64, 1024, torch.float16, True),     # split-d, two passes
    (1, 200, 14, 100, 128, torch.float16, True),    # tiled single query, 256-row block
    (2, 17, 11, 70, 64, torch.bfloat16, True),      # tiled, two short queries, 128-row block
    (3, 50, 9, 80, 192, torch.float16, True),       # tiled d = 192 (masked), 256-row block
    (4, 8, 10, 33, 128, torch.float16, True),       # tiled, four 8-token queries
    (2, 150, 7, 60, 128, torch.float16, False),     # stream, per-query docs, two passes on one XCD
    (3, 40, 5, 30, 640, torch.bfloat16, True),      # split-d, three queries of a shared doc on one XCD
    (3, 32, 9, 140, 100, torch.float16, True),      # tiled register ring, masked width with a partial chunk
    (2, 40, 13, 200, 120, torch.bfloat16, True),    # tiled register ring, masked width, doc walk past 4 tiles
]


def _lengths(seed, n, Ld):
    g = torch.Generator().manual_seed(seed)
    lt = torch.randint(1, Ld + 1, (n,), generator=g, dtype=torch.int32)
    if n > 1:
        lt[0] = 0
        lt[1] = 1
    if n > 2:
        lt[2] = Ld + 5  # clamps to Ld
    if n > 3:
        lt[3] = Ld
    return lt


@pytest.mark.parametrize("case", range(len(CASES)))
def test_forward_sweep(oracle_mod, case):
    Nq, Lq, B, Ld, d, dtype, shared = CASES[case]
    seed = 9000 + 17 * case
    Q = sim((Nq, Lq, d), seed, dtype)
    Drows = B if shared else Nq * B
    D = sim((Drows, Ld, d), seed + 1, dtype)
    lt = _lengths(seed + 2, Drows, Ld)
    if Nq == 1:
        got = fm.flash_maxsim(Q[0].to(DEV), D.to(DEV), lt.to(DEV)).reshape(1, B)
    else:
        Dk = D if shared else D.reshape(Nq, B, Ld, d)
        got = fm.flash_maxsim_batched(Q.to(DEV), Dk.to(DEV), lt.to(DEV), shared)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lt.numpy(), shared_docs=shared)  # [Nq, B]
    got = got.double().cpu().numpy()
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    assert fin.any() and np.abs(got[fin] - ref[fin]).max() <= ATOL


@pytest.mark.parametrize("B, Lq, Ld, d", [(1, 32, 40, 128), (2, 32, 40, 128), (3, 5, 200, 64),
                                          (13, 32, 96, 128), (6, 48, 33, 256),
                                          (11, 100, 70, 128)])  # two 64-token passes
def test_int8_sweep(oracle_mod, B, Lq, Ld, d):
    seed = 9500 + B * 7 + d
    Q = sim((Lq, d), seed)
    x = sim((B, Ld, d), seed + 1, torch.float32)
    codes, s, m = fm.quantize_int8(x)
    lt = _lengths(seed + 2, B, Ld)
    got = fm.flash_maxsim_int8(Q.to(DEV), codes.to(DEV), s.to(DEV), m.to(DEV), lt.to(DEV))
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(s), to_np32(m), lt.numpy())
    got = got.double().cpu().numpy().reshape(ref.shape)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    assert fin.any() and np.abs(got[fin] - ref[fin]).max() <= ATOL
