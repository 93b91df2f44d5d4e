"""GPU parity across the forward's kernel routes near their boundaries.

fmx_fwd picks, for single queries, the streaming kernel with one or two docs
per workgroup or the tiled kernel by query rows, doc length and width, and
pairs per-query docs. This file draws seeded shapes on both sides of those
boundaries (query rows 32/33, 64/65, 128/129; doc lengths 96/97, 160/161,
256/257; widths 64, 96, 128, 256) with ragged lengths, empty docs and odd
doc counts, and checks every score against the float64 oracle (1e-2 absolute,
the fp16 bar).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flash_maxsim_amd as fm
from conftest import sim, to_np32

pytestmark = pytest.mark.gpu

ATOL = 1e-2
DEV = "cuda"


def _check(out: torch.Tensor, ref: np.ndarray):
    got = out.detach().double().cpu().numpy().reshape(ref.shape)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin)
    np.testing.assert_array_equal(got[~fin], ref[~fin])
    if fin.any():
        assert np.abs(got[fin] - ref[fin]).max() <= ATOL


def _shapes(n: int, seed: int):
    rng = np.random.default_rng(seed)
    lqs = [1, 16, 32, 33, 48, 64, 65, 96, 128, 129]
    lds = [1, 16, 64, 96, 97, 160, 161, 256, 257]
    ds = [64, 96, 128, 256]
    bs = [1, 2, 5, 33]
    return [(int(rng.choice(lqs)), int(rng.choice(lds)), int(rng.choice(ds)), int(rng.choice(bs)), i)
            for i in range(n)]


@pytest.mark.parametrize("Lq, Ld, d, B, i", _shapes(24, 7))
def test_single_query_routes(oracle_mod, Lq, Ld, d, B, i):
    dtype = torch.bfloat16 if i % 3 == 0 else torch.float16
    Q = sim((Lq, d), 600 + i, dtype)
    D = sim((B, Ld, d), 700 + i, dtype)
    g = torch.Generator().manual_seed(800 + i)
    lengths = torch.randint(0, Ld + 2, (B,), generator=g, dtype=torch.int32)
    if B > 2:
        lengths[1] = 0
    out = fm.flash_maxsim(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    _check(out, oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0])


@pytest.mark.parametrize("Lq, Ld, d, B, i", _shapes(12, 11))
def test_per_query_doc_routes(oracle_mod, Lq, Ld, d, B, i):
    Nq = 3
    Q = sim((Nq, Lq, d), 900 + i)
    D = sim((Nq, B, Ld, d), 1000 + i)
    g = torch.Generator().manual_seed(1100 + i)
    lengths = torch.randint(0, Ld + 2, (Nq * B,), generator=g, dtype=torch.int32)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV), shared_docs=False)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D.reshape(Nq * B, Ld, d)), lengths.numpy(), shared_docs=False)
    _check(out, ref)


@pytest.mark.parametrize("Lq, Ld, d, B", [(32, 77, 128, 9), (64, 128, 128, 6), (32, 129, 128, 7),
                                          (32, 200, 128, 5), (16, 64, 96, 8), (48, 100, 128, 11)])
def test_int8_doc_length_routes(oracle_mod, Lq, Ld, d, B):
    # uint8 docs of up to 128 tokens run a two-tile ring, longer ones the
    # four-tile ring with group scale loads (aligned rows) or per-tile loads.
    seed = 1200 + Lq + Ld
    Q = sim((Lq, d), seed)
    x = sim((B, Ld, d), seed + 1, torch.float32)
    codes, s, m = fm.quantize_int8(x)
    lengths = torch.randint(0, Ld + 2, (B,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)
    lengths[0] = Ld
    if B > 3:
        lengths[2] = 0
    out = fm.flash_maxsim_int8(Q.to(DEV), codes.to(DEV), s.to(DEV), m.to(DEV), lengths.to(DEV))
    _check(out, oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(s), to_np32(m), lengths.numpy()))
