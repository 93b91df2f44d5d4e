"""GPU parity of the top-k selection kernel and the fused retrieval calls.

topk_scores must return exactly the oracle's selection (oracle.topk: values
descending, NaN first, ties to the smaller index) on the same fp32 scores:
value bits and indices equal. Sizes cover one chunk, chunk boundaries and
several selection levels; k covers both chunk sizes (k <= 512 sorts 2048 keys
per workgroup, larger k 4096).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flash_maxsim_amd as fm
from conftest import sim, to_np32

pytestmark = pytest.mark.gpu

DEV = "cuda"


def scores_with_ties(seed, shape):
    g = np.random.default_rng(seed)
    s = g.standard_normal(shape).astype(np.float32)
    s[..., ::5] = np.round(s[..., ::5] * 4) / 4    # many exact ties
    flat = s.reshape(-1)
    flat[g.integers(0, flat.size, 4)] = np.nan
    flat[g.integers(0, flat.size, 4)] = -np.inf
    flat[g.integers(0, flat.size, 2)] = np.inf
    return s


def assert_same_selection(got, want):
    (gv, gi), (wv, wi) = got, want
    np.testing.assert_array_equal(gv.cpu().numpy().view(np.int32), np.asarray(wv).view(np.int32))
    np.testing.assert_array_equal(gi.cpu().numpy(), wi)


@pytest.mark.parametrize("Nq, B, k", [
    (1, 1, 1), (1, 10, 10), (1, 2048, 100), (1, 2049, 100), (3, 5000, 10), (2, 5000, 512),
    (2, 5000, 513), (1, 4097, 1024), (4, 100000, 64), (1, 300000, 1000), (100, 5000, 100),
])
def test_topk_matches_oracle(oracle_mod, Nq, B, k):
    s = scores_with_ties(B + k, (Nq, B))
    got = fm.topk_scores(torch.from_numpy(s).to(DEV), k)
    assert_same_selection(got, oracle_mod.topk(s, k))


def test_topk_one_dim_and_strided_rows(oracle_mod):
    s = scores_with_ties(9, (6, 3000))
    t = torch.from_numpy(s).to(DEV)
    assert_same_selection(fm.topk_scores(t[2], 50), oracle_mod.topk(s[2], 50))
    assert_same_selection(fm.topk_scores(t[::2, 100:], 20), oracle_mod.topk(s[::2, 100:], 20))
    v, i = fm.topk_scores(t, 0)
    assert v.shape == (6, 0) and i.shape == (6, 0)
    with pytest.raises(ValueError):
        fm.topk_scores(t, 3001)


def test_topk_all_equal_and_all_nan(oracle_mod):
    s = np.full((2, 4500), 0.5, np.float32)
    s[1] = np.nan
    got = fm.topk_scores(torch.from_numpy(s).to(DEV), 300)
    assert_same_selection(got, oracle_mod.topk(s, 300))
    assert got[1][0].tolist() == list(range(300))


def test_fused_retrieval_calls(oracle_mod):
    Q = sim((32, 128), 990)
    Qb = sim((5, 32, 128), 991)
    D = sim((3000, 40, 128), 992)
    lengths = torch.randint(0, 41, (3000,), generator=torch.Generator().manual_seed(1), dtype=torch.int32)
    v, i = fm.flash_maxsim_topk(Q.to(DEV), D.to(DEV), 25, lengths.to(DEV))
    s = fm.flash_maxsim(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    assert_same_selection((v, i), oracle_mod.topk(s.cpu().numpy(), 25))
    # the selected docs are the oracle's best docs up to near-ties of the scores
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0]
    assert np.abs(np.sort(ref)[::-1][:25] - v.double().cpu().numpy()).max() <= 1e-2
    vb, ib = fm.flash_maxsim_batched_topk(Qb.to(DEV), D.to(DEV), 7, lengths.to(DEV))
    sb = fm.flash_maxsim_batched(Qb.to(DEV), D.to(DEV), lengths.to(DEV))
    assert_same_selection((vb, ib), oracle_mod.topk(sb.cpu().numpy(), 7))
    x = sim((3000, 40, 128), 993, torch.float32).to(DEV)
    codes, sc, mn = fm.quantize_int8(x)
    vi, ii = fm.flash_maxsim_int8_topk(Q.to(DEV), codes, sc, mn, 9, lengths.to(DEV))
    si = fm.flash_maxsim_int8(Q.to(DEV), codes, sc, mn, lengths.to(DEV))
    assert_same_selection((vi, ii), oracle_mod.topk(si.cpu().numpy(), 9))
