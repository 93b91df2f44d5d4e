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
    # k above 1024: bitonic sort of the selection; full sorts; several levels
    (2, 5000, 1025), (1, 8192, 8192), (3, 3000, 3000), (2, 40000, 5000), (1, 100000, 8192),
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


def small_row_scores(kind, seed, shape, k):
    """Rows for the 512-thread selection of up to 8192 scores with k <= 128,
    which works on the raw floats and falls back to the exact path for NaN,
    a bound at -inf, or equal values inside the top k."""
    g = np.random.default_rng(seed)
    s = g.standard_normal(shape).astype(np.float32)
    B = shape[-1]
    rows = s.reshape(-1, B)
    if kind == "neg_zero_top":      # the best score is -0.0 (its bits must survive), the rest negative
        rows[:] = -np.abs(rows) - 1e-3
        rows[:, B // 2] = -0.0
    elif kind == "zero_at_k":       # k - 1 positive scores, then +0 and -0 below them
        rows[:] = -np.abs(rows) - 1.0
        top = g.permutation(B)[: k + 1]
        rows[:, top[: k - 1]] = np.arange(1, k, dtype=np.float32)[None, :]
        rows[:, top[k - 1]] = 0.0
        if k < B:
            rows[:, top[k]] = -0.0
    elif kind == "inf_top":         # one +inf (taken as the largest float inside the fast path)
        rows[:, B // 3] = np.inf
    elif kind == "two_inf":         # equal values inside the top k: the exact path
        rows[:, B // 3] = np.inf
        rows[:, (2 * B) // 3] = np.inf
    elif kind == "neg_inf_heavy":   # most docs empty: the bound reaches -inf
        rows[:, : (B * 19) // 20] = -np.inf
    elif kind == "denormal":        # subnormal scores
        rows[:] = rows * np.float32(1e-39)
    elif kind == "ties_outside":    # exact ties everywhere below a distinct top k
        rows[:] = np.round(rows * 4) / 4 - 10.0
        top = g.permutation(B)[:k]
        rows[:, top] = 10.0 + np.arange(k, dtype=np.float32)[None, :] * 0.5
    elif kind == "ties_inside":     # exact ties inside the top k: the exact path
        rows[:] = np.round(rows * 4) / 4
    elif kind == "nan":             # a NaN ranks first: the exact path
        rows[:, B // 5] = np.nan
    return s


@pytest.mark.parametrize("kind", ["normal", "neg_zero_top", "zero_at_k", "inf_top", "two_inf",
                                  "neg_inf_heavy", "denormal", "ties_outside", "ties_inside", "nan"])
@pytest.mark.parametrize("Nq, B, k", [
    (1, 5000, 100), (3, 5000, 128), (1, 1, 1), (1, 7, 7), (2, 300, 10), (1, 511, 64), (1, 512, 128),
    (1, 4096, 1), (1, 4097, 33), (2, 5120, 128), (1, 6144, 100), (1, 8192, 128),
])
def test_topk_small_rows(oracle_mod, kind, Nq, B, k):
    """Rows of up to 8192 scores with k <= 128 (the selection after a
    single-query scoring call): exactly the oracle's selection, value bits
    included, whichever path each row takes."""
    s = small_row_scores(kind, 7 * B + k, (Nq, B), k)
    got = fm.topk_scores(torch.from_numpy(s).to(DEV), k)
    assert_same_selection(got, oracle_mod.topk(s, k))


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


# ------------------------------------ one-call scoring + selection ----

def _topk_inputs(B, Lq, d, dtype, seed):
    """Docs with exact ties (copies of doc 3), a NaN doc and empty docs."""
    Q = sim((Lq, d), seed, dtype)
    D = sim((B, 24, d), seed + 1, dtype)
    if B > 12:
        D[5::9] = D[3]                   # identical docs: equal scores, smaller index first
        D[11, 0, 0] = float("nan")       # a NaN score ranks first
    lengths = torch.randint(1, 25, (B,), generator=torch.Generator().manual_seed(seed), dtype=torch.int32)
    if B > 12:
        lengths[5::9] = lengths[3]
        lengths[11] = 24
        lengths[7::13] = 0               # empty docs score -inf
    return Q.to(DEV), D.to(DEV), lengths.to(DEV)


@pytest.mark.parametrize("B, k, Lq, d, dtype", [
    (1, 1, 32, 128, torch.float16),
    (2, 2, 32, 128, torch.float16),      # k == B
    (255, 17, 32, 128, torch.float16),
    (257, 128, 16, 64, torch.float16),
    (5000, 100, 32, 128, torch.float16),  # config 1 + top-100
    (8192, 128, 32, 128, torch.float16),
    (4000, 50, 64, 256, torch.bfloat16),  # d = 256 in one pass
    (20000, 100, 32, 128, torch.float16),  # two selection levels
    (3000, 700, 32, 128, torch.float16),   # large k
    (2000, 30, 65, 256, torch.float16),    # two streaming passes (workspace)
    (1000, 40, 200, 128, torch.float16),   # tiled kernel
    (5000, 3000, 32, 128, torch.float16),  # k above 1024
])
def test_one_call_topk_equals_selection_of_scores(oracle_mod, B, k, Lq, d, dtype):
    """flash_maxsim_topk (fmx_fwd_topk) returns exactly the oracle's selection
    over flash_maxsim's scores (the same kernel, bit-identical scores), call
    after call."""
    Q, D, L = _topk_inputs(B, Lq, d, dtype, B + k + Lq)
    s = fm.flash_maxsim(Q, D, L)
    want = oracle_mod.topk(s.cpu().numpy(), k)
    for _ in range(3):
        assert_same_selection(fm.flash_maxsim_topk(Q, D, k, L), want)
    if B > 12:
        v, i = fm.flash_maxsim_topk(Q, D, k, L)
        assert torch.isnan(v[0]) and i[0].item() == 11


def test_one_call_topk_alternating_sizes_one_stream(oracle_mod):
    """Calls of different sizes back to back on one stream."""
    cases = [(5000, 100), (300, 7), (5000, 1), (64, 64), (2047, 128), (8000, 300)]
    inputs = [_topk_inputs(B, 32, 128, torch.float16, 7 * B + k) for B, k in cases]
    wants = [oracle_mod.topk(fm.flash_maxsim(Q, D, L).cpu().numpy(), k) for (Q, D, L), (B, k) in zip(inputs, cases)]
    outs = [fm.flash_maxsim_topk(Q, D, k, L) for (Q, D, L), (B, k) in zip(inputs, cases)]
    outs += [fm.flash_maxsim_topk(Q, D, k, L) for (Q, D, L), (B, k) in zip(inputs, cases)]
    for j, got in enumerate(outs):
        assert_same_selection(got, wants[j % len(cases)])


def test_one_call_topk_graph_replays(oracle_mod):
    """Under HIP graph capture the one-call retrieval replays correctly, with
    eager work in between the replays."""
    Q, D, L = _topk_inputs(5000, 32, 128, torch.float16, 4242)
    want = oracle_mod.topk(fm.flash_maxsim(Q, D, L).cpu().numpy(), 100)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fm.flash_maxsim_topk(Q, D, 100, L)  # warm-up on the capture stream
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        v, i = fm.flash_maxsim_topk(Q, D, 100, L)
    for _ in range(3):
        g.replay()
        torch.cuda.synchronize()
        assert_same_selection((v, i), want)
        eager = fm.flash_maxsim_topk(Q, D, 100, L)  # eager work between replays
        torch.cuda.synchronize()
        assert_same_selection(eager, want)


def test_one_call_topk_many_calls(oracle_mod):
    """300 calls over four inputs, each result checked."""
    cases = [(5000, 100, 32), (8192, 128, 16), (1200, 33, 128), (3001, 5, 64)]
    inputs = [_topk_inputs(B, Lq, 128, torch.float16, 31 * B + k) for B, k, Lq in cases]
    wants = []
    for (Q, D, L), (B, k, Lq) in zip(inputs, cases):
        v, i = oracle_mod.topk(fm.flash_maxsim(Q, D, L).cpu().numpy(), k)
        wants.append((torch.from_numpy(np.asarray(v)).to(DEV), torch.from_numpy(np.asarray(i)).to(DEV)))
    bad = 0
    for n in range(300):
        j = n % len(cases)
        Q, D, L = inputs[j]
        v, i = fm.flash_maxsim_topk(Q, D, cases[j][1], L)
        wv, wi = wants[j]
        same = torch.equal(i, wi) and torch.equal(v.view(torch.int32), wv.view(torch.int32))
        bad += 0 if same else 1
    assert bad == 0, f"{bad} of 300 selections differ"
