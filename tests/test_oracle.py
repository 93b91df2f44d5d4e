"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

The reference holds no golden vectors for this path, so the oracle is pinned
by (1) hand-derived fixtures in tests/golden/, (2) agreement of two
independent restatements (C in oracle/maxsim_oracle.c, NumPy in
oracle/oracle_np.py), (3) torch on the CPU (maxsim_naive, quantize_int8 and
autograd, which compute the same definitions through other code), and
(4) planted mistakes: broken variants of the NumPy restatement must fail the
pins, so each pin is shown to discriminate.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from conftest import sim, to_np32
from oracle import oracle_np

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz"))


# ---------------------------------------------------------------- golden ----

@pytest.mark.parametrize("name", ["basis", "ties"])
def test_golden_scores_and_argmax(oracle_mod, name):
    f = load(name)
    for impl in ("c", "np"):
        if impl == "c":
            s, am, _ = oracle_mod.maxsim(f["Q"], f["D"], f["lengths"], want_argmax=True)
        else:
            s, am, _ = oracle_np.maxsim_np(f["Q"], f["D"], f["lengths"])
        np.testing.assert_array_equal(s[0], f["scores"], err_msg=impl)
        valid = np.isfinite(f["scores"])
        np.testing.assert_array_equal(am[valid], f["argmax"][valid], err_msg=impl)


def _nan_pins_hold(maxsim_fn) -> bool:
    """True iff maxsim_fn (Q, D, lengths) -> (scores, argmax) reproduces the
    hand-derived NaN fixture: NaN scores where a NaN similarity is read, the
    first NaN's index as argmax, a NaN past a doc's length masked."""
    f = load("nan")
    for qk, sk, ak in (("Q", "scores", "argmax"), ("Qnan", "scores_qnan", "argmax_qnan")):
        s, am = maxsim_fn(f[qk], f["D"], f["lengths"])
        if not np.array_equal(np.reshape(s, -1), f[sk], equal_nan=True) or not np.array_equal(am, f[ak]):
            return False
    return True


def test_golden_nan(oracle_mod):
    """NaN rule of maxsim_naive's torch.max (reference flash_maxsim.py:301) in both restatements."""
    assert _nan_pins_hold(lambda Q, D, L: oracle_mod.maxsim(Q, D, L, want_argmax=True)[:2])
    assert _nan_pins_hold(lambda Q, D, L: oracle_np.maxsim_np(Q, D, L)[:2])


def test_nan_rule_is_torch_max(oracle_mod):
    """The NaN fixture through torch on the CPU: maxsim_naive's values, and
    torch.max's indices over the same masked similarities."""
    from flash_maxsim_amd import maxsim_naive

    f = load("nan")
    L = torch.from_numpy(f["lengths"])
    for qk, sk, ak in (("Q", "scores", "argmax"), ("Qnan", "scores_qnan", "argmax_qnan")):
        Q, D = torch.from_numpy(f[qk]), torch.from_numpy(f["D"])
        np.testing.assert_array_equal(maxsim_naive(Q, D, L).double().numpy(), f[sk])
        S = torch.matmul(D, Q.t())
        S = S.masked_fill(torch.arange(D.shape[1])[None, :, None] >= L[:, None, None], float("-inf"))
        idx = S.max(dim=1).indices.numpy()
        valid = f["lengths"] > 0
        np.testing.assert_array_equal(idx[valid], f[ak][valid])


def test_nan_pins_reject_nan_skipping_max():
    """Planted mistake: a max that skips NaN (strict > from -inf, i.e. nanmax
    with its first index) must fail the NaN pins."""
    def skip_nan(Q, D, lengths):
        Q, D = np.asarray(Q, np.float64), np.asarray(D, np.float64)
        B, Ld, _ = D.shape
        scores, argmax = np.empty(B), np.zeros((B, Q.shape[0]), np.int32)
        for b in range(B):
            n = min(max(int(lengths[b]), 0), Ld)
            tot = 0.0
            for q in range(Q.shape[0]):
                m, mi = -np.inf, 0
                for j in range(n):
                    s = float(Q[q] @ D[b, j])
                    if s > m:
                        m, mi = s, j
                tot += m
                argmax[b, q] = mi
            scores[b] = tot
        return scores, argmax

    assert not _nan_pins_hold(skip_nan)


def test_golden_quant(oracle_mod):
    from flash_maxsim_amd import quantize_int8

    f = load("quant")
    c_codes, c_s, c_m, _ = oracle_mod.quantize_int8(f["D"])
    n_codes, n_s, n_m, _ = oracle_np.quantize_np(f["D"])
    t_codes, t_s, t_m = quantize_int8(torch.from_numpy(f["D"]))
    for codes, s, m in [(c_codes, c_s, c_m), (n_codes, n_s, n_m),
                        (t_codes.numpy(), t_s.numpy(), t_m.numpy())]:
        np.testing.assert_array_equal(codes, f["codes"])
        np.testing.assert_array_equal(s.view(np.uint16), f["scales"].view(np.uint16))
        np.testing.assert_array_equal(m.view(np.uint16), f["mins"].view(np.uint16))


def test_golden_bwd(oracle_mod):
    f = load("bwd")
    for dQ, dD in [oracle_mod.bwd(f["Q"], f["D"], f["argmax"], f["grad"]),
                   oracle_np.bwd_np(f["Q"], f["D"], f["argmax"], f["grad"])]:
        np.testing.assert_allclose(dQ, f["dQ"], rtol=0, atol=1e-12)
        np.testing.assert_allclose(dD, f["dD"], rtol=0, atol=1e-12)


def test_golden_random_small(oracle_mod):
    f = load("random_small")
    s, am, _ = oracle_mod.maxsim(f["Q"], f["D"], f["lengths"], want_argmax=True)
    np.testing.assert_allclose(s, f["scores"], rtol=0, atol=1e-12)
    np.testing.assert_array_equal(am, f["argmax"])
    s8 = oracle_mod.maxsim_int8(f["Q"][0], f["codes"], f["scales"], f["mins"], f["lengths"])
    np.testing.assert_allclose(s8, f["scores_int8"], rtol=0, atol=1e-12)


# ------------------------------------------- two restatements agree -----

@pytest.mark.parametrize("case", [
    dict(Nq=1, Lq=32, B=6, Ld=37, d=64, shared=True, lengths=[37, 0, 1, 16, 50, -3]),
    dict(Nq=3, Lq=7, B=4, Ld=20, d=40, shared=True, lengths=None),
    dict(Nq=2, Lq=9, B=3, Ld=11, d=24, shared=False, lengths=[11, 4, 0, 2, 9, 11]),
])
def test_c_matches_numpy(oracle_mod, case):
    Q = to_np32(sim((case["Nq"], case["Lq"], case["d"]), 1))
    Bp = case["B"] if case["shared"] else case["Nq"] * case["B"]
    D = to_np32(sim((Bp, case["Ld"], case["d"]), 2))
    s_c, am_c, best_c = oracle_mod.maxsim(Q, D, case["lengths"], shared_docs=case["shared"], want_argmax=True)
    s_n, am_n, best_n = oracle_np.maxsim_np(Q, D, case["lengths"], shared_docs=case["shared"])
    np.testing.assert_allclose(s_c, s_n, rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(best_c, best_n, rtol=1e-12, atol=1e-12)
    np.testing.assert_array_equal(am_c, am_n)


def test_sparse_c_matches_numpy(oracle_mod):
    Q = to_np32(sim((12, 32), 3))
    D = to_np32(sim((5, 19, 32), 4))
    rng = np.random.default_rng(0)
    idx = rng.integers(-2, 14, size=(5, 6)).astype(np.int32)  # includes out-of-range rows
    s_c = oracle_mod.maxsim(Q, D, qidx=idx)
    s_n, _, _ = oracle_np.maxsim_np(Q, D, qidx=idx)
    np.testing.assert_allclose(s_c, s_n, rtol=1e-12, atol=1e-12)


def test_int8_oracle_equals_dequantized(oracle_mod):
    D = to_np32(sim((4, 33, 48), 5))
    Q = to_np32(sim((9, 48), 6))
    codes, s16, m16, _ = oracle_mod.quantize_int8(D)
    lengths = np.array([33, 10, 0, 40], np.int32)
    s8 = oracle_mod.maxsim_int8(Q, codes, s16, m16, lengths)
    Dq = oracle_np.dequantize_np(codes, s16, m16)
    s_ref = oracle_mod.maxsim(Q, Dq, lengths)[0]
    np.testing.assert_array_equal(s8, s_ref)


def _nearest_fp16(vals: np.ndarray, exact: np.ndarray) -> bool:
    """True when every finite fp16 in vals is the one nearest exact (float64),
    ties to an even significand, judged against both fp16 neighbours."""
    fin = np.isfinite(vals)
    g, e = vals[fin].astype(np.float64), exact[fin]
    with np.errstate(over="ignore"):
        up = np.nextafter(vals[fin], np.float16(np.inf)).astype(np.float64)
        dn = np.nextafter(vals[fin], np.float16(-np.inf)).astype(np.float64)
    err = np.abs(g - e)
    if not (np.all(err <= np.abs(up - e)) and np.all(err <= np.abs(dn - e))):
        return False
    ties = (err == np.abs(up - e)) | (err == np.abs(dn - e))
    return bool(np.all((vals[fin].view(np.uint16)[ties] & 1) == 0))


def test_fp16_dequantisation_is_the_nearest_fp16():
    """dequantize_fp16_np returns, for every token value, the fp16 nearest to
    the exact code * scale + min; an fp16 multiply then add (two roundings, a
    plausible slip) fails the same check on these values."""
    rng = np.random.default_rng(21)
    codes = rng.integers(0, 256, size=(64, 257)).astype(np.uint8)
    scales = np.concatenate([rng.uniform(1e-4, 2e-2, 60), [6e-8, 1e-5, 3.0, 250.0]]).astype(np.float16)[:, None]
    mins = np.concatenate([rng.uniform(-1.0, 0.5, 60), [-1e-6, 0.0, -300.0, 65000.0]]).astype(np.float16)[:, None]
    got = oracle_np.dequantize_fp16_np(codes, scales, mins)
    exact = codes.astype(np.float64) * scales.astype(np.float64) + mins.astype(np.float64)
    fin = np.isfinite(got)
    assert not fin.all() and fin.mean() > 0.9  # 65000 + 255 * 250 overflows fp16
    assert np.all(np.abs(exact[~fin]) >= 65520)  # overflow only past the largest fp16 plus half an ulp
    assert _nearest_fp16(got, exact)
    with np.errstate(over="ignore"):
        two_roundings = (codes.astype(np.float16) * scales).astype(np.float16) + mins
    assert not _nearest_fp16(two_roundings, exact)


# --------------------------------------------- torch on the CPU agrees -----

def test_matches_torch_maxsim_naive(oracle_mod):
    from flash_maxsim_amd import maxsim_naive

    Q = sim((32, 128), 7)
    D = sim((20, 300, 128), 8)
    lengths = torch.randint(1, 300, (20,), generator=torch.Generator().manual_seed(9), dtype=torch.int32)
    ref = maxsim_naive(Q, D, lengths).double().numpy()
    s = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0]
    np.testing.assert_allclose(s, ref, rtol=0, atol=1e-4)


def test_f32_to_f16_matches_numpy(oracle_mod):
    rng = np.random.default_rng(1)
    bits = rng.integers(0, 2**32, size=200_000, dtype=np.uint64).astype(np.uint32)
    specials = np.array([0.0, -0.0, 1e-8, 2.0**-25, 2.0**-25 * 1.0000001, 2.0**-24, 65504.0, 65520.0,
                         65519.99, np.inf, -np.inf, 5.960464477539063e-08, 6.097555160522461e-05],
                        np.float32)
    vals = np.concatenate([bits.view(np.float32), specials])
    vals = vals[~np.isnan(vals)]
    lib = oracle_mod._load()
    got = np.array([lib.oracle_f32_to_f16(float(v)) for v in vals[:20000]], np.uint16)
    with np.errstate(over="ignore"):
        want = vals[:20000].astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(got, want)
    # the quantiser path converts whole rows: check the rest through it
    rows = vals[20000:20000 + 160000].reshape(-1, 1)
    rows = rows[np.isfinite(rows[:, 0])]
    _, _, m16, _ = oracle_mod.quantize_int8(rows)
    with np.errstate(over="ignore"):
        want = rows[:, 0].astype(np.float16).view(np.uint16)
    np.testing.assert_array_equal(m16.view(np.uint16)[:, 0], want)


@pytest.mark.parametrize("seed", [0, 1])
def test_quantize_bit_exact_vs_torch(oracle_mod, seed):
    from flash_maxsim_amd import quantize_int8

    D = sim((6, 64, 128), 10 + seed, torch.float32)
    D[0, :5] = 0.25                      # constant rows: scale floor
    D[1] *= 37.0                         # wide range
    D[2, 3, :] = torch.linspace(-1, 1, 128)
    t_codes, t_s, t_m = quantize_int8(D)
    c_codes, c_s, c_m, _ = oracle_mod.quantize_int8(D.numpy())
    np.testing.assert_array_equal(c_codes, t_codes.numpy())
    np.testing.assert_array_equal(c_s.view(np.uint16), t_s.numpy().view(np.uint16))
    np.testing.assert_array_equal(c_m.view(np.uint16), t_m.numpy().view(np.uint16))


def test_bwd_matches_autograd(oracle_mod):
    Q = sim((16, 32), 11).double()
    D = sim((6, 24, 32), 12).double()
    g = torch.linspace(-1.5, 2.0, 6, dtype=torch.float64)
    _, am, _ = oracle_mod.maxsim(Q.float().numpy(), D.float().numpy(), want_argmax=True)
    Qr, Dr = Q.clone().requires_grad_(True), D.clone().requires_grad_(True)
    S = torch.matmul(Dr, Qr.t())            # [B, Ld, Lq]
    (S.max(dim=1).values.sum(dim=1) * g).sum().backward()
    dQ, dD = oracle_mod.bwd(Q.float().numpy(), D.float().numpy(), am, g.numpy())
    np.testing.assert_allclose(dQ, Qr.grad.numpy(), rtol=0, atol=1e-6)
    np.testing.assert_allclose(dD, Dr.grad.numpy(), rtol=0, atol=1e-6)
    # dQ alone (no dD array) is the same dQ, and dQ is additive over chunks of docs
    dQ_only, none = oracle_mod.bwd(Q.float().numpy(), D.float().numpy(), am, g.numpy(), want_dD=False)
    assert none is None
    np.testing.assert_array_equal(dQ_only, dQ)
    parts = [oracle_mod.bwd(Q.float().numpy(), D[b0:b0 + 2].float().numpy(), am[b0:b0 + 2], g[b0:b0 + 2].numpy(),
                            want_dD=False)[0] for b0 in (0, 2, 4)]
    np.testing.assert_allclose(parts[0] + parts[1] + parts[2], dQ, rtol=0, atol=1e-12)


# ------------------------------------------------ planted mistakes ------

def _pins_hold(maxsim_fn) -> bool:
    """True iff maxsim_fn reproduces the basis, ties and random golden fixtures."""
    for name in ("basis", "ties", "random_small"):
        f = load(name)
        Q = f["Q"] if name != "random_small" else f["Q"]
        s, am, _ = maxsim_fn(Q, f["D"], f["lengths"])
        want = f["scores"] if name != "random_small" else f["scores"]
        if s.shape != np.shape(want) and s.reshape(-1).shape != np.reshape(want, -1).shape:
            return False
        if not np.allclose(s.reshape(-1), np.reshape(want, -1), rtol=0, atol=1e-9, equal_nan=False):
            return False
        ok = np.isfinite(np.reshape(want, (-1,)))
        if name != "random_small" and not np.array_equal(am[ok], f["argmax"][ok]):
            return False
    return True


def _mutant(kind):
    def fn(Q, D, lengths):
        Q = np.asarray(Q, np.float64)
        Q = Q[None] if Q.ndim == 2 else Q
        D = np.asarray(D, np.float64)
        Nq, Lq, _ = Q.shape
        B, Ld, _ = D.shape
        lens = np.clip(np.asarray(lengths, np.int64), 0, Ld)
        scores = np.empty((Nq, B))
        argmax = np.zeros((Nq * B, Lq), np.int32)
        pos = np.arange(Ld)
        for qi in range(Nq):
            for b in range(B):
                S = Q[qi] @ D[b].T
                lim = lens[b] + 1 if kind == "mask_off_by_one" else lens[b]
                S = np.where(pos[None, :] < lim, S, -np.inf)
                if kind == "sum_not_max":
                    S = np.where(np.isfinite(S), S, 0.0)
                    m = S.sum(axis=1)
                    am = np.zeros(Lq, np.int64)
                elif kind == "max_over_query":
                    m = S.max(axis=0)[:Lq] if Ld >= Lq else np.resize(S.max(axis=0), Lq)
                    am = np.zeros(Lq, np.int64)
                elif kind == "last_argmax":
                    m = S.max(axis=1)
                    am = Ld - 1 - np.argmax(S[:, ::-1], axis=1)
                else:
                    m = S.max(axis=1)
                    am = np.argmax(S, axis=1)
                if kind == "no_query_sum":
                    scores[qi, b] = m.max()
                else:
                    scores[qi, b] = m.sum()
                argmax[qi * B + b] = am
        return scores, argmax, None
    return fn


def test_pins_accept_the_oracles(oracle_mod):
    assert _pins_hold(lambda Q, D, L: oracle_np.maxsim_np(Q, D, L))
    assert _pins_hold(lambda Q, D, L: oracle_mod.maxsim(Q, D, L, want_argmax=True))
    assert _pins_hold(_mutant("none"))


@pytest.mark.parametrize("kind", ["sum_not_max", "max_over_query", "last_argmax", "mask_off_by_one",
                                  "no_query_sum"])
def test_pins_reject_planted_mistakes(kind):
    assert not _pins_hold(_mutant(kind)), f"pins failed to catch planted mistake {kind!r}"


def test_quant_pins_reject_round_half_away():
    f = load("quant")
    D = f["D"].astype(np.float32)
    mn = D.min(axis=-1, keepdims=True)
    s = np.maximum((D.max(axis=-1, keepdims=True) - mn) / np.float32(255.0), np.float32(1e-8))
    x = (D - mn) / s
    codes = np.clip(np.floor(x + np.float32(0.5)), 0, 255).astype(np.uint8)  # half away from zero
    assert not np.array_equal(codes, f["codes"])


def test_bwd_pins_reject_wrong_scatter():
    f = load("bwd")
    dQ, dD = oracle_np.bwd_np(f["Q"], f["D"], f["argmax"], f["grad"])
    # plant: scatter every doc's tokens into doc 0
    bad = np.zeros_like(dD)
    for b in range(dD.shape[0]):
        for q in range(f["Q"].shape[0]):
            bad[0, f["argmax"][b, q]] += f["grad"][b] * f["Q"][q]
    assert not np.allclose(bad, f["dD"])
    # plant: dQ gathers the wrong token (argmax transposed)
    badQ = np.zeros_like(dQ)
    for q in range(f["Q"].shape[0]):
        for b in range(f["D"].shape[0]):
            badQ[q] += f["grad"][b] * f["D"][b, f["argmax"][q % 2, b % 2]]
    assert not np.allclose(badQ, f["dQ"])


# ------------------------------------------------------------------ top-k ----

def _topk_scores(seed, shape):
    g = np.random.default_rng(seed)
    s = g.standard_normal(shape).astype(np.float32)
    s[..., ::7] = np.round(s[..., ::7])             # many exact ties
    s.reshape(-1)[g.integers(0, s.size, 5)] = np.nan
    s.reshape(-1)[g.integers(0, s.size, 5)] = -np.inf
    s.reshape(-1)[g.integers(0, s.size, 3)] = np.inf
    return s


@pytest.mark.parametrize("shape, k", [((50,), 10), ((3, 257), 257), ((4, 1000), 64), ((2, 31), 1)])
def test_topk_oracle_values_are_torch_topk(oracle_mod, shape, k):
    s = _topk_scores(k, shape)
    v, i = oracle_mod.topk(s, k)
    tv, ti = torch.topk(torch.from_numpy(s), k)
    np.testing.assert_array_equal(np.nan_to_num(v, nan=7e7), np.nan_to_num(tv.numpy(), nan=7e7))
    # every index points at its value; indices are distinct per row
    sv = np.take_along_axis(s.reshape(-1, shape[-1]), i.reshape(-1, k), axis=1).reshape(v.shape)
    np.testing.assert_array_equal(np.isnan(sv), np.isnan(v))
    np.testing.assert_array_equal(sv[~np.isnan(sv)], v[~np.isnan(v)])
    for row in i.reshape(-1, k):
        assert len(set(row.tolist())) == k


def test_topk_oracle_brute_force_ties(oracle_mod):
    g = np.random.default_rng(3)
    for trial in range(200):
        B = int(g.integers(1, 40))
        s = g.integers(-3, 4, B).astype(np.float32)   # dense ties
        if trial % 5 == 0:
            s[g.integers(0, B)] = np.nan
        k = int(g.integers(1, B + 1))
        want = sorted(range(B), key=lambda j: (0 if np.isnan(s[j]) else 1, 0.0 if np.isnan(s[j]) else -s[j], j))[:k]
        v, i = oracle_mod.topk(s, k)
        assert i.tolist() == want


def test_topk_oracle_planted_mistake_fails(oracle_mod):
    # a last-index tie order (as a sort that is not stable could give) must differ
    s = np.array([2.0, 5.0, 2.0, 5.0, 2.0], np.float32)
    _, i = oracle_mod.topk(s, 5)
    assert i.tolist() == [1, 3, 0, 2, 4]
    assert i.tolist() != [3, 1, 4, 2, 0]
