"""Hand-derived fixtures (tests/golden/) through the HIP kernels, bit for bit.

The basis, ties and NaN fixtures hold fp16-exact inputs whose scores and
argmax follow by hand (tests/golden/make_golden.py). Every similarity is a
small multiple of 1/16, so the fp32 GPU results must equal the fixtures
exactly, and the saved argmax must be the first occurrence at exact ties and
the first NaN where a NaN similarity is read (torch.max's rule, reference
flash_maxsim.py:301). Each fixture runs through the three forward kernel
families:
  stream  the fixture as it is (d <= 256, at most 128 query tokens);
  splitd  d zero-padded to 512 (the split-d kernel);
  tiled   the query tokens repeated to 320 rows (the tiled kernel).
Zero padding and query repetition leave every similarity and argmax unchanged;
repeated query tokens repeat the argmax columns and scale the score.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

import flash_maxsim_amd as fm

pytestmark = pytest.mark.gpu

DEV = "cuda"
GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return dict(np.load(GOLDEN / f"{name}.npz"))


def variant(Q, D, scores, argmax, route):
    """(Q, D, scores, argmax) of a fixture rewritten for a kernel route."""
    if route == "splitd":
        d = Q.shape[1]
        Qp = np.zeros((Q.shape[0], 512), np.float32)
        Dp = np.zeros(D.shape[:2] + (512,), np.float32)
        Qp[:, :d], Dp[..., :d] = Q, D
        return Qp, Dp, scores, argmax
    if route == "tiled":
        reps = -(-320 // Q.shape[0])
        Qt = np.tile(Q, (reps, 1))
        return Qt, D, scores * reps, np.tile(argmax, (1, reps))
    return Q, D, scores, argmax


def cases():
    out = []
    for name in ("basis", "ties", "nan"):
        f = load(name)
        out.append((name, f["Q"], f["D"], f["lengths"], f["scores"], f["argmax"]))
        if name == "nan":
            out.append(("nan_query", f["Qnan"], f["D"], f["lengths"], f["scores_qnan"], f["argmax_qnan"]))
    return out


CASES = cases()


def assert_exact(got: torch.Tensor, want: np.ndarray):
    g = got.detach().double().cpu().numpy().reshape(want.shape)
    np.testing.assert_array_equal(g, want)  # NaN == NaN, -inf == -inf, numbers bit-exact


@pytest.mark.parametrize("route", ["stream", "splitd", "tiled"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_golden_forward_exact(case, route, dtype):
    _, Q, D, lengths, scores, _ = case
    Q, D, scores, _ = variant(Q, D, scores, case[5], route)
    L = torch.from_numpy(lengths).to(DEV)
    out = fm.flash_maxsim(torch.from_numpy(Q).to(dtype).to(DEV), torch.from_numpy(D).to(dtype).to(DEV), L)
    assert_exact(out, scores)


@pytest.mark.parametrize("route", ["stream", "splitd", "tiled"])
@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_golden_train_argmax_and_grads_exact(oracle_mod, case, route):
    """flash_maxsim_train with doc lengths: scores, the argmax its forward saved
    (first occurrence, first NaN) and dQ/dD, all exact."""
    name, Q, D, lengths, scores, argmax = case
    Q, D, scores, argmax = variant(Q, D, scores, argmax, route)
    Qg = torch.from_numpy(Q).half().to(DEV).requires_grad_(True)
    Dg = torch.from_numpy(D).half().to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg, torch.from_numpy(lengths).to(DEV))
    assert_exact(s, scores)
    am = s.grad_fn.saved_tensors[2]  # the argmax the forward saved for backward
    valid = lengths > 0  # an empty doc's argmax row is 0 and takes no part
    np.testing.assert_array_equal(am.cpu().numpy()[valid], argmax[valid])
    np.testing.assert_array_equal(am.cpu().numpy()[~valid], 0)
    if "nan" in name:
        return  # gradients through NaN similarities are NaN-laden by definition
    g = torch.linspace(-1.0, 2.0, D.shape[0])
    (s * g.to(DEV)).sum().backward()
    gw = np.where(valid, g.numpy(), 0.0)  # empty docs give and get no gradient
    dQ_ref, dD_ref = oracle_mod.bwd(Q, D, argmax, gw)
    np.testing.assert_array_equal(Qg.grad.double().cpu().numpy(), dQ_ref)
    np.testing.assert_array_equal(Dg.grad.double().cpu().numpy(), dD_ref)


def test_nan_random_docs_all_routes(oracle_mod):
    """Random docs with NaN tokens (inside and past the doc lengths) and a
    NaN query token, scored by every forward kernel against the oracle."""
    from conftest import sim, to_np32

    g = torch.Generator().manual_seed(77)
    for Lq, d in ((32, 128), (32, 512), (300, 128)):
        Q = sim((Lq, d), 78 + d)
        D = sim((12, 90, d), 79 + d)
        lengths = torch.randint(0, 91, (12,), generator=g, dtype=torch.int32)
        lengths[:3] = torch.tensor([90, 50, 0], dtype=torch.int32)
        D[0, 40, 3] = float("nan")       # inside doc 0
        D[1, 70, 0] = float("nan")       # past doc 1's length: masked
        D[2, 0, 0] = float("nan")        # empty doc
        D[5, 10, d - 1] = float("nan")
        Qn = Q.clone()
        Qn[Lq - 1, 1] = float("nan")     # a query token NaN against every doc token
        for Qv in (Q, Qn):
            out = fm.flash_maxsim(Qv.to(DEV), D.to(DEV), lengths.to(DEV)).cpu().double().numpy()
            ref, am_ref, _ = oracle_mod.maxsim(to_np32(Qv), to_np32(D), lengths.numpy(), want_argmax=True)
            ref = ref[0]
            np.testing.assert_array_equal(np.isnan(out), np.isnan(ref))
            np.testing.assert_array_equal(np.isinf(out), np.isinf(ref))
            fin = np.isfinite(ref)
            if fin.any():  # (a NaN query token leaves no finite score)
                assert np.abs(out[fin] - ref[fin]).max() <= 1e-2
            # training forward: NaN rows of the saved argmax are the first NaN
            s = fm.flash_maxsim_train(Qv.to(DEV).requires_grad_(True), D.to(DEV), lengths.to(DEV))
            np.testing.assert_array_equal(np.isnan(s.detach().cpu().numpy()), np.isnan(ref))
            am = s.grad_fn.saved_tensors[2].cpu().numpy()
            _, _, best = oracle_mod.maxsim(to_np32(Qv), to_np32(D), lengths.numpy(), want_argmax=True)
            nanrow = np.isnan(best)
            np.testing.assert_array_equal(am[nanrow], am_ref[nanrow])
