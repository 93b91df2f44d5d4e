"""GPU parity at d > 4096: the wide kernels (similarities of a chunk of
(query, doc) items through the workspace, then a max / argmax / sum
reduction), against the float64 oracle.

The reference pads any d to a power of two (flash_maxsim/flash_maxsim.py:8-9)
and its tests stop at d = 2048 (tests/test_flash_maxsim.py:58); these cases
cover widths past the split-d kernel's 4096 with ragged lengths (0, 1, 15, 16,
17), partial 8-wide chunks (d % 8 != 0), bf16, several queries over shared and
per-query docs, the saved argmax and both gradients of the training path,
uint8 docs with the GPU quantiser (bit-exact against the torch formula on the
CPU), packed uint8 docs, sparse scoring and the one-call top-k. Tolerances as
in test_gpu_parity.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

import flash_maxsim_amd as fm
from conftest import sim, to_np32
from test_gpu_parity import ATOL, assert_argmax, assert_scores

pytestmark = pytest.mark.gpu

DEV = "cuda"
LENS = [45, 0, 1, 15, 16, 17, 33]


@pytest.mark.parametrize("d", [4099, 4104, 5000, 8192])
def test_wide_single_query(oracle_mod, d):
    Q = sim((40, d), 2000 + d)
    D = sim((len(LENS), 45, d), 2001 + d)
    lengths = torch.tensor(LENS, dtype=torch.int32)
    out = fm.flash_maxsim(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    assert_scores(out, oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0])


@pytest.mark.parametrize("shared", [True, False])
def test_wide_batched_bf16(oracle_mod, shared):
    Nq, B, Lq, Ld, d = 3, 5, 20, 37, 4352
    Q = sim((Nq, Lq, d), 2100, torch.bfloat16)
    D = sim((B, Ld, d) if shared else (Nq, B, Ld, d), 2101, torch.bfloat16)
    rows = B if shared else Nq * B
    lengths = torch.tensor(([37, 0, 1, 16, 30] * Nq)[:rows], dtype=torch.int32)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV), shared)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D.reshape(rows, Ld, d)), lengths.numpy(), shared_docs=shared)
    assert_scores(out, ref)


def test_wide_train_argmax_and_grads(oracle_mod):
    """Scores, the argmax the forward saves and dQ / dD at d = 4160 (fp16)."""
    B, Lq, Ld, d = 5, 24, 40, 4160
    Q = sim((Lq, d), 2200)
    D = sim((B, Ld, d), 2201)
    g = torch.linspace(-1.0, 2.0, B, dtype=torch.float32)
    Qg = Q.to(DEV).requires_grad_(True)
    Dg = D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg)
    (s * g.to(DEV)).sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    ref, am_ref, best = oracle_mod.maxsim(Qn, Dn, want_argmax=True)
    assert_scores(s, ref[0])
    from flash_maxsim_amd.flash_maxsim import _launch_fwd, _prep

    _, am = _launch_fwd(_prep(Q.to(DEV), torch.float16)[None], _prep(D.to(DEV), torch.float16), None, 1, B, Lq, Ld,
                        d, True, True)
    assert_argmax(am, am_ref, best, Qn, Dn, d)
    dQ_ref, dD_ref = oracle_mod.bwd(Qn, Dn, am.cpu().numpy(), g.numpy())
    np.testing.assert_allclose(Qg.grad.double().cpu().numpy(), dQ_ref, rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(Dg.grad.double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


@pytest.mark.parametrize("d", [4100, 8192])
def test_wide_int8_and_quantiser(oracle_mod, d):
    """The GPU quantiser's wide-row kernel is bit-exact against the torch
    formula on the CPU; uint8 scoring at that width matches the oracle."""
    x = sim((len(LENS), 45, d), 2300 + d, torch.float32)
    c_gpu, s_gpu, m_gpu = fm.quantize_int8(x.to(DEV))
    codes, s, m = fm.quantize_int8(x)
    assert torch.equal(c_gpu.cpu(), codes)
    assert torch.equal(s_gpu.cpu().view(torch.int16), s.view(torch.int16))
    assert torch.equal(m_gpu.cpu().view(torch.int16), m.view(torch.int16))
    Q = sim((33, d), 2310 + d)
    lengths = torch.tensor(LENS, dtype=torch.int32)
    out = fm.flash_maxsim_int8(Q.to(DEV), c_gpu, s_gpu, m_gpu, lengths.to(DEV))
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(s), to_np32(m), lengths.numpy())
    assert_scores(out, ref)


def test_wide_int8_packed(oracle_mod):
    d = 4608
    x = sim((len(LENS), 45, d), 2400, torch.float32)
    lengths = torch.tensor(LENS, dtype=torch.int32)
    packed = fm.quantize_int8_packed(x.to(DEV), lengths.to(DEV))
    Q = sim((17, d), 2401)
    out = fm.flash_maxsim_int8_packed(Q.to(DEV), packed)
    codes, s, m = fm.quantize_int8(x)
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(s), to_np32(m), lengths.numpy())
    assert_scores(out, ref)


def test_wide_sparse(oracle_mod):
    d, K = 5120, 12
    Q = sim((32, d), 2500)
    D = sim((6, 50, d), 2501)
    idx = torch.stack([torch.randperm(32, generator=torch.Generator().manual_seed(2502 + b))[:K]
                       for b in range(6)]).to(torch.int32)
    out = fm.flash_maxsim_sparse(Q.to(DEV), D.to(DEV), idx.to(DEV))
    assert_scores(out, oracle_mod.maxsim(to_np32(Q), to_np32(D), qidx=idx.numpy())[0])


def test_wide_topk(oracle_mod):
    d, B, k = 4224, 40, 7
    Q = sim((16, d), 2600)
    D = sim((B, 30, d), 2601)
    lengths = torch.randint(0, 31, (B,), generator=torch.Generator().manual_seed(2602), dtype=torch.int32)
    vals, idx = fm.flash_maxsim_topk(Q.to(DEV), D.to(DEV), k, lengths.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0]
    scores = fm.flash_maxsim(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    assert_scores(scores, ref)
    want_v, want_i = torch.topk(scores.cpu(), k)
    assert torch.equal(vals.cpu(), want_v) and torch.equal(idx.cpu(), want_i)
