"""GPU parity at the BASELINE configs' full sizes, checked on sampled docs.

Each test runs the public API on the whole configuration (every doc scored by
the kernel and plan the benchmark uses) and checks a sample of docs, first
and last included, against the float64 CPU oracle on the same fp16 / uint8
values. Tolerances as in test_gpu_parity: scores within 1e-2, argmax exact
except at numerical ties, gradients within 1e-2 (fp16 outputs).
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


def sample_docs(B, n, seed):
    rng = np.random.default_rng(seed)
    pick = set(rng.choice(B, n - 4, replace=False).tolist()) | {0, 1, B - 2, B - 1}
    return sorted(pick)


def test_config2_full_size(oracle_mod):
    """Config 2: Q[1024,128] x D[1000,1024,128] fp16 (tiled kernel, the B = 1000
    plan), 24 docs checked."""
    Q = sim((1024, 128), 2)
    D = sim((1000, 1024, 128), 3)
    out = fm.flash_maxsim(Q.to(DEV), D.to(DEV)).cpu()
    pick = sample_docs(1000, 24, 2)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D[pick]))[0]
    assert_scores(out[pick], ref)


def _config4_docs(B):
    """Config 4's docs built on the GPU: N(0,1) rows, L2-normalised, encoded by
    quantize_int8 (the HIP encoder, bit-identical to the torch formula)."""
    g = torch.Generator(device=DEV).manual_seed(44)
    codes = torch.empty(B, 1024, 128, dtype=torch.uint8, device=DEV)
    scales = torch.empty(B, 1024, 1, dtype=torch.float16, device=DEV)
    mins = torch.empty(B, 1024, 1, dtype=torch.float16, device=DEV)
    for b0 in range(0, B, 1000):
        b1 = min(B, b0 + 1000)
        x = torch.nn.functional.normalize(torch.randn(b1 - b0, 1024, 128, generator=g, device=DEV), dim=-1)
        codes[b0:b1], scales[b0:b1], mins[b0:b1] = fm.quantize_int8(x)
    return codes, scales, mins


def test_config4_full_size(oracle_mod):
    """Config 4: uint8 docs [5000,1024,128], lengths U[32,1024], Q[32,128]; 24
    docs checked, then the first 4999 docs (an odd count: the last workgroup
    holds one doc instead of a pair) must give the same scores."""
    B = 5000
    Q = sim((32, 128), 41)
    codes, scales, mins = _config4_docs(B)
    lengths = torch.randint(32, 1025, (B,), generator=torch.Generator().manual_seed(43), dtype=torch.int32)
    Qd, ld = Q.to(DEV), lengths.to(DEV)
    out = fm.flash_maxsim_int8(Qd, codes, scales, mins, ld).cpu()
    pick = sample_docs(B, 24, 4)
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes[pick].cpu().numpy(), to_np32(scales[pick]),
                                 to_np32(mins[pick]), lengths[pick].numpy())
    assert_scores(out[pick], ref)
    odd = fm.flash_maxsim_int8(Qd, codes[:4999], scales[:4999], mins[:4999], ld[:4999]).cpu()
    assert torch.equal(odd[:4998], out[:4998])
    assert abs(float(odd[4998]) - ref[pick.index(4998)]) <= ATOL


def test_per_query_docs_bench_shape(oracle_mod):
    """shared_docs=False at Q[100,32,128] x D[100,50,300,128] (reference
    flash_maxsim.py:241-244): 3 whole queries plus 300 sampled pairs."""
    Nq, B, Lq, Ld, d = 100, 50, 32, 300, 128
    Q = sim((Nq, Lq, d), 61)
    D = sim((Nq, B, Ld, d), 62)
    lengths = torch.randint(1, Ld + 1, (Nq * B,), generator=torch.Generator().manual_seed(63), dtype=torch.int32)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV), shared_docs=False).cpu()
    assert out.shape == (Nq, B)
    Qn, Dn, ln = to_np32(Q), to_np32(D), lengths.numpy().reshape(Nq, B)
    for qi in (0, 57, Nq - 1):
        assert_scores(out[qi], oracle_mod.maxsim(Qn[qi], Dn[qi], ln[qi])[0])
    rng = np.random.default_rng(64)
    for qi, b in zip(rng.integers(0, Nq, 300), rng.integers(0, B, 300)):
        r = oracle_mod.maxsim(Qn[qi], Dn[qi, b:b + 1], ln[qi, b:b + 1])[0, 0]
        assert abs(float(out[qi, b]) - r) <= ATOL


def test_config5_train_full_checks(oracle_mod):
    """Config 5 shape Q[128,1024] x D[48,512,1024], loss = scores.sum(): scores,
    the saved argmax and dQ/dD (the split-d forward at Lq=128 x Ld=512, the
    6-chunk dQ gather at d=1024, the dD index and writer)."""
    B, Lq, Ld, d = 48, 128, 512, 1024
    Q = sim((Lq, d), 5)
    D = sim((B, Ld, d), 6)
    Qg = Q.to(DEV).requires_grad_(True)
    Dg = D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg)
    am = s.grad_fn.saved_tensors[2]  # the argmax the forward saved (freed by backward)
    s.sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    ref, am_ref, best = oracle_mod.maxsim(Qn, Dn, want_argmax=True)
    assert_scores(s, ref[0])
    assert_argmax(am, am_ref, best, Qn, Dn, d)
    dQ_ref, dD_ref = oracle_mod.bwd(Qn, Dn, am.cpu().numpy(), np.ones(B))
    np.testing.assert_allclose(Qg.grad.double().cpu().numpy(), dQ_ref, rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(Dg.grad.double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


def test_train_many_dq_chunks(oracle_mod):
    """1000 docs at d = 128: the dQ gather runs its maximum of 64 doc chunks."""
    B, Lq, Ld, d = 1000, 32, 64, 128
    Q = sim((Lq, d), 71)
    D = sim((B, Ld, d), 72)
    g = torch.linspace(-1.0, 1.0, B)
    Qg = Q.to(DEV).requires_grad_(True)
    Dg = D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg)
    am = s.grad_fn.saved_tensors[2]
    (s * g.to(DEV)).sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    ref, am_ref, best = oracle_mod.maxsim(Qn, Dn, want_argmax=True)
    assert_scores(s, ref[0])
    assert_argmax(am, am_ref, best, Qn, Dn, d)
    dQ_ref, dD_ref = oracle_mod.bwd(Qn, Dn, am.cpu().numpy(), g.numpy())
    np.testing.assert_allclose(Qg.grad.double().cpu().numpy(), dQ_ref, rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(Dg.grad.double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


def test_dequantize_int8_on_gpu_is_bitwise_cpu():
    """dequantize_int8 (reference flash_maxsim_quant.py:31-33) on GPU tensors
    equals the CPU result bit for bit (two separately rounded fp32 ops)."""
    from oracle.oracle_np import dequantize_np

    D = sim((6, 70, 96), 81, torch.float32)
    c, s, m = fm.quantize_int8(D)
    cpu = fm.dequantize_int8(c, s, m)
    gpu = fm.dequantize_int8(c.to(DEV), s.to(DEV), m.to(DEV)).cpu()
    assert gpu.dtype == torch.float32 and gpu.shape == (6, 70, 96)
    np.testing.assert_array_equal(gpu.numpy().view(np.uint32), cpu.numpy().view(np.uint32))
    np.testing.assert_array_equal(gpu.numpy().view(np.uint32),
                                  dequantize_np(c.numpy(), s.numpy(), m.numpy()).view(np.uint32))
