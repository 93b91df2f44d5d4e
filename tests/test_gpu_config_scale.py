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


def test_u8_lds_ring_and_vgpr_ring_agree(oracle_mod):
    """uint8 docs of a 32-token query at d = 128 stream through the LDS ring
    from 2^28 code bytes (docs x Ld x d) and through the VGPR ring below; both
    feed the MFMAs the same fragments in the same order (and a 128-token query
    reads the codes with the non-temporal policy from that size). 2200 docs of 1024
    tokens (288 MB: LDS ring) must score bit-identically to the same docs in
    batches of 1000 (131 MB: VGPR ring), with empty, one-token, tile-edge and
    full-length docs on both sides of a pair; sampled docs against the oracle."""
    B = 2200
    Q = sim((32, 128), 45)
    codes, scales, mins = _config4_docs(B)
    lengths = torch.randint(0, 1025, (B,), generator=torch.Generator().manual_seed(46), dtype=torch.int32)
    edge = {0: 0, 1: 1, 2: 15, 3: 16, 4: 17, 5: 1024, 998: 0, 999: 1024, 1000: 1, 1001: 0, 2198: 33, 2199: 1023}
    for b, n in edge.items():
        lengths[b] = n
    Qd, ld = Q.to(DEV), lengths.to(DEV)
    whole = fm.flash_maxsim_int8(Qd, codes, scales, mins, ld).cpu()
    parts = torch.cat([fm.flash_maxsim_int8(Qd, codes[b0:b0 + 1000], scales[b0:b0 + 1000], mins[b0:b0 + 1000],
                                            ld[b0:b0 + 1000]).cpu() for b0 in range(0, B, 1000)])
    assert torch.equal(whole, parts)
    pick = sorted(set(sample_docs(B, 16, 5)) | set(edge))
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes[pick].cpu().numpy(), to_np32(scales[pick]),
                                 to_np32(mins[pick]), lengths[pick].numpy())
    assert_scores(whole[pick], ref)
    # a 128-token query on the shared-tile kernel, whose code loads take the
    # non-temporal policy from the same size: both policies, same scores
    Q2 = sim((128, 128), 47).to(DEV)
    whole2 = fm.flash_maxsim_int8(Q2, codes, scales, mins, ld).cpu()
    parts2 = torch.cat([fm.flash_maxsim_int8(Q2, codes[b0:b0 + 1000], scales[b0:b0 + 1000], mins[b0:b0 + 1000],
                                             ld[b0:b0 + 1000]).cpu() for b0 in range(0, B, 1000)])
    assert torch.equal(whole2, parts2)


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


def _config5_docs(B, Ld, d, seed):
    """Config 5's docs built on the GPU from a seeded generator: N(0,1) rows,
    L2-normalised, fp16 (the reference recipe, tests/test_flash_maxsim.py:6-9)."""
    g = torch.Generator(device=DEV).manual_seed(seed)
    D = torch.empty(B, Ld, d, dtype=torch.float16, device=DEV)
    for b0 in range(0, B, 250):
        b1 = min(B, b0 + 250)
        D[b0:b1] = torch.nn.functional.normalize(torch.randn(b1 - b0, Ld, d, generator=g, device=DEV), dim=-1)
    return D


def test_config5_full_size(oracle_mod):
    """Config 5 at its workload size: flash_maxsim_train on Q[128,1024] x
    D[1000,512,1024] fp16, loss = scores.sum() (reference
    flash_maxsim.py:253-291, benchmarks/bench.py:110-122). The split-d forward
    runs persistent here (one workgroup per CU walks docs b, b + G, ...), so
    the sampled docs include the first and last of each walk step at 256
    resident workgroups. Scores and the saved argmax on the sample; dQ over
    all 1000 docs from the GPU's argmax (dQ-only oracle); dD on the sample."""
    B, Lq, Ld, d = 1000, 128, 512, 1024
    Q = sim((Lq, d), 51)
    D = _config5_docs(B, Ld, d, 52)
    Qg = Q.to(DEV).requires_grad_(True)
    Dg = D.requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg)
    am = s.grad_fn.saved_tensors[2]  # [B, Lq] int32, kept alive past backward
    s.sum().backward()
    torch.cuda.synchronize()
    pick = sorted(set(sample_docs(B, 16, 5)) | {0, 255, 256, 511, 512, 767, 768, 999})
    Qn = to_np32(Q)
    Dp = to_np32(D[pick])
    ref, am_ref, best = oracle_mod.maxsim(Qn, Dp, want_argmax=True)
    assert_scores(s[pick], ref[0])
    am_all = am.cpu().numpy()
    assert_argmax(torch.from_numpy(am_all[pick]), am_ref, best, Qn, Dp, d)
    assert am_all.min() >= 0 and am_all.max() < Ld
    # dQ over every doc: sum of the oracle's dQ over chunks of docs (additive in b)
    dQ_ref = np.zeros((Lq, d))
    for b0 in range(0, B, 100):
        part, _ = oracle_mod.bwd(Qn, to_np32(D[b0:b0 + 100]), am_all[b0:b0 + 100], np.ones(100), want_dD=False)
        dQ_ref += part
    np.testing.assert_allclose(Qg.grad.double().cpu().numpy(), dQ_ref, rtol=2e-3, atol=ATOL)
    _, dD_ref = oracle_mod.bwd(Qn, Dp, am_all[pick], np.ones(len(pick)))
    np.testing.assert_allclose(Dg.grad[pick].double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


@pytest.mark.parametrize("Lq, d, B, dtype, with_argmax", [
    (128, 1024, 600, torch.float16, True),    # 132 KB of LDS: one workgroup per CU, up to 3 docs each
    (128, 1024, 600, torch.float16, False),
    (64, 512, 1300, torch.float16, True),     # 64 KB: two per CU, up to 3 docs each
    (64, 512, 1300, torch.bfloat16, False),
    (100, 1024, 700, torch.float16, False),   # masked query rows
    (64, 768, 1300, torch.float16, True),     # masked k (24 of 32 k-steps per slice set)
])
def test_splitd_persistent_walk(oracle_mod, Lq, d, B, dtype, with_argmax):
    """The split-d kernel's persistent form (one query in one pass of 64 rows
    or more) with more docs than resident workgroups: each workgroup scores
    several docs in turn, reusing its LDS row maxima and argmax, with empty
    docs and tile-edge lengths in the later steps of the walk. Every doc is
    checked against the oracle."""
    Ld = 40
    Q = sim((Lq, d), 2000 + Lq + d, dtype)
    D = sim((B, Ld, d), 2001 + B, dtype)
    lengths = torch.randint(1, Ld + 1, (B,), generator=torch.Generator().manual_seed(B + d), dtype=torch.int32)
    for b, n in ((0, Ld), (255, 0), (256, 16), (257, 0), (300, 1), (511, 17), (512, 0), (513, Ld),
                 (B - 2, 0), (B - 1, 15)):
        lengths[b] = n
    Qn, Dn, ln = to_np32(Q), to_np32(D), lengths.numpy()
    if with_argmax:
        from flash_maxsim_amd.flash_maxsim import _launch_fwd, _prep

        out, am = _launch_fwd(_prep(Q.to(DEV), dtype)[None], _prep(D.to(DEV), dtype), lengths.to(DEV), 1, B, Lq,
                              Ld, d, True, True)
        ref, am_ref, best = oracle_mod.maxsim(Qn, Dn, ln, want_argmax=True)
        assert_scores(out[0], ref[0])
        assert_argmax(am, am_ref, best, Qn, Dn, d, ln)
    else:
        out = fm.flash_maxsim(Q.to(DEV), D.to(DEV), lengths.to(DEV))
        assert_scores(out, oracle_mod.maxsim(Qn, Dn, ln)[0])


def test_splitd_persistent_walk_int8(oracle_mod):
    """uint8 docs on the persistent split-d form: 64 query rows at d = 512 over
    1300 docs (several docs per resident workgroup)."""
    B, Lq, Ld, d = 1300, 64, 40, 512
    Q = sim((Lq, d), 2101)
    x = sim((B, Ld, d), 2102, torch.float32)
    codes, sc, mn = fm.quantize_int8(x)
    lengths = torch.randint(0, Ld + 1, (B,), generator=torch.Generator().manual_seed(2103), dtype=torch.int32)
    lengths[600], lengths[1299] = 0, Ld
    out = fm.flash_maxsim_int8(Q.to(DEV), codes.to(DEV), sc.to(DEV), mn.to(DEV), lengths.to(DEV))
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(sc), to_np32(mn), lengths.numpy())
    assert_scores(out, ref)


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
