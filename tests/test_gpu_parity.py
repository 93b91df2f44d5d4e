"""GPU parity: libflashmaxsim's HIP kernels against the CPU oracle.

Every test draws seeded inputs on the CPU (reference recipe: randn, L2
normalise per token, cast), runs the flash_maxsim_amd API on cuda:0 (which
calls the C ABI of include/fmx.h) and compares with the float64 oracle on the
same fp16/bf16 values.

Tolerances: scores within 1e-2 absolute of the oracle (north-star bar for
fp16 inputs with fp32 accumulation). Argmax must equal the oracle's except at
numerical ties (see assert_argmax: Higham's bound for the two similarities,
and a cap on how many such ties one check may accept). Gradients (fp16
outputs) within rtol 2e-3 + atol 1e-2 of the oracle's, computed from the
GPU's accepted argmax; bf16 outputs within rtol 1e-2 + atol 2e-2, since bf16
keeps 8 significant bits (half an ulp is 2^-8 = 3.9e-3 relative).
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


U32 = 2.0**-24          # unit roundoff of fp32
MFMA_MARGIN = 2.0       # the MFMA's internal rounding of its 32-term sums is not specified as
                        # round-to-nearest: 2 allows a directed rounding at every step
TIE_RATE = 5e-5         # accepted ties per (doc, query token) pair: about 5x the expected rate
                        # of near-tie flips for random unit-norm rows at d = 1024 (~1e-5)
TIE_FLOOR = 2           # ...but at least this many in one check


def gamma(d: int) -> float:
    """Higham's gamma_d = d*u / (1 - d*u): a d-term fp32 sum in any order is
    within gamma_d * sum|terms| of the exact sum."""
    return d * U32 / (1.0 - d * U32)


def tie_tol(d: int, a_gpu: float, a_ref: float) -> float:
    """Largest exact gap S(j_ref) - S(j_gpu) at which the GPU's fp32
    similarities can still rank j_gpu first: the two fp32 sums are each within
    gamma_d * sum_k |Q_qk D_jk| (a_gpu, a_ref) of their exact values."""
    return MFMA_MARGIN * gamma(d) * (a_gpu + a_ref)


def assert_scores(gpu: torch.Tensor, ref: np.ndarray, atol: float = ATOL):
    got = gpu.detach().double().cpu().numpy().reshape(ref.shape)
    fin = np.isfinite(ref)
    np.testing.assert_array_equal(np.isfinite(got), fin, err_msg="finite pattern differs")
    np.testing.assert_array_equal(got[~fin], ref[~fin])
    err = np.abs(got[fin] - ref[fin]).max() if fin.any() else 0.0
    assert err <= atol, f"max |gpu - oracle| = {err:.3e} > {atol}"
    return err


def assert_argmax(am_gpu: torch.Tensor, am_ref: np.ndarray, best_ref: np.ndarray, Q, D, d: int,
                  lengths=None):
    """Bit-exact except at numerical ties; returns the number of tie-accepted
    mismatches.

    A GPU index j in place of the oracle's j* is accepted only when the
    oracle's exact similarities satisfy S(j*) - S(j) <= tie_tol, and at most
    max(TIE_FLOOR, TIE_RATE * pairs) such ties are accepted per check, so an
    index bug that picks a near-max token systematically fails the count.
    """
    g = am_gpu.cpu().numpy().reshape(am_ref.shape)
    # an empty doc (every token masked, best = -inf) has no max to point at; the
    # backward ignores its indices, so only docs with tokens are compared
    bad = np.argwhere((g != am_ref) & (best_ref != -np.inf))
    Qn = np.asarray(Q, np.float64)
    Qn = Qn if Qn.ndim == 3 else Qn[None]  # [Nq, Lq, d]; items run qi * B + b over shared docs
    Dn = np.asarray(D, np.float64)
    for item, q in bad:
        j, jr = int(g[item, q]), int(am_ref[item, q])
        qi, b = divmod(int(item), Dn.shape[0])
        qv = Qn[qi, q]
        n = Dn.shape[1] if lengths is None else min(max(int(lengths[b]), 0), Dn.shape[1])
        assert 0 <= j < max(n, 1), f"argmax {j} out of range at ({item}, {q})"
        s = float(qv @ Dn[b, j])
        tol = tie_tol(d, float(np.abs(qv * Dn[b, j]).sum()), float(np.abs(qv * Dn[b, jr]).sum()))
        assert best_ref[item, q] - s <= tol, (
            f"argmax mismatch at ({item}, {q}): gpu {j} (S={s:.9f}) vs oracle {jr} "
            f"(S={best_ref[item, q]:.9f}), gap {best_ref[item, q] - s:.3e} > tie tolerance {tol:.3e}")
    allowed = max(TIE_FLOOR, int(np.ceil(TIE_RATE * g.size)))
    print(f"argmax: {len(bad)} tie-accepted of {g.size} pairs (at most {allowed})")
    assert len(bad) <= allowed, f"{len(bad)} tie-accepted argmax mismatches in {g.size} pairs > {allowed}"
    return len(bad)


def run_single(oracle_mod, B, Lq, Ld, d, seed, dtype=torch.float16, lengths=None):
    Q = sim((Lq, d), seed, dtype)
    D = sim((B, Ld, d), seed + 1, dtype)
    lt = None if lengths is None else torch.as_tensor(lengths, dtype=torch.int32)
    out = fm.flash_maxsim(Q.to(DEV), D.to(DEV), None if lt is None else lt.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths)[0]
    return out, ref


# ---------------------------------------------------------------- forward ----

def test_correctness(oracle_mod):
    """Reference test_correctness shape (tests/test_flash_maxsim.py:18-21)."""
    out, ref = run_single(oracle_mod, 50, 32, 300, 128, 100)
    assert out.shape == (50,) and out.dtype == torch.float32
    assert_scores(out, ref)


def test_variable_lengths(oracle_mod):
    """Reference test_variable_lengths (tests/test_flash_maxsim.py:24-30) plus edge lengths."""
    lengths = torch.randint(64, 256, (20,), generator=torch.Generator().manual_seed(5)).tolist()
    lengths[:8] = [0, 1, 15, 16, 17, 256, 300, -4]  # empty, tile edges, full, > Ld, negative
    out, ref = run_single(oracle_mod, 20, 32, 256, 128, 110, lengths=lengths)
    assert_scores(out, ref)
    assert torch.isinf(out[0]) and out[0] < 0 and torch.isinf(out[7])


@pytest.mark.parametrize("Lq", [1, 7, 16, 17, 33, 64, 100, 128, 129, 200, 300])
def test_query_lengths(oracle_mod, Lq):
    out, ref = run_single(oracle_mod, 12, Lq, 70, 128, 120 + Lq)
    assert_scores(out, ref)


@pytest.mark.parametrize("Lq, d, dtype", [(65, 128, torch.float16), (100, 128, torch.bfloat16),
                                          (128, 128, torch.float16), (64, 256, torch.float16),
                                          (40, 256, torch.bfloat16),
                                          # docs of up to 256 tokens: two per workgroup at any Lq
                                          (32, 128, torch.float16), (16, 128, torch.bfloat16),
                                          (1, 128, torch.float16), (48, 128, torch.float16),
                                          (20, 64, torch.float16), (8, 256, torch.bfloat16),
                                          (32, 96, torch.float16), (24, 100, torch.bfloat16)])
def test_two_docs_per_workgroup(oracle_mod, Lq, d, dtype):
    """Single queries whose query tile fills 128 VGPRs, or docs of up to 256
    tokens, score docs 2x and 2x+1 in one workgroup: odd B (the last workgroup
    holds one doc), empty docs on either side of a pair, tile edges."""
    lengths = [90, 0, 0, 90, 1, 16, 17, 89, 33, 0, 48, 64, 5]
    out, ref = run_single(oracle_mod, 13, Lq, 90, d, 400 + Lq + d, dtype=dtype, lengths=lengths)
    assert_scores(out, ref)
    assert torch.isneginf(out[1]) and torch.isneginf(out[2]) and torch.isneginf(out[9])


@pytest.mark.parametrize("Lq, dtype", [(65, torch.float16), (100, torch.bfloat16), (128, torch.float16)])
def test_two_docs_full_query_tile(oracle_mod, Lq, dtype):
    # 65-128-row queries over docs longer than 160 tokens stay on the streaming
    # kernel, two docs per workgroup (shorter docs go to the tiled kernel).
    lengths = [200, 0, 0, 200, 1, 16, 17, 199, 161, 0, 48, 64, 5]
    out, ref = run_single(oracle_mod, 13, Lq, 200, 128, 430 + Lq, dtype=dtype, lengths=lengths)
    assert_scores(out, ref)


@pytest.mark.parametrize("Lq, Ld, d", [(33, 96, 128), (64, 97, 128), (65, 160, 128), (128, 60, 96),
                                       (100, 161, 128), (48, 96, 100)])
def test_single_query_short_docs(oracle_mod, Lq, Ld, d):
    # Single queries over short docs: the tiled kernel from 33 rows over docs of
    # up to 96 tokens and from 65 rows over up to 160; the boundaries' other
    # sides stay streamed.
    B = 37
    lengths = torch.randint(0, Ld + 1, (B,), generator=torch.Generator().manual_seed(Lq + Ld), dtype=torch.int32)
    lengths[:2] = torch.tensor([Ld, 0])
    out, ref = run_single(oracle_mod, B, Lq, Ld, d, 460 + Lq, lengths=lengths.numpy())
    assert_scores(out, ref)


@pytest.mark.parametrize("Ld", [256, 257, 200, 64])
def test_two_docs_length_boundary(oracle_mod, Ld):
    # 32-token query: docs of up to 256 tokens pair up in a workgroup, longer
    # ones (257) take one each; both sides of the boundary, full and ragged
    # lengths.
    B = 41
    lengths = torch.randint(0, Ld + 1, (B,), generator=torch.Generator().manual_seed(Ld), dtype=torch.int32)
    lengths[:3] = torch.tensor([Ld, 0, Ld - 1])
    out, ref = run_single(oracle_mod, B, 32, Ld, 128, 450 + Ld, lengths=lengths.numpy())
    assert_scores(out, ref)


@pytest.mark.parametrize("d", [8, 32, 40, 64, 96, 100, 33, 160, 256])
def test_embedding_dims_stream(oracle_mod, d):
    out, ref = run_single(oracle_mod, 9, 32, 45, d, 130 + d, lengths=[45, 3, 0, 17, 44, 45, 1, 32, 33])
    assert_scores(out, ref)


@pytest.mark.parametrize("d", [256, 512, 1024, 2048, 300, 600, 1000, 2056, 3000, 4096])
def test_large_embedding_dim(oracle_mod, d):
    """Reference test_large_embedding_dim (tests/test_flash_maxsim.py:58-64) plus non-power-of-2 d."""
    out, ref = run_single(oracle_mod, 20, 32, 128, d, 140 + d)
    assert_scores(out, ref)


@pytest.mark.parametrize("Lq", [1, 48, 128, 130, 257])
def test_splitd_query_lengths_and_varlen(oracle_mod, Lq):
    lengths = [128, 0, 1, 16, 17, 127, 200, 64]
    out, ref = run_single(oracle_mod, 8, Lq, 128, 1024, 150 + Lq, lengths=lengths)
    assert_scores(out, ref)


@pytest.mark.parametrize("d", [128, 1024])
def test_bf16(oracle_mod, d):
    out, ref = run_single(oracle_mod, 16, 32, 100, d, 160 + d, dtype=torch.bfloat16,
                          lengths=[100, 50, 0, 99] * 4)
    assert_scores(out, ref)


def test_fp32_inputs_are_cast_to_fp16(oracle_mod):
    Q = sim((32, 128), 170, torch.float32)
    D = sim((10, 64, 128), 171, torch.float32)
    out = fm.flash_maxsim(Q.to(DEV), D.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q.half()), to_np32(D.half()))[0]
    assert_scores(out, ref)


def test_non_contiguous_inputs(oracle_mod):
    Q = sim((64, 128), 172)[::2]           # strided rows
    D = sim((10, 128, 64), 173).transpose(1, 2)  # [10, 64, 128] non-contiguous
    out = fm.flash_maxsim(Q.to(DEV), D.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D.contiguous()))[0]
    assert_scores(out, ref)


def test_config1_parity_size(oracle_mod):
    """BASELINE config 1 (Q[32,128], D[1000,300,128])."""
    out, ref = run_single(oracle_mod, 1000, 32, 300, 128, 1)
    assert_scores(out, ref)


def test_metric_config_full_size(oracle_mod):
    """Metric workload: Q[32,128], D[5000,300,128] fp16, checked on every doc."""
    out, ref = run_single(oracle_mod, 5000, 32, 300, 128, 11)
    assert_scores(out, ref)


# ---------------------------------------------------------------- batched ----

def test_batched_shape_and_values(oracle_mod):
    """Reference test_batched (tests/test_flash_maxsim.py:33-38), with values checked."""
    Q = sim((5, 32, 128), 200)
    D = sim((20, 300, 128), 201)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), shared_docs=True)
    assert out.shape == (5, 20)
    assert_scores(out, oracle_mod.maxsim(to_np32(Q), to_np32(D)))
    # positional call as in the reference benchmark (bench.py:103)
    out2 = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), None, True)
    assert torch.equal(out, out2)


def test_batched_varlen_and_not_shared(oracle_mod):
    Q = sim((3, 20, 64), 210)
    D = sim((3, 7, 50, 64), 211)
    lengths = torch.randint(0, 60, (21,), generator=torch.Generator().manual_seed(3), dtype=torch.int32)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV), shared_docs=False)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D.reshape(21, 50, 64)), lengths.numpy(), shared_docs=False)
    assert out.shape == (3, 7)
    assert_scores(out, ref)


@pytest.mark.parametrize("Nq, Lq, B, Ld, d, dtype", [
    (4, 32, 9, 77, 128, torch.float16),     # odd B: each query's last pair holds one doc
    (5, 32, 10, 77, 128, torch.bfloat16),
    (3, 128, 7, 300, 128, torch.float16),   # full query tile: pairs at any doc length
    (6, 24, 5, 60, 96, torch.float16),      # masked width
])
def test_per_query_docs_pairs(oracle_mod, Nq, Lq, B, Ld, d, dtype):
    # Per-query docs score two of one query's docs per workgroup.
    Q = sim((Nq, Lq, d), 230 + Lq, dtype)
    D = sim((Nq, B, Ld, d), 231 + B, dtype)
    lengths = torch.randint(0, Ld + 3, (Nq * B,), generator=torch.Generator().manual_seed(Nq * B), dtype=torch.int32)
    lengths[1] = 0
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV), shared_docs=False)
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D.reshape(Nq * B, Ld, d)), lengths.numpy(), shared_docs=False)
    assert out.shape == (Nq, B)
    assert_scores(out, ref)


def test_batched_large_query(oracle_mod):
    Q = sim((3, 300, 128), 220)
    D = sim((6, 80, 128), 221)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV))
    assert_scores(out, oracle_mod.maxsim(to_np32(Q), to_np32(D)))


def test_config3_sampled(oracle_mod):
    """BASELINE config 3 at full size (Q[100,32,128], D[5000,300,128]); 4 docs x 100 queries checked
    exhaustively, plus a random sample of 300 (query, doc) pairs."""
    Q = sim((100, 32, 128), 3)
    D = sim((5000, 300, 128), 4)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV)).cpu()
    Qn, Dn = to_np32(Q), to_np32(D)
    cols = [0, 1, 2499, 4999]
    ref = oracle_mod.maxsim(Qn, Dn[cols])
    assert_scores(out[:, cols], ref)
    rng = np.random.default_rng(0)
    qs, bs = rng.integers(0, 100, 300), rng.integers(0, 5000, 300)
    for qi, b in zip(qs, bs):
        r = oracle_mod.maxsim(Qn[qi], Dn[b:b + 1])[0, 0]
        assert abs(float(out[qi, b]) - r) <= ATOL


def test_config2_sampled(oracle_mod):
    """BASELINE config 2 shape (Q[1024,128], D[B,1024,128]) on 24 docs."""
    out, ref = run_single(oracle_mod, 24, 1024, 1024, 128, 2)
    assert_scores(out, ref)


# ------------------------------------------------------------------- int8 ----

def run_int8(oracle_mod, B, Lq, Ld, d, seed, lengths=None):
    Q = sim((Lq, d), seed)
    D = sim((B, Ld, d), seed + 1, torch.float32)
    codes, s, m = fm.quantize_int8(D)  # CPU torch, bit-exact with the oracle's quantiser
    lt = None if lengths is None else torch.as_tensor(lengths, dtype=torch.int32)
    out = fm.flash_maxsim_int8(Q.to(DEV), codes.to(DEV), s.to(DEV), m.to(DEV),
                               None if lt is None else lt.to(DEV))
    ref = oracle_mod.maxsim_int8(to_np32(Q), codes.numpy(), to_np32(s), to_np32(m), lengths)
    return out, ref, (Q, D, codes, s, m)


def test_int8(oracle_mod):
    """Reference test_int8 (tests/test_flash_maxsim.py:41-46), with values checked."""
    out, ref, _ = run_int8(oracle_mod, 50, 32, 300, 128, 300)
    assert out.shape == (50,)
    assert_scores(out, ref)


def test_int8_varlen_config4_like(oracle_mod):
    """BASELINE config 4 recipe (lengths U[32,1024], Ld=1024) on 300 docs."""
    lengths = torch.randint(32, 1025, (300,), generator=torch.Generator().manual_seed(4)).tolist()
    lengths[:4] = [0, 1, 1024, 2000]
    out, ref, _ = run_int8(oracle_mod, 300, 32, 1024, 128, 310, lengths=lengths)
    assert_scores(out, ref)


@pytest.mark.parametrize("d", [64, 96, 100, 256, 512, 1024, 4096])
def test_int8_dims(oracle_mod, d):
    out, ref, _ = run_int8(oracle_mod, 20, 32, 128, d, 320 + d, lengths=[128, 3, 77, 0] * 5)
    assert_scores(out, ref)


@pytest.mark.parametrize("d", [256, 512, 1024])
def test_large_dim_int8_ranking(oracle_mod, d):
    """Reference test_large_dim_int8 (tests/test_flash_maxsim.py:79-89): top-3 of int8 equals fp16."""
    out, ref, (Q, D, *_rest) = run_int8(oracle_mod, 20, 32, 128, d, 330 + d)
    fp = fm.flash_maxsim(Q.to(DEV), D.half().to(DEV))
    assert torch.equal(fp.argsort(descending=True)[:3], out.argsort(descending=True)[:3])
    assert_scores(out, ref)


def test_int8_long_query(oracle_mod):
    out, ref, _ = run_int8(oracle_mod, 6, 300, 64, 128, 340)
    assert_scores(out, ref)


@pytest.mark.parametrize("lengths", [[0, 5, 512, 0, 0, 17, 16, 33, 1],
                                     [512, 0, 16, 15, 0, 0, 300, 511, 64, 65, 2]])
def test_int8_doc_pairs(oracle_mod, lengths):
    """Single-query uint8 scoring runs two docs per workgroup: odd doc counts
    (the last workgroup has one doc), empty docs on either side of a pair, and
    pairs whose tiles split unevenly over the workgroup's four waves."""
    out, ref, _ = run_int8(oracle_mod, len(lengths), 32, 512, 128, 360 + len(lengths), lengths=lengths)
    assert_scores(out, ref)


@pytest.mark.parametrize("Lq, d", [(65, 128), (100, 128), (128, 128), (100, 120), (129, 128)])
def test_int8_full_query_tile(oracle_mod, Lq, d):
    """uint8 queries of 65-128 tokens at d <= 128 run one 128-row pass, two
    docs per workgroup with a two-tile ring (d = 120: the generic load
    instance); 129 tokens run two such passes."""
    lengths = [512, 0, 16, 15, 0, 0, 300, 511, 64, 65, 2]
    out, ref, _ = run_int8(oracle_mod, len(lengths), Lq, 512, d, 370 + Lq + d, lengths=lengths)
    assert_scores(out, ref)


def test_int8_unaligned_scale_rows(oracle_mod):
    """Ld % 4 != 0 makes the kernel read scales one token at a time."""
    out, ref, _ = run_int8(oracle_mod, 7, 32, 301, 128, 350, lengths=[301, 300, 299, 1, 0, 150, 17])
    assert_scores(out, ref)


# ----------------------------------------------------------------- sparse ----

@pytest.mark.parametrize("keep", [0.25, 0.5, 0.75, 1.0])
def test_sparse_maxsim(oracle_mod, keep):
    """Reference test_sparse_maxsim (tests/test_flash_maxsim.py:67-76)."""
    Q = sim((32, 128), 400)
    D = sim((50, 300, 128), 401)
    K = max(1, int(32 * keep))
    imp = torch.randn(50, 32, generator=torch.Generator().manual_seed(402))
    idx = imp.topk(K, dim=1).indices.to(torch.int32)
    out = fm.flash_maxsim_sparse(Q.to(DEV), D.to(DEV), idx.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), qidx=idx.numpy())[0]
    assert_scores(out, ref)
    naive = fm.maxsim_sparse_naive(Q.to(DEV), D.to(DEV), idx.to(DEV))
    assert_scores(naive, ref, atol=1e-3)


def test_sparse_varlen_large_d(oracle_mod):
    Q = sim((40, 512), 410)
    D = sim((9, 70, 512), 411)
    idx = torch.randint(0, 40, (9, 20), generator=torch.Generator().manual_seed(412), dtype=torch.int32)
    lengths = [70, 0, 1, 33, 69, 70, 16, 17, 50]
    out = fm.flash_maxsim_sparse(Q.to(DEV), D.to(DEV), idx.to(DEV), torch.tensor(lengths).to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths, qidx=idx.numpy())[0]
    assert_scores(out, ref)


# --------------------------------------------------------------- training ----

def grad_tol(dtype):
    """(rtol, atol) for gradients stored in dtype: fp16 keeps 11 significant
    bits (half an ulp is 2^-11 = 4.9e-4 relative), bf16 only 8 (2^-8 = 3.9e-3,
    above the fp16 rtol of 2e-3)."""
    return (1e-2, 2e-2) if dtype == torch.bfloat16 else (2e-3, ATOL)


def run_train(oracle_mod, B, Lq, Ld, d, seed, dtype=torch.float16):
    Q = sim((Lq, d), seed, dtype)
    D = sim((B, Ld, d), seed + 1, dtype)
    g = torch.linspace(-1.0, 2.0, B, dtype=torch.float32)
    Qg = Q.to(DEV).requires_grad_(True)
    Dg = D.to(DEV).requires_grad_(True)
    s = fm.flash_maxsim_train(Qg, Dg)
    (s * g.to(DEV)).sum().backward()
    Qn, Dn = to_np32(Q), to_np32(D)
    ref, am_ref, best = oracle_mod.maxsim(Qn, Dn, want_argmax=True)
    return s, Qg.grad, Dg.grad, ref, am_ref, best, Qn, Dn, g


@pytest.mark.parametrize("shape", [(10, 16, 64, 128), (7, 32, 300, 128), (5, 128, 100, 1024),
                                   (6, 40, 50, 96), (4, 1024, 64, 128)])
def test_train_scores_argmax_grads(oracle_mod, shape):
    B, Lq, Ld, d = shape
    s, dQ, dD, ref, am_ref, best, Qn, Dn, g = run_train(oracle_mod, B, Lq, Ld, d, 500 + d + Lq)
    assert_scores(s, ref[0])
    # argmax the kernel saved: rerun the forward with the argmax exposed
    from flash_maxsim_amd.flash_maxsim import _launch_fwd, _prep

    Q2, D2 = _prep(torch.from_numpy(Qn).half().to(DEV), torch.float16), _prep(
        torch.from_numpy(Dn).half().to(DEV), torch.float16)
    _, am = _launch_fwd(Q2[None], D2, None, 1, B, Lq, Ld, d, True, True)
    assert_argmax(am, am_ref, best, Qn, Dn, d)
    dQ_ref, dD_ref = oracle_mod.bwd(Qn, Dn, am.cpu().numpy(), g.numpy())
    assert dQ.dtype == torch.float16 and dD.dtype == torch.float16
    np.testing.assert_allclose(dQ.double().cpu().numpy(), dQ_ref, rtol=2e-3, atol=ATOL)
    np.testing.assert_allclose(dD.double().cpu().numpy(), dD_ref, rtol=2e-3, atol=ATOL)


def test_train_reference_case():
    """Reference test_train (tests/test_flash_maxsim.py:49-55): Q.grad exists, D without grad."""
    Q = sim((16, 128), 600).to(DEV).requires_grad_(True)
    D = sim((10, 64, 128), 601).to(DEV)
    s = fm.flash_maxsim_train(Q, D)
    s.sum().backward()
    assert Q.grad is not None and Q.grad.shape == Q.shape and torch.isfinite(Q.grad).all()


def test_train_bf16_and_fp32_leaves(oracle_mod):
    s, dQ, dD, ref, am_ref, best, Qn, Dn, g = run_train(oracle_mod, 6, 32, 80, 128, 610, torch.bfloat16)
    assert_scores(s, ref[0])
    assert dQ.dtype == torch.bfloat16
    Qf = sim((32, 128), 620, torch.float32).to(DEV).requires_grad_(True)
    Df = sim((5, 40, 128), 621, torch.float32).to(DEV).requires_grad_(True)
    fm.flash_maxsim_train(Qf, Df).sum().backward()
    assert Qf.grad.dtype == torch.float32 and Df.grad.dtype == torch.float32


def test_train_is_deterministic():
    Q = sim((64, 128), 630).to(DEV)
    D = sim((40, 200, 128), 631).to(DEV)
    outs = []
    for _ in range(2):
        Qg, Dg = Q.clone().requires_grad_(True), D.clone().requires_grad_(True)
        s = fm.flash_maxsim_train(Qg, Dg)
        s.sum().backward()
        outs.append((s.detach().clone(), Qg.grad.clone(), Dg.grad.clone()))
    for a, b in zip(outs[0], outs[1]):
        assert torch.equal(a, b)


def test_maxsim_naive_on_gpu(oracle_mod):
    Q = sim((32, 128), 700)
    D = sim((10, 60, 128), 701)
    lengths = torch.tensor([60, 0, 1, 30, 59, 60, 10, 20, 40, 50], dtype=torch.int32)
    out = fm.maxsim_naive(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    assert_scores(out, oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())[0], atol=1e-4)


# ------------------------------------------------- tiled (many query rows) ----

@pytest.mark.parametrize("Nq, Lq, B, Ld, d", [
    (1, 256, 30, 100, 128),     # smallest row count routed to the tiled kernel
    (1, 2048, 5, 70, 128),      # one query over two row blocks: partial sums
    (3, 700, 9, 90, 128),       # queries straddling row-block boundaries
    (40, 32, 37, 75, 128),      # batched, B not a multiple of the doc groups
    (16, 32, 300, 64, 256),     # d = 256 (8 k-steps)
    (8, 64, 20, 50, 200),       # d not a multiple of 32
    (2, 300, 3, 1030, 96),      # long docs, few docs (fewer doc groups than CUs)
])
def test_tiled_shapes(oracle_mod, Nq, Lq, B, Ld, d):
    Q = sim((Nq, Lq, d), 800 + Lq + d)
    D = sim((B, Ld, d), 801 + B)
    lengths = torch.randint(0, Ld + 20, (B,), generator=torch.Generator().manual_seed(B), dtype=torch.int32)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())
    assert_scores(out, ref)


@pytest.mark.parametrize("Nq, Lq, B, Ld, d", [
    (100, 32, 300, 40, 128),    # 3200 rows: five 640-row blocks (NB = 5)
    (24, 32, 300, 50, 128),     # 768 rows: one 768-row block (NB = 6)
    (12, 32, 300, 64, 256),     # d = 256, 384 rows (NB = 3)
    (1, 300, 300, 70, 128),     # single query, 300 rows: one 384-row block (NB = 3)
    (8, 32, 300, 50, 128),      # 256 rows (NB = 2)
    (3, 64, 300, 45, 96),       # 192 rows, masked width (NB = 2)
    (2, 32, 300, 60, 128),      # two queries: one 128-row block (NB = 1)
    (1, 96, 300, 40, 256),      # d = 256, single query past one streaming pass (NB = 1)
])
def test_tiled_row_block_sizes(oracle_mod, Nq, Lq, B, Ld, d):
    # Shapes whose plan (256 CUs) picks each row-block size; the oracle checks
    # every fourth query (first and last included) to stay within seconds.
    Q = sim((Nq, Lq, d), 900 + Nq)
    D = sim((B, Ld, d), 901 + d)
    lengths = torch.randint(0, Ld + 5, (B,), generator=torch.Generator().manual_seed(Nq), dtype=torch.int32)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    pick = sorted(set(range(0, Nq, 4)) | {Nq - 1})
    ref = oracle_mod.maxsim(to_np32(Q[pick]), to_np32(D), lengths.numpy())
    assert_scores(out[pick], ref)


def test_tiled_bf16_and_argmax(oracle_mod):
    s, dQ, dD, ref, am_ref, best, Qn, Dn, g = run_train(oracle_mod, 6, 512, 100, 128, 820, torch.bfloat16)
    assert_scores(s, ref[0])
    from flash_maxsim_amd.flash_maxsim import _launch_fwd, _prep

    Q2 = _prep(torch.from_numpy(Qn).to(torch.bfloat16).to(DEV), torch.bfloat16)
    D2 = _prep(torch.from_numpy(Dn).to(torch.bfloat16).to(DEV), torch.bfloat16)
    _, am = _launch_fwd(Q2[None], D2, None, 1, 6, 512, 100, 128, True, True)
    assert_argmax(am, am_ref, best, Qn, Dn, 128)
    dQ_ref, dD_ref = oracle_mod.bwd(Qn, Dn, am.cpu().numpy(), g.numpy())
    rtol, atol = grad_tol(torch.bfloat16)
    np.testing.assert_allclose(dQ.double().cpu().numpy(), dQ_ref, rtol=rtol, atol=atol)
    np.testing.assert_allclose(dD.double().cpu().numpy(), dD_ref, rtol=rtol, atol=atol)


@pytest.mark.parametrize("Nq, Lq, B, Ld, d, dtype", [
    (8, 32, 1500, 40, 128, torch.float16),    # 256 rows: one 256-row block (NB = 4)
    (1, 512, 1600, 40, 128, torch.bfloat16),  # one query over two 256-row blocks: partial sums
    (6, 64, 1600, 30, 128, torch.bfloat16),   # 384 rows: two 192-row blocks (NB = 3)
    (3, 100, 1600, 40, 96, torch.float16),    # 192-row blocks, masked width, straddling queries
    (2, 150, 1600, 30, 100, torch.float16),   # masked width with a partial chunk, straddling
])
def test_tiled_four_wave_blocks(oracle_mod, Nq, Lq, B, Ld, d, dtype):
    # Shapes whose plan (256 CUs) picks four-wave workgroups, three per CU.
    Q = sim((Nq, Lq, d), 950 + Lq, dtype)
    D = sim((B, Ld, d), 951 + d, dtype)
    lengths = torch.randint(0, Ld + 5, (B,), generator=torch.Generator().manual_seed(Lq), dtype=torch.int32)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())
    assert_scores(out, ref)


@pytest.mark.parametrize("Nq, Lq, d, dtype", [
    (300, 1, 128, torch.float16),    # one row per query: no lane exchange
    (150, 2, 128, torch.bfloat16),
    (70, 4, 100, torch.float16),     # masked width (VGPR staging)
    (40, 16, 128, torch.float16),
    (9, 64, 256, torch.bfloat16),    # d = 256 (8 k-steps), a full 64-row window per query
    (20, 64, 128, torch.float16),
])
def test_tiled_window_sums(oracle_mod, Nq, Lq, d, dtype):
    # Query lengths dividing 64: each 64-row window of a row block holds whole
    # queries, summed by one lane-group sum per window.
    B, Ld = 70, 60
    Q = sim((Nq, Lq, d), 970 + Lq, dtype)
    D = sim((B, Ld, d), 971 + d, dtype)
    lengths = torch.randint(0, Ld + 5, (B,), generator=torch.Generator().manual_seed(Nq), dtype=torch.int32)
    out = fm.flash_maxsim_batched(Q.to(DEV), D.to(DEV), lengths.to(DEV))
    ref = oracle_mod.maxsim(to_np32(Q), to_np32(D), lengths.numpy())
    assert_scores(out, ref)


@pytest.mark.parametrize("Lq, Ld, d, dtype", [
    (400, 40, 128, torch.bfloat16),  # two 256-row blocks
    (300, 30, 96, torch.float16),    # two 192-row blocks, masked width
])
def test_tiled_four_wave_argmax(oracle_mod, Lq, Ld, d, dtype):
    B = 1600
    s, dQ, dD, ref, am_ref, best, Qn, Dn, g = run_train(oracle_mod, B, Lq, Ld, d, 960 + d, dtype)
    assert_scores(s, ref[0])
    from flash_maxsim_amd.flash_maxsim import _launch_fwd, _prep

    Q2 = _prep(torch.from_numpy(Qn).to(dtype).to(DEV), dtype)
    D2 = _prep(torch.from_numpy(Dn).to(dtype).to(DEV), dtype)
    _, am = _launch_fwd(Q2[None], D2, None, 1, B, Lq, Ld, d, True, True)
    assert_argmax(am, am_ref, best, Qn, Dn, d)
    dQ_ref, dD_ref = oracle_mod.bwd(Qn, Dn, am.cpu().numpy(), g.numpy())
    rtol, atol = grad_tol(dtype)
    np.testing.assert_allclose(dQ.double().cpu().numpy(), dQ_ref, rtol=rtol, atol=atol)
    np.testing.assert_allclose(dD.double().cpu().numpy(), dD_ref, rtol=rtol, atol=atol)
